"""A seeded sweep of the expert-LoRA backward passes over shapes the fixed
tests do not pick: u = s big[b] @ B[e] and dB[e] = sum bf16(rs big[b])^T L in
one pass (af3_lora_u_wgrad) against the oracle per expert, and dB bit for bit
against the two-pass weight-gradient kernel.  Wide sides W of 16 to 3840
columns (last column groups and slices of any multiple of 8), r = 16 / 32,
gathered or sorted rows, with and without the row scale, 3-9 experts with
idle, single-row and multi-chunk experts (the routing draws of the GEMM
sweep, other seeds)."""
import random

import pytest
import torch

from agent_factory_3_amd import quantization as Q
from oracle import moe
from tests._tol import check_close
from tests.test_gpu_gemm_sweep import _case, _routing

pytestmark = pytest.mark.gpu
N_CASES = 16


@pytest.mark.parametrize("case", range(N_CASES))
def test_lora_u_and_dB_sweep(dev, case):
    seed = 5000 + case
    c = _case(seed)
    rnd = random.Random(seed)
    W = rnd.choice([8 * rnd.randint(2, 400), 64 * rnd.randint(1, 60)])
    r = rnd.choice([16, 32])
    gather = rnd.random() < 0.5
    rowscale = rnd.random() < 0.5
    E, K, T = c["E"], c["topk"], c["T"]
    print(f"lora sweep seed {seed}: E={E} topk={K} T={T} counts={c['counts']} W={W} r={r} gather={gather} "
          f"rowscale={rowscale}", flush=True)
    g = torch.Generator().manual_seed(seed)
    ref, rd, gi = _routing(dev, g, c["counts"], T, K)
    R_ = T * K
    big = torch.randn(T if gather else R_, W, generator=g).to(torch.bfloat16)
    L = torch.randn(R_, r, generator=g).to(torch.bfloat16)
    Bw = (torch.randn(E, W, r, generator=g) * 0.1).to(torch.bfloat16)
    rs = rd.gate_scal.to(torch.bfloat16) if rowscale else None
    gx = gi.src_indx if gather else None
    div = K if gather else 1
    ed = rd.expt_data
    u, dB = Q._lora_u_and_dB(big.to(dev), gx, div, rs, L.to(dev), Bw.to(dev), 0.5, ed, E, W)
    dB2 = Q._lora_wgrad(big.to(dev), gx, div, rs, L.to(dev), None, 1, ed, E, W, r)
    u, dB, dB2 = u.cpu(), dB.cpu(), dB2.cpu()
    assert torch.equal(dB.view(torch.int16), dB2.view(torch.int16))
    offs, ti = ref["offs"], ref["topk_indx"].long()
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi == lo:
            assert dB[e].abs().max() == 0
            continue
        ib = ti[lo:hi] // K if gather else torch.arange(lo, hi)
        uref, umag = moe.expert_lora_rows(big, Bw[e], ib, 0.5, trans=True)
        check_close(u[lo:hi], uref, mag=umag, n=W, what=f"u expert {e}")
        dref, dmag = moe.expert_wgrad(big[ib], L[lo:hi], rs.cpu()[lo:hi] if rowscale else None)
        check_close(dB[e], dref, mag=dmag, n=hi - lo, what=f"dB expert {e}")
