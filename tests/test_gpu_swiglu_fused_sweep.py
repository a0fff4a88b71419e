"""A seeded sweep of the grouped GEMMs' fused SwiGLU epilogues over shapes the
fixed tests do not pick: the gate_up forward's (epi 2: the pre-activation
rows and their clamped SwiGLU from one launch) and the down input gradient's
(epi 1: dGU from the GEMM's bf16 rows and the saved pre-activation), each
bit for bit against the same GEMM without the epilogue followed by the
separate SwiGLU kernel, with the stored and the tiled weight / scale copies,
the expert-LoRA segment, gathered rows and routing weights (the routing
draws of the GEMM sweep, other seeds).  Pre-activations are scaled so that
both clamps (gate above the limit, up outside +-limit) occur."""
import random

import pytest
import torch

from agent_factory_3_amd import kernels
from agent_factory_3_amd import quantization as Q
from tests.test_gpu_gemm_sweep import _case, _routing

pytestmark = pytest.mark.gpu
N_CASES = 12
ALPHA, LIMIT = 1.702, 7.0


@pytest.mark.parametrize("case", range(N_CASES))
def test_fused_swiglu_sweep(dev, case):
    seed = 7000 + case
    c = _case(seed)
    rnd = random.Random(seed)
    I_ = 64 * rnd.randint(1, 12)          # intermediate width: gate_up N = 2 I, down dX output I
    H = 64 * rnd.randint(1, 16)           # hidden: the forward's reduction and the dX reduction
    r = rnd.choice([16, 32])
    lora = rnd.random() < 0.5
    tiled = rnd.random() < 0.6
    E, K, T = c["E"], c["topk"], c["T"]
    print(f"swiglu sweep seed {seed}: E={E} topk={K} T={T} counts={c['counts']} I={I_} H={H} lora={lora and r} "
          f"tiled={tiled}", flush=True)
    g = torch.Generator().manual_seed(seed)
    ref, rd, gi = _routing(dev, g, c["counts"], T, K)
    Rr = T * K
    # gate_up forward: W [E, 2I, H]
    wb = torch.randint(0, 256, (E, 2 * I_, H // 32, 16), generator=g).to(torch.uint8).to(dev)
    ws = torch.randint(120, 127, (E, 2 * I_, H // 32), generator=g).to(torch.uint8).to(dev)
    x = (torch.randn(T, H, generator=g) * 2).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, 2 * I_, generator=g)).float().to(dev)
    L = (torch.randn(Rr, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Bx = (torch.randn(E, 2 * I_, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    kw = {"w_tiled": Q.mxfp4_tile_fwd(wb)} if tiled else {}
    res = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx, swiglu=("fwd", ALPHA, LIMIT), **kw)
    assert res is not None
    gu, act = res
    gu_plain = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx, **kw)
    assert torch.equal(gu.view(torch.int16), gu_plain.view(torch.int16))
    assert torch.equal(act.view(torch.int16), kernels.swiglu_forward(gu_plain, ALPHA, LIMIT).view(torch.int16))
    assert (gu.float()[:, 0::2] > LIMIT).any() and (gu.float()[:, 1::2].abs() > LIMIT).any()
    # down input gradient: W [E, H, I] read transposed (output I), reduction H
    db = torch.randint(0, 256, (E, H, I_ // 32, 16), generator=g).to(torch.uint8).to(dev)
    ds = torch.randint(118, 125, (E, H, I_ // 32), generator=g).to(torch.uint8).to(dev)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16).to(dev)
    u = (torch.randn(Rr, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Ax = (torch.randn(E, r, I_, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    kw = {"s_tiled": Q.mxfp4_tile_dx_scales(ds)} if tiled else {}
    dgu = Q.moe_rows(dy, db, ds, None, rd, gi, rd.gate_scal, True, u, Ax, swiglu=("bwd", gu, ALPHA, LIMIT), **kw)
    d_act = Q.moe_rows(dy, db, ds, None, rd, gi, rd.gate_scal, True, u, Ax, **kw)
    assert dgu is not None and dgu.shape == (Rr, 2 * I_)
    assert torch.equal(dgu.view(torch.int16), kernels.swiglu_backward_raw(d_act, gu, ALPHA, LIMIT).view(torch.int16))
