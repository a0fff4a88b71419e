"""A seeded sweep of the default grouped GEMMs over shapes the fixed-shape
tests do not pick, against the oracle: forward and input gradient, the stored
and the tiled weight / scale copies, gathered and sorted rows, the expert-LoRA
segment at r = 16 / 32, routing weights on the input gradient, 3-9 experts
with idle, single-row and near-T experts, N from 64 to 1536 (tail n-tiles of
64-192 columns) and reductions from 64 to 1536 (1-24 k-steps, multiples of
three among them: the forward's three-buffer k-loop).  Each case is drawn
from its own seed, so a failure names a reproducible shape."""
import random

import pytest
import torch

from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import moe, mxfp4
from oracle import routing as O

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 1e-2
N_CASES = 24


def _case(seed):
    """Shape, routing counts and options of one case (bounded draws)."""
    rnd = random.Random(seed)
    E = rnd.randint(3, 9)
    topk = rnd.choice([2, 4])
    if topk >= E:
        topk = 2
    T = rnd.randint(150, 700)
    for _ in range(200):  # rows per expert: sum T * topk, each <= T (distinct experts per token)
        w = [rnd.random() ** 2 for _ in range(E)]
        for z in rnd.sample(range(E), rnd.randint(0, 1)):
            w[z] = 0.0
        s = sum(w)
        counts = [int(T * topk * x / s) for x in w]
        counts[counts.index(max(counts))] += T * topk - sum(counts)
        if max(counts) <= T:
            break
    else:
        counts = [T * topk // E] * E
        counts[0] += T * topk - sum(counts)
    return dict(E=E, topk=topk, T=T, counts=counts, trans=rnd.random() < 0.5, N=64 * rnd.randint(1, 24),
                K=rnd.choice([64 * rnd.randint(1, 24), 192 * rnd.randint(1, 8)]), gather=rnd.random() < 0.6,
                lora=rnd.random() < 0.5, r=rnd.choice([16, 32]), tiled=rnd.random() < 0.7)


def _routing(dev, g, counts, T, topk):
    order = sorted(range(len(counts)), key=lambda e: -counts[e])
    multiset = [e for e in order for _ in range(counts[e])]
    ids = torch.empty(T, topk, dtype=torch.int32)
    for j, e in enumerate(multiset):
        ids[j % T, j // T] = e
    ids = ids[torch.randperm(T, generator=g)].sort(dim=1).values
    logits = torch.randn(T, len(counts), generator=g).to(torch.bfloat16)
    ref = O.routing_replay(logits, ids, topk)
    rd, gi, _ = R.routing_replay(logits.to(dev), ids.to(dev), topk)
    assert ref["hist"].tolist() == counts
    return ref, rd, gi


@pytest.mark.parametrize("case", range(N_CASES))
def test_default_gemm_shape_sweep(dev, case):
    seed = 1000 + case
    c = _case(seed)
    E, topk, T, N, K, trans, gather, lora, r = (c[k] for k in ("E", "topk", "T", "N", "K", "trans", "gather", "lora",
                                                              "r"))
    print(f"sweep seed {seed}: {c}", flush=True)
    g = torch.Generator().manual_seed(seed)
    ref, rd, gi = _routing(dev, g, c["counts"], T, topk)
    Rr = T * topk
    rows, cols = (K, N) if trans else (N, K)  # W [E, N, K]; trans: [E, K, N] packed along N
    blocks = torch.randint(0, 256, (E, rows, cols // 32, 16), generator=g).to(torch.uint8)
    scales = torch.randint(116, 127, (E, rows, cols // 32), generator=g).to(torch.uint8)
    x = torch.randn(T if gather else Rr, K, generator=g).to(torch.bfloat16)
    bias = None if trans else (torch.randn(E, N, generator=g) * 0.1).to(torch.bfloat16)
    L = (torch.randn(Rr, r, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    Bx = None
    if lora:
        Bx = ((torch.randn(E, r, N, generator=g) if trans else torch.randn(E, N, r, generator=g)) * 0.3).to(
            torch.bfloat16)
    gam = rd.gate_scal if trans and gather else None
    wb, ws = blocks.to(dev), scales.to(dev)
    kw = {}
    if c["tiled"]:
        kw = {"s_tiled": Q.mxfp4_tile_dx_scales(ws)} if trans else {"w_tiled": Q.mxfp4_tile_fwd(wb)}
    y = Q.moe_rows(x.to(dev), wb, ws, None if bias is None else bias.float().to(dev), rd, gi if gather else None,
                   gam, trans, None if L is None else L.to(dev), None if Bx is None else Bx.to(dev), **kw)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, topk, bias=bias,
                  gammas=None if gam is None else gam.cpu(), trans=trans, lora_l=L, lora_b=Bx)
    a = y.float().cpu().double()
    assert y.shape == (Rr, N)
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())
