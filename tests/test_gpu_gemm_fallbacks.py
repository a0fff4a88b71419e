"""The general fallback grouped GEMMs at gpt-oss sizes, against the oracle on
every row of every expert: tile_cfg 4 (gemm2: 256x256 tiles, weights
dequantised into LDS) for the forward (N = 5760, K = 2880, gathered rows,
bias, expert LoRA) and the input gradient (N = 2880, K = 5760, routing
weights), and the single-buffered row tiles (tile_cfg 9) that any reduction
depth which is not a multiple of 64 selects (K = 2912) in both directions.
Experts of 1000, 700, 357 and 0 rows plus a 128-row and a 1-row one, so full,
partial and idle tiles all occur."""
import pytest
import torch

from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import moe, mxfp4
from oracle import routing as O
from tests._tol import check_close

pytestmark = pytest.mark.gpu
COUNTS = [1000, 700, 357, 0, 128, 1]   # max <= T: distinct experts per token
TOPK = 2
T = sum(COUNTS) // TOPK  # 1093


def _routing(dev, seed):
    g = torch.Generator().manual_seed(seed)
    E = len(COUNTS)
    order = sorted(range(E), key=lambda e: -COUNTS[e])
    multiset = [e for e in order for _ in range(COUNTS[e])]
    ids = torch.empty(T, TOPK, dtype=torch.int32)
    for j, e in enumerate(multiset):
        ids[j % T, j // T] = e
    ids = ids[torch.randperm(T, generator=g)].sort(dim=1).values
    assert (ids[:, 0] != ids[:, 1]).all()
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    ref = O.routing_replay(logits, ids, TOPK)
    rd, gi, si = R.routing_replay(logits.to(dev), ids.to(dev), TOPK)
    assert ref["hist"].tolist() == COUNTS
    return g, ref, rd, gi


def _weights(g, E, rows, cols):
    blocks = torch.randint(0, 256, (E, rows, cols // 32, 16), generator=g).to(torch.uint8)
    scales = torch.randint(118, 125, (E, rows, cols // 32), generator=g).to(torch.uint8)
    return blocks, scales


def _check(y, x, W, ref, gather, trans, bias=None, gammas=None, L=None, B=None, what=""):
    offs = ref["offs"]
    n_red = x.shape[1] + (L.shape[1] if L is not None else 0)
    for e in range(len(COUNTS)):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi == lo:
            continue
        idx = (ref["topk_indx"][lo:hi].long() // TOPK) if gather else torch.arange(lo, hi)
        r, mag = moe.expert_rows(x, W[e], idx, trans=trans, lora_l=None if L is None else L[lo:hi],
                                 lora_b=None if B is None else B[e], bias=None if bias is None else bias[e],
                                 gammas=None if gammas is None else gammas[lo:hi])
        check_close(y[lo:hi], r, mag=mag, n=n_red, what=f"{what} expert {e} ({hi - lo} rows)")
    assert torch.isfinite(y.float()).all()


def _run(rows_args, cfg):
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=256, tile_cfg=cfg)
    try:
        return Q.moe_rows(*rows_args)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)


@pytest.mark.parametrize("cfg,K", [(4, 2880), (0, 2912)])
def test_fallback_forward(dev, cfg, K):
    N, E = 5760, len(COUNTS)
    print(f"fallback forward tile_cfg {cfg} N={N} K={K}", flush=True)
    g, ref, rd, gi = _routing(dev, 31)
    blocks, scales = _weights(g, E, N, K)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16)
    bias = (torch.randn(E, N, generator=g) * 0.1).to(torch.bfloat16)
    L = (torch.randn(T * TOPK, 32, generator=g) * 0.3).to(torch.bfloat16) if cfg == 4 else None
    Bx = (torch.randn(E, N, 32, generator=g) * 0.3).to(torch.bfloat16) if cfg == 4 else None
    y = _run((x.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi, None, False,
              L.to(dev) if L is not None else None, Bx.to(dev) if Bx is not None else None), cfg)
    torch.cuda.synchronize()
    W = mxfp4.dequant_f32(blocks, scales)
    _check(y.cpu(), x, W, ref, True, False, bias=bias, L=L, B=Bx, what=f"fwd cfg {cfg} K={K}")


@pytest.mark.parametrize("cfg,K", [(4, 5760), (0, 2912)])
def test_fallback_input_gradient(dev, cfg, K):
    N, E = 2880, len(COUNTS)
    print(f"fallback input gradient tile_cfg {cfg} N={N} K={K}", flush=True)
    g, ref, rd, gi = _routing(dev, 32)
    blocks, scales = _weights(g, E, K, N)          # W [E, K, N] packed along N
    x = torch.randn(T * TOPK, K, generator=g).to(torch.bfloat16)
    gam = rd.gate_scal
    y = _run((x.to(dev), blocks.to(dev), scales.to(dev), None, rd, None, gam, True, None, None), cfg)
    torch.cuda.synchronize()
    W = mxfp4.dequant_f32(blocks, scales)
    _check(y.cpu(), x, W, ref, False, True, gammas=gam.cpu(), what=f"dX cfg {cfg} K={K}")
