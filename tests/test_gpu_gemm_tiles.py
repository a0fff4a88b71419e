"""Grouped-GEMM kernel variants (tile_cfg) vs the oracle at shapes with full and
partial 256x256 tiles, several k-steps and scale bytes outside [2, 252].

The forward kernels (A6 / A8) and the input-gradient kernels (A9 / A11) each
run on: N = 576 (two full 256-column tiles and a 64-column one), reduction 640
(ten 64-deep k-steps), experts with two full 256-row tiles plus a tail, a
small expert and an idle one.  The "odd" variants put e8m0 bytes 254 / 255 in
some blocks with nibble codes for which the reference rule
(kernels.py:137-158) gives signed zeros while a plain scaled conversion would
give inf / NaN, so a kernel that skipped the exact rule fails loudly.
"""
import pytest
import torch

from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import moe, mxfp4
from oracle import routing as O

pytestmark = pytest.mark.gpu
RTOL, ATOL = 2e-2, 1e-2
KRED, NOUT, T, E, TOPK = 640, 576, 700, 7, 4


# rows per expert: two full 256-row tiles + a tail of 188 / 178 / 138 rows
# (full-width tail tiles), 256 + 44 and 256 + 104 rows and 100 rows (tiles of
# <= 128 rows, which the default kernels of both directions run two n-tiles at
# a time, with N = 576 leaving a lone third n-tile), and an idle expert
COUNTS = [700, 300, 690, 650, 100, 360, 0]


def _routing(dev, seed):
    """Replay routing with exactly COUNTS rows per expert (distinct experts per token)."""
    g = torch.Generator().manual_seed(seed)
    E_ = len(COUNTS)
    assert sum(COUNTS) == T * TOPK and max(COUNTS) <= T
    order = sorted(range(E_), key=lambda e: -COUNTS[e])
    multiset = [e for e in order for _ in range(COUNTS[e])]
    ids = torch.empty(T, TOPK, dtype=torch.int32)
    for j, e in enumerate(multiset):
        ids[j % T, j // T] = e
    ids = ids[torch.randperm(T, generator=g)].sort(dim=1).values
    logits = torch.randn(T, E_, generator=g).to(torch.bfloat16)
    ref = O.routing_replay(logits, ids, TOPK)
    rd, gi, si = R.routing_replay(logits.to(dev), ids.to(dev), TOPK)
    assert ref["hist"].tolist() == COUNTS
    return g, ref, rd, gi


def _weights(g, rows, cols, odd):
    """MXFP4 blocks [E, rows, cols/32, 16] with codes uniform and scales 118..124;
    ``odd`` plants bytes 255 / 254 in a few blocks with zero-valued codes."""
    G = cols // 32
    blocks = torch.randint(0, 256, (E, rows, G, 16), generator=g).to(torch.uint8)
    scales = torch.randint(118, 125, (E, rows, G), generator=g).to(torch.uint8)
    if odd:
        def force(sel_blocks, codes):
            lo = torch.tensor(codes)[torch.randint(0, len(codes), sel_blocks.shape, generator=g)]
            hi = torch.tensor(codes)[torch.randint(0, len(codes), sel_blocks.shape, generator=g)]
            return (lo | (hi << 4)).to(torch.uint8)
        # S = 255: every code with a non-zero exponent field flushes (exponent > 254); no subnormal codes
        sl = (1, slice(130, 141), 5 % G)
        blocks[sl] = force(blocks[sl], [0, 2, 3, 4, 5, 6, 7, 8, 10, 11, 12, 13, 14, 15])
        scales[sl] = 255
        # S = 254: codes with exponent field 2 or 3 flush
        sl = (0, slice(300, 305), 1)
        blocks[sl] = force(blocks[sl], [0, 4, 5, 6, 7, 8, 12, 13, 14, 15])
        scales[sl] = 254
        # S = 0 / 1: underflow flushes (values far below the rest; checked for finiteness)
        scales[2, 10:20, 2] = 0
        scales[3, 40:44, 0] = 1
    return blocks, scales


CASES = [  # (gather, lora, odd)
    (True, False, False),
    (True, True, True),
    (False, False, True),
]


@pytest.mark.parametrize("cfg,nout", [(0, NOUT), (0, 640), (4, NOUT), (22, NOUT), (22, 640), (126, NOUT)])
@pytest.mark.parametrize("gather,lora,odd", CASES)
def test_forward_tiles(dev, cfg, nout, gather, lora, odd):
    """N = 576 / 640 end in a 64- / 128-column n-tile (waves past the tile's
    columns keep only the copy / barrier protocol).  The default forward
    (tile_cfg 0 = 26: 128 x 256 items on the 128-row map, two blocks per CU,
    packed weights loaded into registers) sees tails of 10, 44, 50, 60, 100
    and 104 rows; 126 is the same kernel with one m-tile per work group."""
    g, ref, rd, gi = _routing(dev, 11)
    blocks, scales = _weights(g, nout, KRED, odd)          # W [E, N, K]
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    bias = (torch.randn(E, nout, generator=g) * 0.1).to(torch.bfloat16)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    Bx = (torch.randn(E, nout, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=256, tile_cfg=cfg)
    try:
        y = Q.moe_rows(x.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi if gather else None,
                       None, False, L.to(dev) if lora else None, Bx.to(dev) if lora else None)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK, bias=bias, lora_l=L, lora_b=Bx)
    a = y.float().cpu().double()
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())


@pytest.mark.parametrize("cfg,nout", [(0, NOUT), (0, 640), (4, NOUT), (23, NOUT), (23, 640), (228, NOUT)])
@pytest.mark.parametrize("gather,lora,odd", CASES)
def test_dgrad_tiles(dev, cfg, nout, gather, lora, odd):
    """N = 576 / 640 end in a 64- / 128-column n-tile, which the 256-row kernel
    (tile_cfg 23) runs with the tile's rows split over the waves; the default
    (tile_cfg 0 = 28: 128 x 256 items on the 128-row map, two blocks per CU)
    sees tails of 10, 44, 50, 60, 100 and 104 rows; 228 is it with two m-tiles
    per work group."""
    g, ref, rd, gi = _routing(dev, 12)
    blocks, scales = _weights(g, KRED, nout, odd)          # W [E, K, N] packed along N
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    Ax = (torch.randn(E, 32, nout, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    gam = rd.gate_scal if gather else None
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=128 if cfg % 100 == 28 else 256, tile_cfg=cfg)
    try:
        y = Q.moe_rows(x.to(dev), blocks.to(dev), scales.to(dev), None, rd, gi if gather else None, gam, True,
                       L.to(dev) if lora else None, Ax.to(dev) if lora else None)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK,
                  gammas=gam.cpu() if gather else None, trans=True, lora_l=L, lora_b=Ax)
    assert y.shape == (Rr, nout)
    a = y.float().cpu().double()
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())


@pytest.mark.parametrize("dx_cfg", [(0, 256), (23, 256)])
@pytest.mark.parametrize("lora", [False, True])
def test_fused_swiglu_epilogues_bit_equal(dev, lora, dx_cfg):
    """af3_moe_gemm_swiglu: the forward epilogue's SwiGLU and the input-gradient
    epilogue's SwiGLU backward equal the separate kernels bit for bit, on full,
    partial and short (two n-tiles per work item) tiles."""
    from agent_factory_3_amd import kernels
    g, ref, rd, gi = _routing(dev, 13)
    alpha, limit = 1.702, 7.0
    Rr, r, I_ = T * TOPK, 32, 320          # 2I = 640: n-tiles 256, 256, 128; I = 320: 256 + 64
    # gate_up: W [E, 2I, H], H = KRED
    gu_blocks, gu_scales = _weights(g, 2 * I_, KRED, False)
    x = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, 2 * I_, generator=g) * 0.5).float().to(dev)
    L = (torch.randn(Rr, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Bx = (torch.randn(E, 2 * I_, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    wb, ws = gu_blocks.to(dev), gu_scales.to(dev)
    res = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx, swiglu=("fwd", alpha, limit))
    assert res is not None
    gu, act = res
    gu_plain = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx)
    assert torch.equal(gu, gu_plain)
    assert torch.equal(act, kernels.swiglu_forward(gu_plain, alpha, limit))
    # down dX: W [E, H, I] read transposed (output I), reduction H = KRED
    dn_blocks, dn_scales = _weights(g, KRED, I_, False)
    dy = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    u = (torch.randn(Rr, r, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Ax = (torch.randn(E, r, I_, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    gam = rd.gate_scal
    db, ds = dn_blocks.to(dev), dn_scales.to(dev)
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=dx_cfg[1], tile_cfg=dx_cfg[0])
    try:
        dgu = Q.moe_rows(dy, db, ds, None, rd, gi, gam, True, u, Ax, swiglu=("bwd", gu, alpha, limit))
        d_act = Q.moe_rows(dy, db, ds, None, rd, gi, gam, True, u, Ax)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    assert dgu is not None and dgu.shape == (Rr, 2 * I_)
    assert torch.equal(dgu, kernels.swiglu_backward_raw(d_act, gu, alpha, limit))


# expert sizes whose last m-tile lands on every row-group variant of the
# input-gradient kernel and its boundaries: tails of 225 (all 8 row groups),
# 193 / 224 (7), 161 / 188 (6), 160 (5), and 47 / 64 (2 of 4) / 65 (4) rows
# in the 128x512 item
COUNTS_RG = [481, 449, 160, 161, 193, 224, 64, 65, 700, 303]


@pytest.mark.parametrize("dx_cfg", [(0, 256), (23, 256)])
@pytest.mark.parametrize("gather", [True, False])
def test_dgrad_row_group_tails(dev, gather, dx_cfg):
    """gemm5's row-group variants (partial m-tiles run only their live 32-row
    groups) against the oracle, LoRA segment and routing weights included."""
    Ec = len(COUNTS_RG)
    g = torch.Generator().manual_seed(21)
    assert sum(COUNTS_RG) == T * TOPK and max(COUNTS_RG) <= T
    order = sorted(range(Ec), key=lambda e: -COUNTS_RG[e])
    multiset = [e for e in order for _ in range(COUNTS_RG[e])]
    ids = torch.empty(T, TOPK, dtype=torch.int32)
    for j, e in enumerate(multiset):
        ids[j % T, j // T] = e
    ids = ids[torch.randperm(T, generator=g)].sort(dim=1).values
    logits = torch.randn(T, Ec, generator=g).to(torch.bfloat16)
    ref = O.routing_replay(logits, ids, TOPK)
    rd, gi, si = R.routing_replay(logits.to(dev), ids.to(dev), TOPK)
    assert ref["hist"].tolist() == COUNTS_RG
    G = NOUT // 32
    blocks = torch.randint(0, 256, (Ec, KRED, G, 16), generator=g).to(torch.uint8)   # W [E, K, N] packed along N
    scales = torch.randint(118, 125, (Ec, KRED, G), generator=g).to(torch.uint8)
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16)
    Ax = (torch.randn(Ec, 32, NOUT, generator=g) * 0.3).to(torch.bfloat16)
    gam = rd.gate_scal if gather else None
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=dx_cfg[1], tile_cfg=dx_cfg[0])
    try:
        y = Q.moe_rows(x.to(dev), blocks.to(dev), scales.to(dev), None, rd, gi if gather else None, gam, True,
                       L.to(dev), Ax.to(dev))
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK,
                  gammas=gam.cpu() if gather else None, trans=True, lora_l=L, lora_b=Ax)
    a = y.float().cpu().double()
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())
