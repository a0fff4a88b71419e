"""Tiled weights (af3_mxfp4_tile_fwd) and tiled input-gradient scales
(af3_mxfp4_tile_dx_scales): the byte permutations themselves, and the default
forward / input-gradient kernels reading them give the same bits as reading
the blocks and scales as stored, on the shapes of test_gpu_gemm_tiles (full
and partial tiles, 64- / 128-column tail n-tiles, tails of 1 to 4 row groups,
gathered rows, the LoRA segment, scale bytes outside [2, 252], the fused
SwiGLU forward and backward), and against the oracle.  Kernels that do not
read a tiled copy decline it and run on the stored bytes."""
import pytest
import torch

from agent_factory_3_amd import _capi
from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import moe, mxfp4
from oracle import routing as O
from test_gpu_gemm_tiles import ATOL, CASES, E, KRED, RTOL, T, TOPK, _routing, _weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(3, 96, 6), (1, 32, 2), (5, 640, 20)])
def test_tile_fwd_permutation(dev, shape):
    """out[e, n // 32, kt, h, n % 32] == blocks[e, n, 2 kt + h] for every byte."""
    En, N, G = shape
    g = torch.Generator().manual_seed(N + G)
    blocks = torch.randint(0, 256, (En, N, G, 16), generator=g).to(torch.uint8)
    out = Q.mxfp4_tile_fwd(blocks.to(dev)).cpu()
    assert out.shape == blocks.shape
    want = blocks.view(En, N // 32, 32, G // 2, 2, 16).permute(0, 1, 3, 4, 2, 5).contiguous()
    assert torch.equal(out.view(En, N // 32, G // 2, 2, 32, 16), want)
    # spot check of the indexing rule itself on a few bytes
    t = out.view(En, N // 32, G // 2, 2, 32, 16)
    for e, n, j in [(0, 0, 0), (En - 1, N - 1, G - 1), (En // 2, N // 2 + 1, G // 2)]:
        assert torch.equal(t[e, n // 32, j // 2, j % 2, n % 32], blocks[e, n, j])


def test_tile_fwd_rejects_bad_shapes(dev):
    with pytest.raises(RuntimeError, match="N % 32"):
        Q.mxfp4_tile_fwd(torch.zeros(2, 48, 4, 16, dtype=torch.uint8, device=dev))
    with pytest.raises(RuntimeError, match="K % 64"):
        Q.mxfp4_tile_fwd(torch.zeros(2, 64, 3, 16, dtype=torch.uint8, device=dev))


@pytest.mark.parametrize("cfg,nout", [(0, 576), (0, 640), (126, 576), (22, 640), (4, 576)])
@pytest.mark.parametrize("gather,lora,odd", CASES)
def test_forward_tiled_bit_equal(dev, cfg, nout, gather, lora, odd):
    """moe_rows with w_tiled equals moe_rows on the stored blocks bit for bit
    (tile_cfg 0 / 126 read the tiled copy; 22 and 4 decline it)."""
    g, ref, rd, gi = _routing(dev, 21)
    blocks, scales = _weights(g, nout, KRED, odd)
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, nout, generator=g) * 0.1).float().to(dev)
    gam = rd.gate_scal if gather else None
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Bx = (torch.randn(E, nout, 32, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    wb, ws = blocks.to(dev), scales.to(dev)
    wt = Q.mxfp4_tile_fwd(wb)
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE.update(block_m=256, tile_cfg=cfg)
    try:
        y_ref = Q.moe_rows(x, wb, ws, bias, rd, gi if gather else None, gam, False, L, Bx)
        y = Q.moe_rows(x, wb, ws, bias, rd, gi if gather else None, gam, False, L, Bx, w_tiled=wt)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    assert torch.isfinite(y.float()).all()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))


@pytest.mark.parametrize("lora", [False, True])
def test_forward_tiled_swiglu_bit_equal(dev, lora):
    """The gate_up forward with its fused SwiGLU (epi 2) on the tiled copy."""
    g, ref, rd, gi = _routing(dev, 22)
    alpha, limit, I_ = 1.702, 7.0, 320
    blocks, scales = _weights(g, 2 * I_, KRED, False)
    Rr = T * TOPK
    x = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    bias = (torch.randn(E, 2 * I_, generator=g) * 0.5).float().to(dev)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    Bx = (torch.randn(E, 2 * I_, 32, generator=g) * 0.3).to(torch.bfloat16).to(dev) if lora else None
    wb, ws = blocks.to(dev), scales.to(dev)
    gu_ref, act_ref = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx, swiglu=("fwd", alpha, limit))
    gu, act = Q.moe_rows(x, wb, ws, bias, rd, gi, None, False, L, Bx, swiglu=("fwd", alpha, limit),
                         w_tiled=Q.mxfp4_tile_fwd(wb))
    assert torch.equal(gu.view(torch.int16), gu_ref.view(torch.int16))
    assert torch.equal(act.view(torch.int16), act_ref.view(torch.int16))


def test_tiled_flag_declined_by_other_kernels(dev):
    """The C entry point returns AF3_EUNSUPPORTED (nothing launched) for the
    tiled flag on the input gradient."""
    g, ref, rd, gi = _routing(dev, 23)
    blocks, scales = _weights(g, KRED, 576, False)
    wb, ws = blocks.to(dev), scales.to(dev)
    x = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    ed = rd.expt_data
    y = torch.zeros(T * TOPK, 576, dtype=torch.bfloat16, device=dev)
    pid = ed.block_pid_map[128]
    gp = Q._gather_ptr(gi)
    ok = _capi.try_call("af3_moe_gemm", x.data_ptr(), KRED, gp.data_ptr(), TOPK, wb.data_ptr(),
                        ws.data_ptr(), 1, None, None, 0, None, 0, None, 0, ed.token_offs_raw.data_ptr(),
                        pid.data_ptr(), ed.token_offs_pad[128].data_ptr(), pid.numel(), 128, _capi.W_FWD_TILED,
                        E, 576, KRED, y.data_ptr(), 576, _capi.stream_of(dev))
    torch.cuda.synchronize()
    assert not ok
    assert int(y.view(torch.int16).abs().sum()) == 0


def test_module_cache(dev):
    """The expert module makes the tiled weights and the tiled scales once per
    weight version."""
    from agent_factory_3_amd import workloads
    m = workloads.make_experts(workloads.layer(2, T=64, E=4, H=256, I=128), dev)
    a = m._fwd_tiled("gate_up_proj")
    assert a is not None and m._fwd_tiled("gate_up_proj") is a
    blocks, _ = m._get_uint8_weights("gate_up_proj")
    assert torch.equal(a, Q.mxfp4_tile_fwd(blocks))
    with torch.no_grad():
        w = getattr(m, "gate_up_proj_blocks")
        w.copy_(w.clone())  # an in-place write (same bytes) bumps the version
    b = m._fwd_tiled("gate_up_proj")
    assert b is not a and torch.equal(b, a)
    # the input gradient's tiled scales, the same way
    s1 = m._dx_tiled_scales("down_proj")
    assert s1 is not None and m._dx_tiled_scales("down_proj") is s1
    _, scales = m._get_uint8_weights("down_proj")
    assert torch.equal(s1, Q.mxfp4_tile_dx_scales(scales))
    with torch.no_grad():
        w = getattr(m, "down_proj_scales")
        w.copy_(w.clone())
    s2 = m._dx_tiled_scales("down_proj")
    assert s2 is not s1 and torch.equal(s2, s1)


# rows per expert whose last 128-row tile has 2, 3, 1, 1, 4 and 4 live 32-row
# groups (tails of 60, 74, 20, 10, 100 and 104 rows) and an idle expert
COUNTS_NB3 = [700, 330, 660, 650, 100, 360, 0]


def _routing_counts(dev, seed, counts):
    g = torch.Generator().manual_seed(seed)
    assert sum(counts) == T * TOPK and max(counts) <= T
    order = sorted(range(len(counts)), key=lambda e: -counts[e])
    multiset = [e for e in order for _ in range(counts[e])]
    ids = torch.empty(T, TOPK, dtype=torch.int32)
    for j, e in enumerate(multiset):
        ids[j % T, j // T] = e
    ids = ids[torch.randperm(T, generator=g)].sort(dim=1).values
    logits = torch.randn(T, len(counts), generator=g).to(torch.bfloat16)
    ref = O.routing_replay(logits, ids, TOPK)
    rd, gi, si = R.routing_replay(logits.to(dev), ids.to(dev), TOPK)
    assert ref["hist"].tolist() == counts
    return g, ref, rd, gi


@pytest.mark.parametrize("nout", [576, 640])
@pytest.mark.parametrize("gather,lora,odd", CASES)
def test_forward_three_weight_buffers(dev, nout, gather, lora, odd):
    """K = 576 (nine k-steps, a multiple of three) with N % 64 == 0 runs the
    forward with the weight words two k-steps ahead and a k-loop compiled per
    count of live row groups (tails of 1, 2, 3 and 4 groups, the exact
    conversion for out-of-range scale bytes among them): against the oracle,
    with the stored and with the tiled weights, and with scalar-base (x within
    4 GiB, the default) and 64-bit addressing."""
    K = 576
    g, ref, rd, gi = _routing_counts(dev, 31, COUNTS_NB3)
    blocks, scales = _weights(g, nout, K, odd)
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, K, generator=g).to(torch.bfloat16)
    bias = (torch.randn(E, nout, generator=g) * 0.1).to(torch.bfloat16)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    Bx = (torch.randn(E, nout, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    wb, ws = blocks.to(dev), scales.to(dev)
    args = (x.to(dev), wb, ws, bias.float().to(dev), rd, gi if gather else None, None, False,
            L.to(dev) if lora else None, Bx.to(dev) if lora else None)
    y = Q.moe_rows(*args)
    wt = Q.mxfp4_tile_fwd(wb)
    yt = Q.moe_rows(*args, w_tiled=wt)
    assert torch.equal(y.view(torch.int16), yt.view(torch.int16))
    # the same kernel with 64-bit addresses (no 32-bit offset guarantee from the caller)
    old = dict(Q.GEMM_TILE)
    Q.GEMM_TILE["x_off32"] = False
    try:
        y64 = Q.moe_rows(*args, w_tiled=wt)
    finally:
        Q.GEMM_TILE.clear()
        Q.GEMM_TILE.update(old)
    assert torch.equal(y.view(torch.int16), y64.view(torch.int16))
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK, bias=bias, lora_l=L, lora_b=Bx)
    a = y.float().cpu().double()
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())



@pytest.mark.parametrize("shape", [(3, 128, 18), (2, 64, 8), (1, 192, 20)])
def test_tile_dx_scales_permutation(dev, shape):
    """out[e, k // 64, n // 256, (n // 32) % 8, k % 64] == scales[e, k, n // 32],
    127 past N / 32, for every byte; then one flag per (matrix, n-tile): 1 when
    a byte of its columns lies outside [2, 252]."""
    En, K, G = shape
    g = torch.Generator().manual_seed(K + G)
    scales = torch.randint(2, 253, (En, K, G), generator=g).to(torch.uint8)
    scales[0, K - 1, G - 1] = 255                       # odd byte in the last n-tile of matrix 0
    if En > 1:
        scales[1, 3, 0] = 1                             # and in the first n-tile of matrix 1
    out = Q.mxfp4_tile_dx_scales(scales.to(dev)).cpu()
    nt = (G * 32 + 255) // 256
    nbytes = En * (K // 64) * nt * 512
    assert out.shape == (nbytes + En * nt,)
    padded = torch.full((En, K, nt * 8), 127, dtype=torch.uint8)
    padded[:, :, :G] = scales
    want = padded.view(En, K // 64, 64, nt, 8).permute(0, 1, 3, 4, 2)
    assert torch.equal(out[:nbytes].view(En, K // 64, nt, 8, 64), want)
    flags = torch.zeros(En, nt, dtype=torch.uint8)
    flags[0, nt - 1] = 1
    if En > 1:
        flags[1, 0] = 1
    assert torch.equal(out[nbytes:].view(En, nt), flags)


@pytest.mark.parametrize("nout", [576, 640])
@pytest.mark.parametrize("gather,lora,odd", CASES)
def test_dgrad_tiled_scales_bit_equal(dev, nout, gather, lora, odd):
    """The default input-gradient kernel (tile_cfg 28) reading the tiled
    scales equals it on the stored scales bit for bit (scale bytes outside
    [2, 252] included: the exact conversion), and the oracle; tails of 1, 2
    and 3 row groups take its row-group variants."""
    g, ref, rd, gi = _routing_counts(dev, 32, COUNTS_NB3)
    blocks, scales = _weights(g, KRED, nout, odd)          # W [E, K, N] packed along N
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    L = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    Ax = (torch.randn(E, 32, nout, generator=g) * 0.3).to(torch.bfloat16) if lora else None
    gam = rd.gate_scal if gather else None
    wb, ws = blocks.to(dev), scales.to(dev)
    args = (x.to(dev), wb, ws, None, rd, gi if gather else None, gam, True, L.to(dev) if lora else None,
            Ax.to(dev) if lora else None)
    y = Q.moe_rows(*args)
    yt = Q.moe_rows(*args, s_tiled=Q.mxfp4_tile_dx_scales(ws))
    assert torch.equal(y.view(torch.int16), yt.view(torch.int16))
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK,
                  gammas=gam.cpu() if gather else None, trans=True, lora_l=L, lora_b=Ax)
    a = yt.float().cpu().double()
    assert torch.isfinite(a).all()
    bad = (a - yr.double()).abs() > ATOL + RTOL * yr.double().abs()
    assert not bad.any(), float(bad.float().mean())


def test_dgrad_tiled_scales_swiglu_bit_equal(dev):
    """The down projection's input gradient with the fused SwiGLU backward
    (epi 1) on the tiled scales."""
    g, ref, rd, gi = _routing_counts(dev, 33, COUNTS_NB3)
    alpha, limit, I_ = 1.702, 7.0, 320
    Rr = T * TOPK
    gu = (torch.randn(Rr, 2 * I_, generator=g) * 3).to(torch.bfloat16).to(dev)
    blocks, scales = _weights(g, KRED, I_, True)           # down W [E, H, I] read transposed
    dy = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    u = (torch.randn(Rr, 32, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    Ax = (torch.randn(E, 32, I_, generator=g) * 0.3).to(torch.bfloat16).to(dev)
    wb, ws = blocks.to(dev), scales.to(dev)
    args = (dy, wb, ws, None, rd, gi, rd.gate_scal, True, u, Ax)
    dgu = Q.moe_rows(*args, swiglu=("bwd", gu, alpha, limit))
    dgu_t = Q.moe_rows(*args, swiglu=("bwd", gu, alpha, limit), s_tiled=Q.mxfp4_tile_dx_scales(ws))
    assert dgu is not None and dgu_t is not None
    assert torch.equal(dgu.view(torch.int16), dgu_t.view(torch.int16))


def test_tiled_scales_declined_by_the_forward(dev):
    """AF3_S_DX_TILED on a forward call: AF3_EUNSUPPORTED, nothing launched."""
    g, ref, rd, gi = _routing(dev, 24)
    blocks, scales = _weights(g, 576, KRED, False)
    wb, ws = blocks.to(dev), scales.to(dev)
    x = torch.randn(T, KRED, generator=g).to(torch.bfloat16).to(dev)
    ed = rd.expt_data
    y = torch.zeros(T * TOPK, 576, dtype=torch.bfloat16, device=dev)
    pid = ed.block_pid_map[128]
    gp = Q._gather_ptr(gi)
    ok = _capi.try_call("af3_moe_gemm", x.data_ptr(), KRED, gp.data_ptr(), TOPK, wb.data_ptr(),
                        ws.data_ptr(), 0, None, None, 0, None, 0, None, 0, ed.token_offs_raw.data_ptr(),
                        pid.data_ptr(), ed.token_offs_pad[128].data_ptr(), pid.numel(), 128, _capi.S_DX_TILED,
                        E, 576, KRED, y.data_ptr(), 576, _capi.stream_of(dev))
    torch.cuda.synchronize()
    assert not ok
    assert int(y.view(torch.int16).abs().sum()) == 0
