"""fp8 mode on the GPU: MXFP4 -> E5M2 (row- and column-major) and per-token
E4M3 quantization bit-exact against oracle/fp8.py; DequantMoEMatmul with
dequant_dtype="fp8" (forward and dX) against the oracle's fp8 arithmetic
(E4M3 codes x MXFP4 values, fp32 accumulation, per-token scale on the
accumulator, then bias) within the BASELINE tolerance."""
import numpy as np
import pytest
import torch

from agent_factory_3_amd import kernels
from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import fp8, moe, mxfp4
from oracle import routing as O

pytestmark = pytest.mark.gpu


def _u8(t):
    return t.view(torch.uint8).cpu().numpy()


def test_e5m2_rows_every_byte_and_scale(dev):
    blocks = np.tile(np.arange(256, dtype=np.uint8).reshape(16, 16), (256, 1, 1))      # [256 scales, 16, 16]
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    out = kernels.mxfp4_to_fp8_e5m2(torch.from_numpy(blocks).to(dev), torch.from_numpy(scales).to(dev))
    assert out.dtype == torch.float8_e5m2 and out.shape == (256, 512)
    assert np.array_equal(_u8(out), fp8.e5m2_rows(blocks, scales))


def test_e5m2_rows_weight_shape(dev):
    g = np.random.default_rng(3)
    blocks = g.integers(0, 256, (3, 576, 90, 16), dtype=np.uint8)
    scales = g.integers(118, 131, (3, 576, 90), dtype=np.uint8)
    out = kernels.mxfp4_to_fp8_e5m2_triton(torch.from_numpy(blocks).to(dev), torch.from_numpy(scales).to(dev))
    assert out.shape == (3, 576, 2880)
    assert np.array_equal(_u8(out), fp8.e5m2_rows(blocks, scales))


def test_e5m2_colmajor(dev):
    g = np.random.default_rng(4)
    blocks = g.integers(0, 256, (3, 300, 5, 16), dtype=np.uint8)
    scales = g.integers(0, 256, (3, 300, 5), dtype=np.uint8)          # every scale byte, in and out of format
    out = kernels.mxfp4_to_fp8_e5m2_colmajor(torch.from_numpy(blocks).to(dev), torch.from_numpy(scales).to(dev))
    assert out.shape == (3, 160, 300)
    assert np.array_equal(_u8(out), fp8.e5m2_colmajor(blocks, scales))


@pytest.mark.parametrize("M,K", [(257, 2880), (129, 5760), (66, 6144), (5, 6152), (33, 100), (1, 8)])
def test_quantize_per_token(dev, M, K):
    g = torch.Generator().manual_seed(M + K)
    x = (torch.randn(M, K, generator=g) * torch.logspace(-4, 4, M)[:, None]).to(torch.bfloat16)
    if M > 2:
        x[2] = 0
        x[1, : K // 2] = 3e-30          # subnormal codes next to normal ones
    codes, scale, vals = kernels.quantize_per_token_e4m3(x.to(dev), with_bf16=True)
    rc, rs = fp8.quantize_per_token(x.float().numpy())
    assert np.array_equal(scale.cpu().numpy(), rs)
    assert np.array_equal(_u8(codes.contiguous()), rc)
    assert np.array_equal(vals.float().cpu().numpy(), fp8.e4m3_to_f32(rc).astype(np.float32))
    c2, s2 = kernels.dynamic_quantize_per_token(x.to(dev))
    assert c2.dtype == torch.float8_e4m3fn and torch.equal(s2, scale)


@pytest.mark.parametrize("shift", [0, 9, -20])
def test_quantize_every_bf16_value(dev, shift):
    """Every finite bf16 value of magnitude <= 448 2^shift, in rows whose
    maximum is 448 2^shift (so the scale is 2^shift and x / scale is the bf16
    value times a power of two): every E4M3 rounding tie, the subnormal codes
    and the top of the range, bit-exact against the oracle's round-to-nearest-
    even rule, with the codes' bf16 values."""
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = bits.float()
    lim = 448.0 * 2.0 ** shift
    vals = bits[torch.isfinite(v) & (v.abs() <= lim)]
    K = 2880
    n = vals.numel()
    M = (n + K - 2) // (K - 1)
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    x[:, 0] = lim
    flat = torch.zeros(M * (K - 1), dtype=torch.bfloat16)
    flat[:n] = vals
    x[:, 1:] = flat.view(M, K - 1)
    codes, scale, out_bf16 = kernels.quantize_per_token_e4m3(x.to(dev), with_bf16=True)
    rc, rs = fp8.quantize_per_token(x.float().numpy())
    assert np.array_equal(scale.cpu().numpy(), rs) and np.all(rs == np.float32(2.0 ** shift))
    assert np.array_equal(_u8(codes.contiguous()), rc)
    assert np.array_equal(out_bf16.float().cpu().numpy(), fp8.e4m3_to_f32(rc).astype(np.float32))


def _fp8_rows(x, W, offs, gather, k, trans, bias=None, gammas=None):
    """oracle: (sum_k E4M3(x/s)[a(r)] W[e]) * s[a(r)] + bias, then gammas, bf16."""
    codes, s = fp8.quantize_per_token(x.float().numpy())
    xq = torch.from_numpy(fp8.e4m3_to_f32(codes))
    acc = moe.rows(xq, W.double(), offs, gather, k, trans=trans, rd=torch.float64)
    a = (gather.long() // k) if gather is not None else torch.arange(acc.shape[0])
    a = a.clamp_min(0)
    y = acc * torch.from_numpy(s).double()[a][:, None]
    if bias is not None:
        e = torch.repeat_interleave(torch.arange(offs.numel() - 1), (offs[1:] - offs[:-1]).long())
        y = y + bias.double()[e]
    if gammas is not None:
        y = y * gammas.double()[:, None]
    return y.to(torch.bfloat16)


@pytest.mark.parametrize("block_scaled", [True, False])
def test_dequant_moe_matmul_fp8(dev, block_scaled):
    old = Q.FP8_BLOCK_SCALED
    Q.FP8_BLOCK_SCALED = block_scaled
    try:
        _dequant_moe_matmul_fp8(dev)
    finally:
        Q.FP8_BLOCK_SCALED = old


def _dequant_moe_matmul_fp8(dev):
    g = torch.Generator().manual_seed(5)
    T, E, H, N, k = 300, 6, 256, 320, 4
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    blocks = torch.randint(0, 256, (E, N, H // 32, 16), generator=g).to(torch.uint8)
    scales = torch.randint(118, 124, (E, N, H // 32), generator=g).to(torch.uint8)
    bias = (torch.randn(E, N, generator=g) * 0.1).to(torch.bfloat16)
    ref = O.routing_topk(logits, k)
    rd, gi, si = R.routing(logits.to(dev), k)
    xd = x.to(dev).requires_grad_(True)
    y = Q.DequantMoEMatmul.apply(xd, blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi, None, None,
                                 None, si, None, "fp8", k, None, None)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = _fp8_rows(x, W, ref["offs"], ref["topk_indx"], k, False, bias=bias)
    a, b = y.float().cpu().double(), yr.double()
    assert y.shape == yr.shape and torch.isfinite(a).all()
    assert ((a - b).abs() <= 1e-2 + 2e-2 * b.abs()).all()
    # dX: the incoming gradient rows quantized per row, W[e] (not transposed), combined per token
    dy = torch.randn(y.shape, generator=g).to(torch.bfloat16)
    y.backward(dy.to(dev))
    dxr = _fp8_rows(dy, W, ref["offs"], None, 1, True)
    dx = moe.combine(dxr, ref["gate_indx"], k)
    a, b = xd.grad.float().cpu().double(), dx.double()
    assert ((a - b).abs() <= 1e-2 + 2e-2 * b.abs()).all()
    # bf16 mode on the same inputs differs (the activations are quantized here)
    y16 = Q.DequantMoEMatmul.apply(x.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi, None,
                                   None, None, si, None, "bf16", k, None, None)
    assert not torch.equal(y16, y)


@pytest.mark.parametrize("gather,odd", [(True, False), (False, False), (True, True)])
def test_block_scaled_forward_tiles(dev, gather, odd):
    """The block-scaled fp8 forward kernel on full, partial, <= 128-row (two
    n-tiles per work item) and idle-expert tiles, ten k-steps, N = 576; with
    ``odd`` also e8m0 bytes 0, 1, 254, 255 (the MFMA applies them as powers of
    two where the reference's E5M2 bytes flush or wrap: checked for finiteness
    and against the oracle outside those blocks)."""
    from test_gpu_gemm_tiles import KRED, NOUT, T, TOPK, _routing, _weights
    g, ref, rd, gi = _routing(dev, 21)
    blocks, scales = _weights(g, NOUT, KRED, odd)
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    bias = (torch.randn(blocks.shape[0], NOUT, generator=g) * 0.1).to(torch.bfloat16)
    codes, s = kernels.quantize_per_token_e4m3(x.to(dev))
    y = Q.moe_rows_f8(codes, s, blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi if gather else None)
    assert y is not None and y.shape == (Rr, NOUT)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = _fp8_rows(x, W, ref["offs"], ref["topk_indx"] if gather else None, TOPK, False, bias=bias)
    a, b = y.float().cpu().double(), yr.double()
    skip = torch.zeros(a.shape, dtype=torch.bool)
    if odd:   # output columns whose weight row holds a scale byte outside [2, 252] (see the docstring)
        bad_rows = ((scales < 2) | (scales > 252)).any(dim=2)          # [E, N]
        e_of = torch.repeat_interleave(torch.arange(len(ref["offs"]) - 1), (ref["offs"][1:] - ref["offs"][:-1]).long())
        skip = bad_rows[e_of]
        assert skip.any() and not skip.all()
    assert torch.isfinite(a[~skip]).all()
    ok = ((a - b).abs() <= 1e-2 + 2e-2 * b.abs()) | skip
    assert ok.all(), float((~ok).float().mean())


@pytest.mark.parametrize("gather,odd", [(True, False), (False, False), (True, True)])
def test_block_scaled_dgrad_tiles(dev, gather, odd):
    """The fp8 input-gradient kernel (weights converted to E5M2 in registers) on
    the tile shapes of the bf16 kernels' tests, against the oracle over the
    reference's E5M2 weight bytes (kernels.py:238-312) and the per-token E4M3
    gradient.  ``odd`` plants e8m0 bytes 0, 1, 254, 255, which the kernel's
    exact integer path turns into the reference's flushed / wrapped bytes, so
    every output is compared."""
    from test_gpu_gemm_tiles import KRED, NOUT, T, TOPK, _routing, _weights
    g, ref, rd, gi = _routing(dev, 22)
    blocks, scales = _weights(g, KRED, NOUT, odd)          # W [E, K, N], packed along N
    Rr = T * TOPK
    x = torch.randn(T if gather else Rr, KRED, generator=g).to(torch.bfloat16)
    gam = rd.gate_scal if gather else None
    codes, s = kernels.quantize_per_token_e4m3(x.to(dev))
    y = Q.moe_rows_f8(codes, s, blocks.to(dev), scales.to(dev), None, rd, gi if gather else None, gam, trans_w=True)
    assert y is not None and y.shape == (Rr, NOUT)
    w8 = fp8.e5m2_colmajor(blocks.numpy(), scales.numpy())            # [E, N, K] bytes
    W8 = torch.from_numpy(fp8.e5m2_to_f32(w8)).transpose(1, 2)        # [E, K, N] values
    assert torch.isfinite(W8).all()
    yr = _fp8_rows(x, W8, ref["offs"], ref["topk_indx"] if gather else None, TOPK, True,
                   gammas=gam.cpu() if gather else None)
    a, b = y.float().cpu().double(), yr.double()
    assert torch.isfinite(a).all()
    ok = (a - b).abs() <= 1e-2 + 2e-2 * b.abs()
    assert ok.all(), float((~ok).float().mean())
