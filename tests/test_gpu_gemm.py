"""Grouped GEMM / combine / expert-LoRA HIP kernels vs the oracle (A6, A8, A9, A11, A13)."""
import pytest
import torch

from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from oracle import moe, mxfp4
from oracle import routing as O
from tests._tol import ATOL, RTOL, check_close, combined_slack

pytestmark = pytest.mark.gpu



def _close(gpu, ref, rtol=RTOL, atol=ATOL, **kw):
    check_close(gpu, ref, rtol=rtol, atol=atol, **kw)
    return True, 0.0


def _problem(T=300, E=6, K=4, H=128, N=192, seed=0, scale_lo=118, scale_hi=124, skew=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    if skew:  # expert 0 popular (>128 rows), expert E-1 idle
        logits[:, 0] += 3.0
        logits[:, E - 1] -= 50.0
    blocks = torch.randint(0, 256, (E, N, H // 32, 16), generator=g).to(torch.uint8)
    scales = torch.randint(scale_lo, scale_hi + 1, (E, N, H // 32), generator=g).to(torch.uint8)
    bias = (torch.randn(E, N, generator=g) * 0.1).to(torch.bfloat16)
    return g, x, logits, blocks, scales, bias


def _route(logits, K, dev):
    ref = O.routing_topk(logits, K)
    out = R.routing(logits.to(dev), K)
    return ref, out


def test_gate_up_forward_gather_bias(dev):
    g, x, logits, blocks, scales, bias = _problem()
    ref, (rd, gi, si) = _route(logits, 4, dev)
    assert int(ref["hist"][0]) > 128 and int(ref["hist"][-1]) == 0
    y = Q.moe_rows(x.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(x, W, ref["offs"], ref["topk_indx"], 4, bias=bias)
    ok, frac = _close(y, yr)
    assert ok, frac


def test_down_forward_gammas_and_combine(dev):
    g, x, logits, blocks, scales, bias = _problem(H=192, N=128, seed=1)
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    R_ = x.shape[0] * K
    act = torch.randn(R_, 192, generator=g).to(torch.bfloat16)
    y = Q.matmul_ogs(act.to(dev), (blocks.to(dev), scales.to(dev)), bias.float().to(dev), rd, None, si,
                     rd.gate_scal)
    W = mxfp4.dequant_f32(blocks, scales)
    gam = rd.gate_scal.cpu()  # the GPU routing's weights, so both sides see identical inputs
    yr = moe.rows(act, W, ref["offs"], None, 1, bias=bias, gammas=gam)
    check_close(y, moe.combine(yr, ref["gate_indx"], K), extra=combined_slack(yr, ref["gate_indx"], K),
                what="down rows + combine")
    # the combine kernel alone, on identical rows: fp32 sum of bf16 rows, one rounding
    rows_dev = Q.moe_rows(act.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, None, rd.gate_scal)
    out = Q.moe_combine(rows_dev, si, K)
    assert torch.equal(out.cpu(), moe.combine(rows_dev.cpu(), ref["gate_indx"], K))


@pytest.mark.parametrize("K", [1, 3, 6, 10])
def test_combine_any_k_bit_exact(dev, K):
    """af3_moe_combine at k = 1 .. 10 (all rows in flight for k <= 4 and <= 8,
    one at a time beyond), with dropped (-1) entries: bit-equal to the
    oracle's in-order fp32 sum of the bf16 rows."""
    import types
    g = torch.Generator().manual_seed(40 + K)
    T, N = 300, 264
    rows = torch.randn(T * K + 5, N, generator=g).to(torch.bfloat16)
    src = torch.randperm(T * K + 5, generator=g)[:T * K].to(torch.int32)
    src[torch.randint(0, T * K, (T // 3,), generator=g)] = -1
    out = Q.moe_combine(rows.to(dev), types.SimpleNamespace(src_indx=src.to(dev)), K)
    assert out.shape == (T, N)
    assert torch.equal(out.cpu(), moe.combine(rows, src, K))


@pytest.mark.parametrize("gather", [True, False])
def test_dgrad_transposed_weights(dev, gather):
    g, x, logits, blocks, scales, bias = _problem(H=160, N=224, seed=2)  # W [E, 224, 160]
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    R_ = x.shape[0] * K
    rows_in = torch.randn(x.shape[0] if gather else R_, 224, generator=g).to(torch.bfloat16)
    gam = rd.gate_scal if gather else None
    y = Q.moe_rows(rows_in.to(dev), blocks.to(dev), scales.to(dev), None, rd, gi if gather else None, gam,
                   trans_w=True)
    W = mxfp4.dequant_f32(blocks, scales)
    yr = moe.rows(rows_in, W, ref["offs"], ref["topk_indx"] if gather else None, K,
                  gammas=rd.gate_scal.cpu() if gather else None, trans=True)
    assert y.shape == (R_, 160)
    ok, frac = _close(y, yr)
    assert ok, frac


@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("r", [8, 16, 24, 40, 64])
def test_lora_extension_segment(dev, trans, r):
    """The rank-r segment after the main k-loop: ranks that end inside a
    16-deep MFMA sub-step (8, 24, 40) and that fill the whole 64-deep step."""
    g, x, logits, blocks, scales, bias = _problem(H=128, N=192, seed=3 + r)
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    E = blocks.shape[0]
    W = mxfp4.dequant_f32(blocks, scales)
    L = (torch.randn(x.shape[0] * K, r, generator=g) * 0.5).to(torch.bfloat16)
    if not trans:
        Bx = (torch.randn(E, 192, r, generator=g) * 0.5).to(torch.bfloat16)
        y = Q.moe_rows(x.to(dev), blocks.to(dev), scales.to(dev), bias.float().to(dev), rd, gi, None, False,
                       L.to(dev), Bx.to(dev))
        yr = moe.rows(x, W, ref["offs"], ref["topk_indx"], K, bias=bias, lora_l=L, lora_b=Bx)
    else:
        xin = torch.randn(x.shape[0], 192, generator=g).to(torch.bfloat16)
        Ax = (torch.randn(E, r, 128, generator=g) * 0.5).to(torch.bfloat16)
        y = Q.moe_rows(xin.to(dev), blocks.to(dev), scales.to(dev), None, rd, gi, rd.gate_scal, True,
                       L.to(dev), Ax.to(dev))
        yr = moe.rows(xin, W, ref["offs"], ref["topk_indx"], K, gammas=rd.gate_scal.cpu(), trans=True,
                      lora_l=L, lora_b=Ax)
    ok, frac = _close(y, yr)
    assert ok, frac


@pytest.mark.parametrize("trans,r", [(False, 16), (True, 16), (False, 32), (True, 32)])
def test_lora_rows(dev, trans, r):
    g, x, logits, blocks, scales, bias = _problem(seed=4)
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    E, Kd = blocks.shape[0], 128
    Wl = (torch.randn(E, Kd, r, generator=g) if trans else torch.randn(E, r, Kd, generator=g)).to(torch.bfloat16)
    out = Q._lora_rows(x.to(dev), gi.src_indx, K, Wl.to(dev), 1 if trans else 0, 2.0, rd.expt_data, r, Kd)
    refo = moe.lora_rows(x, Wl, ref["offs"], ref["topk_indx"], K, 2.0, trans=trans)
    ok, frac = _close(out, refo)
    assert ok, frac


@pytest.mark.parametrize("M,N,gather_a,gather_b,rowscale", [
    (192, 16, False, False, True), (16, 128, False, True, False), (192, 32, False, True, True),
    (32, 160, False, False, False),
    (320, 32, True, False, True),   # the dB form: wide operand gathered + row-scaled, rank side plain
    (32, 384, False, True, True),   # the dA form: rank side row-scaled, wide operand gathered
])
def test_lora_wgrad(dev, M, N, gather_a, gather_b, rowscale):
    g, x, logits, blocks, scales, bias = _problem(seed=5)
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    R_ = x.shape[0] * K
    a = torch.randn(x.shape[0] if gather_a else R_, M, generator=g).to(torch.bfloat16)
    b = torch.randn(x.shape[0] if gather_b else R_, N, generator=g).to(torch.bfloat16)
    E = blocks.shape[0]
    rs = rd.gate_scal if rowscale else None
    out = Q._lora_wgrad(a.to(dev), gi.src_indx if gather_a else None, K if gather_a else 1, rs, b.to(dev),
                        gi.src_indx if gather_b else None, K if gather_b else 1, rd.expt_data, E, M, N).cpu()
    assert int(ref["hist"][-1]) == 0 and out[-1].abs().max() == 0     # idle expert -> zero gradient
    offs, ti = ref["offs"], ref["topk_indx"].long()
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi == lo:
            continue
        ia = ti[lo:hi] // K if gather_a else torch.arange(lo, hi)
        ib = ti[lo:hi] // K if gather_b else torch.arange(lo, hi)
        # the GPU routing's weights as the row scale, so both sides see identical inputs
        refo, mag = moe.expert_wgrad(a[ia], b[ib], rs.cpu()[lo:hi] if rowscale else None)
        check_close(out[e], refo, mag=mag, n=hi - lo, what=f"wgrad expert {e}")


@pytest.mark.parametrize("W,r,gather,rowscale", [
    (2880, 32, True, True),     # the down projection's form: dY gathered, gammas on dB
    (5760, 16, False, False),   # gate_up's form; the last column group has one empty slice
    (264, 32, False, True),     # one group, a 8-column last slice
    (1288, 16, True, False),    # two groups, the second with 264 columns
])
def test_lora_u_and_dB_one_pass(dev, W, r, gather, rowscale):
    """u = s big[b] @ B[e] and dB[e] = sum bf16(rs big[b])^T L in one pass over big: u against the
    oracle, dB against the oracle and bit for bit against the two-pass kernels (same sums in the
    same order).  Expert 0 holds > 512 rows (several chunks), the last expert none."""
    g, x, logits, blocks, scales, bias = _problem(T=700, seed=11)
    K = 4
    ref, (rd, gi, si) = _route(logits, K, dev)
    E, R_ = blocks.shape[0], x.shape[0] * K
    assert int(ref["hist"][0]) > 512 and int(ref["hist"][-1]) == 0
    big = torch.randn(x.shape[0] if gather else R_, W, generator=g).to(torch.bfloat16)
    L = torch.randn(R_, r, generator=g).to(torch.bfloat16)
    Bw = (torch.randn(E, W, r, generator=g) * 0.1).to(torch.bfloat16)
    rs = rd.gate_scal.to(torch.bfloat16) if rowscale else None
    gx = gi.src_indx if gather else None
    div = K if gather else 1
    ed = rd.expt_data
    u, dB = Q._lora_u_and_dB(big.to(dev), gx, div, rs, L.to(dev), Bw.to(dev), 0.5, ed, E, W)
    u2 = Q._lora_rows(big.to(dev), gx, div, Bw.to(dev), 1, 0.5, ed, r, W)
    dB2 = Q._lora_wgrad(big.to(dev), gx, div, rs, L.to(dev), None, 1, ed, E, W, r)
    u, dB, u2, dB2 = u.cpu(), dB.cpu(), u2.cpu(), dB2.cpu()
    assert torch.equal(dB.view(torch.int16), dB2.view(torch.int16))
    assert dB[-1].abs().max() == 0
    offs, ti = ref["offs"], ref["topk_indx"].long()
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi == lo:
            continue
        ib = ti[lo:hi] // K if gather else torch.arange(lo, hi)
        uref, umag = moe.expert_lora_rows(big, Bw[e], ib, 0.5, trans=True)
        check_close(u[lo:hi], uref, mag=umag, n=W, what=f"u expert {e}")
        check_close(u2[lo:hi], uref, mag=umag, n=W, what=f"u (two-pass) expert {e}")
        dref, dmag = moe.expert_wgrad(big[ib], L[lo:hi], rs.cpu()[lo:hi] if rowscale else None)
        check_close(dB[e], dref, mag=dmag, n=hi - lo, what=f"dB expert {e}")


def test_dense_routing_none(dev):
    """matmul_ogs with routing_data=None: one expert, plain GEMM."""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(70, 64, generator=g).to(torch.bfloat16)
    blocks = torch.randint(0, 256, (96, 2, 16), generator=g).to(torch.uint8)
    scales = torch.randint(120, 126, (96, 2), generator=g).to(torch.uint8)
    y = Q.matmul_ogs(x.to(dev), (blocks.to(dev), scales.to(dev)), None)
    W = mxfp4.dequant_f32(blocks, scales)
    ok, frac = _close(y, (x.float() @ W.T).to(torch.bfloat16))
    assert ok, frac
