"""LM-head log-probabilities / entropy (linear_cross_entropy) on the GPU
against oracle/lmhead.py on the same bf16 inputs, in both logits modes
(library: fp32 logits of each vocabulary chunk from a plain GEMM, then the
statistics / gradient kernels; fused: the GEMM kernel with them in its
epilogue): forward values (the GEMMs accumulate in fp32, so only summation
order separates them from float64), the fused logits gradient per vocabulary
split (bit-equal to the whole-vocabulary kernel), gradients of hidden and
weight through the split backward, the three reductions, out-of-range labels,
partial row / vocabulary tiles, chunks that split the vocabulary raggedly and
rows the vector loads cannot take, the full gpt-oss vocabulary (201,088), and
rows more than 4 GiB past the fused kernel's bases (its 64-bit copy addresses)."""
import pytest
import torch

from agent_factory_3_amd import _capi
from agent_factory_3_amd import linear_cross_entropy as lce
from agent_factory_3_amd.linear_cross_entropy import linear_cross_entropy
from oracle import lmhead
from tests._tol import check_close

pytestmark = pytest.mark.gpu


def _inputs(M, H, V, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(M, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) * scale).to(torch.bfloat16)
    lab = torch.randint(0, V, (M,), generator=g)
    return h, w, lab


def _close(got, ref, atol, rtol):
    """Fraction of elements outside atol + rtol |ref| (a non-finite value fails)."""
    got = got.detach().float().cpu().double()
    assert torch.isfinite(got).all(), "non-finite values"
    return float(((got - ref).abs() > atol + rtol * ref.abs()).float().mean())


def _split(monkeypatch, M, cols):
    """Force backward splits of ``cols`` vocabulary columns for M rows."""
    monkeypatch.setattr(lce, "SPLIT_BYTES", 2 * M * cols)
    assert lce.vocab_split(M, 10 ** 6) == cols


def _mode(monkeypatch, mode, M, chunk):
    """Logits modes "forward/backward"; library chunks of ``chunk`` vocabulary columns."""
    fwd, bwd = mode.split("/")
    monkeypatch.setattr(lce, "LOGITS_GEMM", fwd)
    monkeypatch.setattr(lce, "DLOGITS_GEMM", bwd)
    if chunk:
        monkeypatch.setattr(lce, "CHUNK_BYTES", 4 * M * chunk)
        assert lce.logits_chunk(M, 10 ** 6) == chunk


MODES = [("library/library", 256), ("library/fused", 0), ("fused/fused", 0), ("fused/library", 0)]


def _check_grads(hd, wd, h, w, lab, T, dlp, dent, hr, wr, lse, ez, what):
    """d_hidden / d_weight against (1) the exact float64 gradients, within the
    north-star tolerance scaled to the gradient's size (the bf16 logits gradient
    is the only rounding that separates them), and (2) the same GEMMs in float64
    over the GPU's own bf16 logits gradient (the mode's lm_head_dlogits, which
    forms the values the backward forms), within a bf16 output rounding plus
    the fp32 accumulation allowance."""
    for got, ref in ((hd.grad, hr.grad), (wd.grad, wr.grad)):
        scale = float(ref.abs().max())
        check_close(got, ref, rtol=2e-2, atol=1e-2 * scale, what=f"{what} vs float64")
    dz = lce.lm_head_dlogits(hd.detach(), wd.detach(), lab.to(hd.device), T, lse, ez, dlp.to(hd.device),
                             dent.to(hd.device)).double().cpu()
    h64, w64 = h.double(), w.double()
    V = w.shape[0]
    check_close(hd.grad, dz @ w64, rtol=2.0 ** -8, atol=1e-9, mag=dz.abs() @ w64.abs(), n=V,
                what=f"{what} d_hidden vs the GEMM over the GPU logits gradient")
    check_close(wd.grad, dz.t() @ h64, rtol=2.0 ** -8, atol=1e-9, mag=dz.abs().t() @ h64.abs(), n=h.shape[0],
                what=f"{what} d_weight vs the GEMM over the GPU logits gradient")


@pytest.mark.parametrize("mode,chunk", MODES)
@pytest.mark.parametrize("M,H,V,T,cols", [(300, 128, 1000, 1.0, 256), (257, 96, 513, 0.7, 512),
                                          (64, 64, 256, 1.3, 256), (300, 128, 1000, 1.0, 1024)])
def test_forward_and_backward(dev, monkeypatch, M, H, V, T, cols, mode, chunk):
    h, w, lab = _inputs(M, H, V, seed=M + V)
    lab[5] = -100
    lab[6], lab[7], lab[8] = 255, 256, V - 1  # the last and first column of two splits, the last entry
    _split(monkeypatch, M, cols)
    _mode(monkeypatch, mode, M, chunk)
    print(f"lm_head M={M} H={H} V={V} T={T} split={cols} {mode} chunk={chunk}", flush=True)
    hd = h.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    lp, ent = linear_cross_entropy(hd, wd, lab.to(dev), T, "none")
    g = torch.Generator().manual_seed(1)
    dlp = torch.randn(M, generator=g)
    dent = torch.randn(M, generator=g)
    (lp * dlp.to(dev)).sum().add((ent * dent.to(dev)).sum()).backward()
    torch.cuda.synchronize()

    hr = h.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    lpr, entr = lmhead.lm_head(hr, wr, lab, T)
    ((lpr * dlp.double()).sum() + (entr * dent.double()).sum()).backward()
    assert _close(lp, lpr.detach(), 1e-3, 1e-3) == 0.0
    assert _close(ent, entr.detach(), 1e-3, 1e-3) == 0.0
    _, _, lse, ez = lce.lm_head_forward(hd.detach(), wd.detach(), lab.to(dev), T)
    _check_grads(hd, wd, h, w, lab, T, dlp, dent, hr, wr, lse, ez, f"M={M} V={V} split={cols}")


def test_dlogits_range_equals_whole_vocabulary_columns(dev, monkeypatch):
    """The per-split kernel reproduces the whole-vocabulary logits gradient's
    columns bit for bit (same 256-column tiles, same k order), labels mapped
    into the split, for splits that start on any 256-column tile."""
    monkeypatch.setattr(lce, "DLOGITS_GEMM", "fused")
    M, H, V, T = 200, 96, 1300, 0.9
    h, w, lab = _inputs(M, H, V, seed=21)
    lab[:6] = torch.tensor([0, 255, 256, 511, 512, V - 1])
    hd, wd, labd = h.to(dev), w.to(dev), lab.to(dev)
    _, _, lse, ez = lce.lm_head_forward(hd, wd, labd, T)
    g = torch.Generator().manual_seed(3)
    dlp = torch.randn(M, generator=g).to(dev)
    dent = torch.randn(M, generator=g).to(dev)
    full = lce.lm_head_dlogits(hd, wd, labd, T, lse, ez, dlp, dent)
    for v0, n in ((0, 256), (256, 256), (512, 768), (1280, 20), (768, 532)):
        dz = torch.full((M, n + 8), 7.0, dtype=torch.bfloat16, device=dev)
        _capi.call("af3_lm_head_dlogits_range", hd.data_ptr(), hd.stride(0), wd.data_ptr(), wd.stride(0), M, v0, n,
                   H, labd.data_ptr(), T, lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), 1, 1.0, dent.data_ptr(),
                   dz.data_ptr(), dz.stride(0), _capi.stream_of(dev))
        torch.cuda.synchronize()
        assert torch.equal(dz[:, :n].view(torch.int16), full[:, v0:v0 + n].view(torch.int16)), (v0, n)
        assert (dz[:, n:] == 7.0).all(), "columns past the split untouched"


@pytest.mark.parametrize("mode,chunk", MODES)
@pytest.mark.parametrize("reduction", ["sum", "mean"])
def test_reductions(dev, monkeypatch, reduction, mode, chunk):
    M, H, V = 200, 64, 700
    h, w, lab = _inputs(M, H, V, seed=9)
    _split(monkeypatch, M, 256)
    _mode(monkeypatch, mode, M, chunk)
    hd = h.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    lp, ent = linear_cross_entropy(hd, wd, lab.to(dev), 1.0, reduction)
    assert lp.dim() == 0 and ent.shape == (M,)
    lp.backward()
    hr = h.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    lpr, _ = lmhead.lm_head(hr, wr, lab, 1.0)
    red = lpr.sum() if reduction == "sum" else lpr.mean()
    red.backward()
    assert abs(lp.item() - red.item()) <= 1e-3 * max(1.0, abs(red.item()))
    for got, ref in ((hd.grad, hr.grad), (wd.grad, wr.grad)):
        check_close(got, ref, rtol=2e-2, atol=1e-2 * float(ref.abs().max()), what=f"{reduction} gradients")


@pytest.mark.parametrize("mode,chunk", [("library/library", 4096), ("library/fused", 0), ("fused/fused", 0)])
def test_full_vocabulary(dev, monkeypatch, mode, chunk):
    """Forward and backward over the whole gpt-oss vocabulary, the backward in
    22 splits of 9472 columns (the last one ragged); library chunks of 4096
    columns (forward: 50, the last one ragged; backward: three per split, the
    third ragged)."""
    M, H, V = 96, 256, 201088
    h, w, lab = _inputs(M, H, V, seed=4, scale=0.1)
    lab[:3] = torch.tensor([9471, 9472, V - 1])
    _split(monkeypatch, M, 9472)
    _mode(monkeypatch, mode, M, chunk)
    print(f"lm_head full vocabulary {mode}", flush=True)
    hd = h.to(dev).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    lp, ent = linear_cross_entropy(hd, wd, lab.to(dev), 1.0, "none")
    g = torch.Generator().manual_seed(5)
    dlp = torch.randn(M, generator=g)
    dent = torch.randn(M, generator=g)
    (lp * dlp.to(dev)).sum().add((ent * dent.to(dev)).sum()).backward()
    torch.cuda.synchronize()
    hr = h.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    lpr, entr = lmhead.lm_head(hr, wr, lab, 1.0)
    ((lpr * dlp.double()).sum() + (entr * dent.double()).sum()).backward()
    assert _close(lp, lpr.detach(), 2e-3, 1e-3) == 0.0
    assert _close(ent, entr.detach(), 2e-3, 1e-3) == 0.0
    _, _, lse, ez = lce.lm_head_forward(hd.detach(), wd.detach(), lab.to(dev), 1.0)
    _check_grads(hd, wd, h, w, lab, 1.0, dlp, dent, hr, wr, lse, ez, "full vocabulary")


def test_library_statistics_and_gradient_kernels_on_given_logits(dev):
    """af3_lm_head_chunk_stats / _reduce / _dz_chunk on fp32 logits given
    directly (no GEMM): per-row statistics over chunks that split the
    vocabulary raggedly, rows of odd length (no vector loads) and aligned ones,
    against float64 softmax statistics and the closed-form logits gradient."""
    M, V, T = 70, 1037, 0.8
    g = torch.Generator().manual_seed(11)
    z = torch.randn(M, V, generator=g) * 4
    lab = torch.randint(0, V, (M,), generator=g)
    lab[:4] = torch.tensor([-1, V, 0, V - 1])
    zd, labd = z.to(dev), lab.to(dev)
    stream = _capi.stream_of(dev)
    for ch in (1037, 256, 255):  # one chunk; 4 + a ragged one; odd widths (scalar loads)
        parts = (V + ch - 1) // ch
        ws = torch.zeros(parts * M * 4 + M, dtype=torch.float32, device=dev)
        zlab = ws.data_ptr() + parts * M * 16
        for j, v0 in enumerate(range(0, V, ch)):
            n = min(ch, V - v0)
            zc = zd[:, v0:v0 + n].contiguous()
            _capi.call("af3_lm_head_chunk_stats", zc.data_ptr(), n, M, v0, n, labd.data_ptr(), T,
                       ws.data_ptr() + j * M * 16, zlab, stream)
        outs = [torch.empty(M, dtype=torch.float32, device=dev) for _ in range(4)]
        _capi.call("af3_lm_head_reduce", ws.data_ptr(), M, parts, zlab, labd.data_ptr(), V,
                   *[o.data_ptr() for o in outs], stream)
        torch.cuda.synchronize()
        x = z.double() / T
        lse = torch.logsumexp(x, 1)
        p = torch.softmax(x, 1)
        ez = (p * x).sum(1)
        zl = torch.where((lab >= 0) & (lab < V), x.gather(1, lab.clamp(0, V - 1)[:, None])[:, 0], torch.zeros(M,
                         dtype=torch.float64))
        for got, ref, name in ((outs[0], zl - lse, "logprobs"), (outs[1], lse - ez, "entropy"), (outs[2], lse, "lse"),
                               (outs[3], ez, "ez")):
            err = float((got.cpu().double() - ref).abs().max())
            assert err <= 1e-5 * max(1.0, float(ref.abs().max())), (ch, name, err)
        # the gradient from the same statistics
        dlp = torch.randn(M, generator=g)
        dent = torch.randn(M, generator=g)
        dlpd, dentd = dlp.to(dev), dent.to(dev)   # held: the kernel reads them after the call returns
        dz = torch.full((M, V + 3), 9.0, dtype=torch.bfloat16, device=dev)
        for v0 in range(0, V, ch):
            n = min(ch, V - v0)
            zc = zd[:, v0:v0 + n].contiguous()
            _capi.call("af3_lm_head_dz_chunk", zc.data_ptr(), n, M, v0, n, labd.data_ptr(), T, outs[2].data_ptr(),
                       outs[3].data_ptr(), dlpd.data_ptr(), 1, 1.0, dentd.data_ptr(),
                       dz.data_ptr() + 2 * v0, dz.stride(0), stream)
        torch.cuda.synchronize()
        onehot = torch.zeros(M, V, dtype=torch.float64)
        ok = (lab >= 0) & (lab < V)
        onehot[ok.nonzero()[:, 0], lab[ok]] = 1.0
        ref = (dlp.double()[:, None] * (onehot - p) - dent.double()[:, None] * p * (x - ez[:, None])) / T
        got = dz[:, :V].float().cpu().double()
        assert float((got - ref).abs().max()) <= 2.0 ** -8 * float(ref.abs().max()) + 1e-6, ch
        assert (dz[:, V:] == 9.0).all()


def test_fused_kernels_with_rows_past_4_gib(dev):
    """Rows of hidden and weight more than 4 GiB past their bases (strided views
    of two 5 GiB buffers) make the fused GEMM kernel copy through 64-bit lane
    addresses; its log-probabilities, entropy, statistics and logits gradient
    (whole vocabulary and a split starting at column 256) equal, bit for bit,
    those of contiguous copies, whose copies take 32-bit offsets from scalar
    bases.  Both are checked against the float64 oracle as well."""
    M, H, V, T = 300, 128, 600, 0.9
    h, w, lab = _inputs(M, H, V, seed=5)
    lab[:2] = torch.tensor([V - 1, -100])
    ldh, ldw = (1 << 23) + 64, (1 << 22) + 64
    assert (M - 1) * ldh * 2 > 1 << 32 and (V - 1) * ldw * 2 > 1 << 32
    hb = torch.empty((M - 1) * ldh + H, dtype=torch.bfloat16, device=dev)
    wb = torch.empty((V - 1) * ldw + H, dtype=torch.bfloat16, device=dev)
    hs, ws_ = hb.as_strided((M, H), (ldh, 1)), wb.as_strided((V, H), (ldw, 1))
    hs.copy_(h.to(dev))
    ws_.copy_(w.to(dev))
    hc, wc, labd = h.to(dev), w.to(dev), lab.to(dev)
    stream = _capi.stream_of(dev)
    ws_n = int(_capi.load().af3_lm_head_workspace_bytes(M, V))
    g = torch.Generator().manual_seed(6)
    dlp, dent = torch.randn(M, generator=g).to(dev), torch.randn(M, generator=g).to(dev)
    res = []
    for hh, ww in ((hs, ws_), (hc, wc)):
        print(f"lm_head fused ldh={hh.stride(0)} ldw={ww.stride(0)}", flush=True)
        outs = [torch.empty(M, dtype=torch.float32, device=dev) for _ in range(4)]
        wsp = torch.empty(ws_n, dtype=torch.uint8, device=dev)
        _capi.call("af3_lm_head_logprobs", hh.data_ptr(), hh.stride(0), ww.data_ptr(), ww.stride(0), M, V, H,
                   labd.data_ptr(), T, *[o.data_ptr() for o in outs], wsp.data_ptr(), ws_n, stream)
        dz = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
        _capi.call("af3_lm_head_dlogits", hh.data_ptr(), hh.stride(0), ww.data_ptr(), ww.stride(0), M, V, H,
                   labd.data_ptr(), T, outs[2].data_ptr(), outs[3].data_ptr(), dlp.data_ptr(), 1, 1.0,
                   dent.data_ptr(), dz.data_ptr(), dz.stride(0), stream)
        dzs = torch.empty(M, V - 256, dtype=torch.bfloat16, device=dev)
        _capi.call("af3_lm_head_dlogits_range", hh.data_ptr(), hh.stride(0), ww.data_ptr(), ww.stride(0), M, 256,
                   V - 256, H, labd.data_ptr(), T, outs[2].data_ptr(), outs[3].data_ptr(), dlp.data_ptr(), 1, 1.0,
                   dent.data_ptr(), dzs.data_ptr(), dzs.stride(0), stream)
        torch.cuda.synchronize()
        res.append(outs + [dz, dzs])
    for a, b in zip(*res):
        assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a.view(torch.int32),
                           b.view(torch.int16) if b.dtype == torch.bfloat16 else b.view(torch.int32))
    assert torch.equal(res[0][5].view(torch.int16), res[0][4][:, 256:].view(torch.int16))
    lpr, entr = lmhead.lm_head(h.double(), w.double(), lab, T)
    assert _close(res[0][0], lpr, 1e-3, 1e-3) == 0.0
    assert _close(res[0][1], entr, 1e-3, 1e-3) == 0.0
