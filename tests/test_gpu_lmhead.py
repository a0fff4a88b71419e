"""Fused LM-head log-probabilities / entropy (linear_cross_entropy) on the GPU
against oracle/lmhead.py on the same bf16 inputs: forward values (the GEMM
accumulates in fp32, so only summation order separates it from float64),
gradients of hidden and weight through the bf16 logits gradient, the three
reductions, out-of-range labels, partial row / vocabulary tiles and the full
gpt-oss vocabulary (201,088)."""
import pytest
import torch

from agent_factory_3_amd.linear_cross_entropy import linear_cross_entropy
from oracle import lmhead

pytestmark = pytest.mark.gpu


def _inputs(M, H, V, seed, scale=0.05):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(M, H, generator=g).to(torch.bfloat16)
    w = (torch.randn(V, H, generator=g) * scale).to(torch.bfloat16)
    lab = torch.randint(0, V, (M,), generator=g)
    return h, w, lab


def _close(got, ref, atol, rtol):
    got = got.detach().float().cpu().double()
    return float(((got - ref).abs() > atol + rtol * ref.abs()).float().mean())


@pytest.mark.parametrize("M,H,V,T", [(300, 128, 1000, 1.0), (257, 96, 513, 0.7), (64, 64, 256, 1.3)])
def test_forward_and_backward(dev, M, H, V, T):
    h, w, lab = _inputs(M, H, V, seed=M + V)
    lab[5] = -100
    print(f"lm_head M={M} H={H} V={V} T={T}", flush=True)
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
    for got, ref in ((hd.grad, hr.grad), (wd.grad, wr.grad)):
        scale = float(ref.abs().max())
        assert _close(got, ref, 1e-2 * scale, 2e-2) < 1e-2
        d = (got.float().cpu().double() - ref).norm() / ref.norm()
        assert float(d) < 1e-2


@pytest.mark.parametrize("reduction", ["sum", "mean"])
def test_reductions(dev, reduction):
    M, H, V = 200, 64, 700
    h, w, lab = _inputs(M, H, V, seed=9)
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
    d = (hd.grad.float().cpu().double() - hr.grad).norm() / hr.grad.norm()
    assert float(d) < 1e-2


def test_full_vocabulary(dev):
    M, H, V = 96, 256, 201088
    h, w, lab = _inputs(M, H, V, seed=4, scale=0.1)
    print("lm_head full vocabulary", flush=True)
    lp, ent = linear_cross_entropy(h.to(dev), w.to(dev), lab.to(dev), 1.0, "none")
    torch.cuda.synchronize()
    lpr, entr = lmhead.lm_head(h, w, lab, 1.0)
    assert _close(lp, lpr, 2e-3, 1e-3) == 0.0
    assert _close(ent, entr, 2e-3, 1e-3) == 0.0
