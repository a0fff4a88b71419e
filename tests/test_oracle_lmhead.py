"""Pins oracle/lmhead.py (CPU): loop restatement, normalisation, bounds, gradient."""
import math

import torch

from oracle import lmhead


def _inputs(M=5, H=8, V=11, seed=0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, H, generator=g, dtype=torch.float64), torch.randn(V, H, generator=g, dtype=torch.float64),
            torch.randint(0, V, (M,), generator=g))


def test_matches_a_loop_restatement():
    h, w, lab = _inputs()
    lab[2] = -100                                  # out of range: z_label = 0
    T = 0.7
    lp, ent = lmhead.lm_head(h, w, lab, T)
    for m in range(h.shape[0]):
        z = [sum(h[m, k].item() * w[v, k].item() for k in range(h.shape[1])) / T for v in range(w.shape[0])]
        mx = max(z)
        s = sum(math.exp(x - mx) for x in z)
        lse = mx + math.log(s)
        ez = sum(math.exp(x - mx) * x for x in z) / s
        zl = z[lab[m]] if 0 <= lab[m] < len(z) else 0.0
        assert abs(lp[m].item() - (zl - lse)) < 1e-12
        assert abs(ent[m].item() - (lse - ez)) < 1e-12


def test_normalisation_and_entropy_bounds():
    h, w, _ = _inputs(M=3, V=7, seed=1)
    V = w.shape[0]
    tot = torch.zeros(3, dtype=torch.float64)
    for v in range(V):
        lp, ent = lmhead.lm_head(h, w, torch.full((3,), v), 1.3)
        tot += lp.exp()
    assert torch.allclose(tot, torch.ones(3, dtype=torch.float64), atol=1e-12)
    assert bool((ent >= 0).all()) and bool((ent <= math.log(V) + 1e-12).all())


def test_closed_form_gradient_equals_autograd():
    h, w, lab = _inputs(M=6, H=5, V=9, seed=2)
    T = 0.8
    g = torch.Generator().manual_seed(3)
    dlp = torch.randn(6, generator=g, dtype=torch.float64)
    dent = torch.randn(6, generator=g, dtype=torch.float64)
    hh = h.clone().requires_grad_(True)
    ww = w.clone().requires_grad_(True)
    lp, ent = lmhead.lm_head(hh, ww, lab, T)
    ((lp * dlp).sum() + (ent * dent).sum()).backward()
    dz = lmhead.dlogits(h, w, lab, T, dlp, dent)
    assert torch.allclose(hh.grad, dz @ w, atol=1e-12)
    assert torch.allclose(ww.grad, dz.t() @ h, atol=1e-12)
