"""Pins oracle.swiglu (CPU): closed form vs float64 autograd, strict masks, special points."""
import torch

from oracle import swiglu


def _inputs(n=4096, seed=0):
    g = torch.Generator().manual_seed(seed)
    gu = (torch.randn(8, 2 * n, generator=g) * 3).to(torch.bfloat16)
    # plant the boundary points the strict masks distinguish
    gu[0, 0:8:2] = torch.tensor([7.0, -7.0, 6.96875, 100.0]).to(torch.bfloat16)
    gu[0, 1:9:2] = torch.tensor([7.0, -7.0, 0.0, -100.0]).to(torch.bfloat16)
    dO = torch.randn(8, n, generator=g).to(torch.bfloat16)
    return gu, dO


def test_forward_matches_autograd_reference():
    gu, dO = _inputs()
    out, _, _ = swiglu.forward(gu)
    ref, _ = swiglu.autograd_reference(gu, dO)
    assert torch.allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_backward_matches_autograd_reference():
    gu, dO = _inputs()
    ref_out, ref_grad = swiglu.autograd_reference(gu, dO)
    grad = swiglu.backward_from_raw(dO, gu)
    assert torch.allclose(grad, ref_grad, rtol=1e-10, atol=1e-12)


def test_strict_masks_at_limit():
    gu, dO = _inputs()
    grad = swiglu.backward_from_raw(dO, gu)
    assert grad[0, 0] == 0.0          # gate == 7 -> no gradient (strict g < limit)
    assert grad[0, 1] == 0.0          # up == 7 -> no gradient
    assert grad[0, 3] == 0.0          # up == -7 -> no gradient
    assert grad[0, 4] != 0.0          # gate just below the limit passes


def test_saturated_sigmoid_and_zero():
    gu = torch.tensor([[-100.0, 3.0, 0.0, 5.0]], dtype=torch.bfloat16)
    out, g, u = swiglu.forward(gu)
    assert abs(float(out[0, 0])) < 1e-60 and float(out[0, 1]) == 0.0
