"""gpt-oss clamped SwiGLU restated on the CPU (test infrastructure only).

Forward kernels.py:427-448, backward kernels.py:529-553 (strict masks
``g < limit`` and ``-limit < u < limit``).  Computed in float64 from the bf16
inputs; outputs are rounded to bf16 by the caller when comparing.
"""
from __future__ import annotations

import numpy as np
import torch

ALPHA = 1.702  # quantization.py:485
LIMIT = 7.0    # quantization.py:486 (config.swiglu_limit default)


def _split(gate_up: torch.Tensor):
    x = gate_up.to(torch.float64)
    return x[..., 0::2], x[..., 1::2]


def forward(gate_up: torch.Tensor, alpha: float = ALPHA, limit: float = LIMIT):
    """-> (out, g, u) float64; out = g*sigmoid(alpha*g)*(u+1) with g=min(G,limit), u=clamp(U)."""
    graw, uraw = _split(gate_up)
    g = torch.clamp(graw, max=limit)
    u = torch.clamp(uraw, -limit, limit)
    s = 1.0 / (1.0 + torch.exp(-alpha * g))
    return g * s * (u + 1.0), g, u


def backward(grad_out: torch.Tensor, g: torch.Tensor, u: torch.Tensor, alpha: float = ALPHA,
             limit: float = LIMIT) -> torch.Tensor:
    """-> interleaved [.., 2N] float64 gradient of the raw input (kernels.py:539-553)."""
    d = grad_out.to(torch.float64)
    g = g.to(torch.float64)
    u = u.to(torch.float64)
    s = 1.0 / (1.0 + torch.exp(-alpha * g))
    dg = d * (u + 1.0) * s * (1.0 + alpha * g * (1.0 - s))
    dg = torch.where(g < limit, dg, torch.zeros_like(dg))
    du = d * g * s
    du = torch.where((u > -limit) & (u < limit), du, torch.zeros_like(du))
    out = torch.empty(*d.shape[:-1], 2 * d.shape[-1], dtype=torch.float64)
    out[..., 0::2] = dg
    out[..., 1::2] = du
    return out


def backward_from_raw(grad_out: torch.Tensor, gate_up: torch.Tensor, alpha: float = ALPHA,
                      limit: float = LIMIT) -> torch.Tensor:
    _, g, u = forward(gate_up, alpha, limit)
    return backward(grad_out, g, u, alpha, limit)


def autograd_reference(gate_up: torch.Tensor, grad_out: torch.Tensor, alpha: float = ALPHA,
                       limit: float = LIMIT):
    """float64 autograd of the forward expression with the strict clamp masks applied.

    torch.clamp's autograd passes gradient at the boundary (x == limit); the
    reference kernel does not, so the masks are applied explicitly here.
    """
    x = gate_up.to(torch.float64).clone().requires_grad_(True)
    graw, uraw = x[..., 0::2], x[..., 1::2]
    g_mask = (graw < limit).to(torch.float64)
    u_mask = ((uraw > -limit) & (uraw < limit)).to(torch.float64)
    # straight-through of the identity where the mask is open, constant elsewhere
    g = graw * g_mask + (torch.clamp(graw, max=limit) * (1 - g_mask)).detach()
    u = uraw * u_mask + (torch.clamp(uraw, -limit, limit) * (1 - u_mask)).detach()
    out = g * torch.sigmoid(alpha * g) * (u + 1.0)
    out.backward(grad_out.to(torch.float64))
    return out.detach(), x.grad


def bf16_round(x: torch.Tensor) -> torch.Tensor:
    return x.to(torch.float32).to(torch.bfloat16)


def numpy_bf16_bits(x: torch.Tensor) -> np.ndarray:
    return x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
