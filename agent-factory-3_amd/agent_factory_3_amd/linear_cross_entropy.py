"""Fused LM-head log-probabilities and entropy (``linear_cross_entropy``).

Same call as the reference's ``trainer/losses/linear_cross_entropy.py``
(``LinearCrossEntropy.apply(hidden, weight, labels, temperature, reduction,
dist_process_group)`` -> ``(logprobs, entropy)``, gradients for ``hidden``
and ``weight``), over gfx950 kernels instead of its Triton ones
(``trainer/losses/kernels.py``):

* forward: ``af3_lm_head_logprobs`` — a bf16 MFMA GEMM whose epilogue keeps
  only per-row softmax statistics of each 256-column vocabulary tile, then a
  per-row combine; the [tokens, vocab] logits are never written;
* backward: ``af3_lm_head_dlogits`` recomputes the logits tile by tile and
  writes the logits gradient (bf16), then ``d_hidden = dz @ W`` and
  ``d_weight = dz^T @ hidden`` run as plain GEMMs (hipBLASLt through torch).

``logprobs`` = z[label] - logsumexp(z), ``entropy`` = logsumexp(z) - E_p[z],
z = hidden @ W^T / temperature, fp32 (reduction "none"; "sum" / "mean"
return the scalar of the log-probabilities, as the reference does).
Differences: one rank only (``dist_process_group`` must be None: the
vocabulary-parallel form is not built), a label outside [0, V) counts as
z = 0 (the reference leaves that entry unwritten).
"""
from __future__ import annotations

import typing

import torch

from . import _capi

_REDUCTIONS = {"none": 0, "sum": 1, "mean": 2}


def _check(hidden, weight, labels):
    if not (hidden.is_cuda and weight.is_cuda and labels.is_cuda):
        raise RuntimeError("linear_cross_entropy runs on the GPU (the MI355X path has no CPU implementation)")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("hidden and weight must be bfloat16")
    if hidden.dim() != 2 or weight.dim() != 2 or labels.dim() != 1:
        raise ValueError("hidden [M, H], weight [V, H], labels [M] expected")
    if hidden.shape[0] != labels.shape[0] or hidden.shape[1] != weight.shape[1]:
        raise ValueError(f"shape mismatch: hidden {tuple(hidden.shape)}, weight {tuple(weight.shape)}, "
                         f"labels {tuple(labels.shape)}")
    if hidden.shape[1] % 32:
        raise ValueError(f"hidden_size must be divisible by 32, got {hidden.shape[1]}")


def lm_head_forward(hidden, weight, labels, temperature=1.0):
    """-> (logprobs [M], entropy [M], lse [M], ez [M]) in fp32."""
    _check(hidden, weight, labels)
    h = hidden.contiguous()
    w = weight.contiguous()
    lab = labels.to(torch.int64).contiguous()
    M, H = h.shape
    V = w.shape[0]
    dev = h.device
    outs = [torch.empty(M, dtype=torch.float32, device=dev) for _ in range(4)]
    ws_n = int(_capi.load().af3_lm_head_workspace_bytes(M, V))
    ws = torch.empty(max(ws_n, 16), dtype=torch.uint8, device=dev)
    _capi.call("af3_lm_head_logprobs", h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), M, V, H, lab.data_ptr(),
               float(temperature), *[o.data_ptr() for o in outs], ws.data_ptr(), ws_n, _capi.stream_of(dev))
    return tuple(outs)


def lm_head_dlogits(hidden, weight, labels, temperature, lse, ez, dlogprobs, dentropy, reduction=0):
    """The bf16 logits gradient [M, V] for upstream gradients of logprobs / entropy."""
    h, w = hidden.contiguous(), weight.contiguous()
    lab = labels.to(torch.int64).contiguous()
    M, H = h.shape
    V = w.shape[0]
    dev = h.device
    dlp = dlogprobs.float().contiguous()
    dent = (dentropy.float().contiguous() if dentropy is not None
            else torch.zeros(M, dtype=torch.float32, device=dev))
    stride = 1 if reduction == 0 else 0
    scale = 1.0 / M if reduction == 2 else 1.0
    dz = torch.empty(M, V, dtype=torch.bfloat16, device=dev)
    _capi.call("af3_lm_head_dlogits", h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), M, V, H, lab.data_ptr(),
               float(temperature), lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), stride, scale, dent.data_ptr(),
               dz.data_ptr(), dz.stride(0), _capi.stream_of(dev))
    return dz


class LinearCrossEntropy(torch.autograd.Function):
    """trainer/losses/linear_cross_entropy.py:LinearCrossEntropy on gfx950."""

    @staticmethod
    def forward(ctx, hidden: torch.Tensor, weight: torch.Tensor, labels: torch.Tensor,
                temperature: typing.Optional[float] = 1.0, reduction: typing.Optional[str] = "none",
                dist_process_group=None):
        if not isinstance(temperature, float):
            raise TypeError(f"temperature must be a float, but got {type(temperature)}")
        if not isinstance(reduction, str) or reduction.lower() not in _REDUCTIONS:
            raise ValueError(f"reduction must be one of {sorted(_REDUCTIONS)}")
        if dist_process_group is not None:
            raise NotImplementedError("vocabulary-parallel linear_cross_entropy is not built (single GPU)")
        shape = hidden.shape
        h = hidden.reshape(-1, shape[-1]) if hidden.dim() != 2 else hidden
        lab = labels.reshape(-1) if labels.dim() != 1 else labels
        logprobs, entropy, lse, ez = lm_head_forward(h, weight, lab, temperature)
        red = _REDUCTIONS[reduction.lower()]
        ctx.save_for_backward(h, weight, lab, lse, ez)
        ctx.shape, ctx.red, ctx.temperature = shape, red, temperature
        if red == 1:
            logprobs = logprobs.sum()
        elif red == 2:
            logprobs = logprobs.mean()
        return logprobs, entropy

    @staticmethod
    def backward(ctx, dlogprobs, dentropy):
        h, w, lab, lse, ez = ctx.saved_tensors
        M = h.shape[0]
        if dlogprobs is None:
            dlogprobs = torch.zeros(M if ctx.red == 0 else (), dtype=torch.float32, device=h.device)
        dlp = dlogprobs.reshape(-1) if ctx.red == 0 else dlogprobs.reshape(1)
        dz = lm_head_dlogits(h, w, lab, ctx.temperature, lse, ez, dlp, dentropy, ctx.red)
        d_hidden = d_weight = None
        if ctx.needs_input_grad[0]:
            d_hidden = torch.mm(dz, w).view(ctx.shape)
        if ctx.needs_input_grad[1]:
            d_weight = torch.mm(dz.t(), h)
        return d_hidden, d_weight, None, None, None, None


linear_cross_entropy = LinearCrossEntropy.apply
