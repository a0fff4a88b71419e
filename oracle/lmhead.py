"""LM-head log-probabilities and entropy restated on the CPU (test infrastructure only).

The fused linear cross entropy of the reference's trainer
(trainer/losses/kernels.py: mainloop 157-292 and epilogue 296-385 forward,
829-839 logits gradient; wrapper trainer/losses/linear_cross_entropy.py),
written from its definition in float64:

    z = hidden @ W^T / temperature
    logprobs = z[label] - logsumexp(z),  entropy = logsumexp(z) - sum softmax(z) * z

with a label outside [0, V) counting as z = 0.  ``dlogits`` is the closed-form
gradient the backward kernel evaluates; ``lm_head`` is differentiable (torch
autograd gives the reference gradients of hidden and W).

Pinning (tests/test_oracle_lmhead.py): a pure-Python loop restatement on tiny
inputs, softmax normalisation (sum over labels of exp(logprob) = 1), entropy
bounds 0 <= H <= log V, and autograd of ``lm_head`` against ``dlogits``.
"""
from __future__ import annotations

import torch

F64 = torch.float64


def lm_head(hidden, weight, labels, temperature=1.0):
    """-> (logprobs [M], entropy [M]) in float64 (differentiable)."""
    h = hidden if hidden.dtype == F64 else hidden.to(F64)
    w = weight if weight.dtype == F64 else weight.to(F64)
    z = h @ w.t() / temperature
    lse = torch.logsumexp(z, dim=-1)
    p = torch.softmax(z, dim=-1)
    V = z.shape[1]
    lab = labels.long()
    ok = (lab >= 0) & (lab < V)
    zl = torch.where(ok, z.gather(1, lab.clamp(0, V - 1)[:, None])[:, 0], torch.zeros_like(lse))
    return zl - lse, lse - (p * z).sum(-1)


def dlogits(hidden, weight, labels, temperature, dlogprobs, dentropy):
    """Closed-form gradient w.r.t. hidden @ W^T (before the temperature division):
    (dlp (onehot - p) - dent p (z - E_p[z])) / temperature, float64."""
    z = hidden.to(F64) @ weight.to(F64).t() / temperature
    p = torch.softmax(z, dim=-1)
    ez = (p * z).sum(-1, keepdim=True)
    V = z.shape[1]
    lab = labels.long()
    onehot = torch.zeros_like(z)
    ok = (lab >= 0) & (lab < V)
    onehot[ok.nonzero()[:, 0], lab[ok]] = 1.0
    return (dlogprobs.to(F64)[:, None] * (onehot - p) - dentropy.to(F64)[:, None] * p * (z - ez)) / temperature
