"""Fused LM-head log-probabilities and entropy (``linear_cross_entropy``).

Same call as the reference's ``trainer/losses/linear_cross_entropy.py``
(``LinearCrossEntropy.apply(hidden, weight, labels, temperature, reduction,
dist_process_group)`` -> ``(logprobs, entropy)``, gradients for ``hidden``
and ``weight``), over gfx950 kernels instead of its Triton ones
(``trainer/losses/kernels.py``):

* forward (``LOGITS_GEMM = "library"``, the default): per vocabulary chunk
  of at most ``CHUNK_BYTES`` of fp32 logits ([tokens, chunk]), the logits
  from a plain GEMM with fp32 output (hipBLASLt through torch), then
  ``af3_lm_head_chunk_stats`` (per-row softmax statistics of the chunk and
  the label logit), and ``af3_lm_head_reduce`` over the chunks; at the
  default 128 MiB a chunk stays in the 256 MB Infinity Cache between the
  GEMM's write and the statistics' read.  ``LOGITS_GEMM = "fused"``:
  ``af3_lm_head_logprobs``, a bf16 MFMA GEMM whose epilogue keeps only the
  per-row statistics of each 256-column vocabulary tile (the logits are
  never written), then the same combine;
* backward: the vocabulary is cut into splits of at most ``SPLIT_BYTES`` of
  bf16 gradient ([tokens, split]); per split the logits are recomputed
  (``DLOGITS_GEMM = "fused"``, the default: ``af3_lm_head_dlogits_range``,
  tile by tile; "library": the fp32 GEMM per chunk and
  ``af3_lm_head_dz_chunk``) into that split's logits gradient dz (bf16), then ``d_hidden += dz @ W[split]`` (fp32 accumulation across the
  splits, one bf16 rounding at the end) and ``d_weight[split] = dz^T @ hidden``
  run as plain GEMMs (hipBLASLt through torch).  This is the reference's
  default backward (``BackwardEnum._Split_Dlogits_N``, kernels.py:1528-1585);
  the [tokens, vocab] gradient is never formed, and at the default 128 MiB a
  split stays in the 256 MB Infinity Cache between its write and the GEMMs'
  reads.

``logprobs`` = z[label] - logsumexp(z), ``entropy`` = logsumexp(z) - E_p[z],
z = hidden @ W^T / temperature, fp32 (reduction "none"; "sum" / "mean"
return the scalar of the log-probabilities, as the reference does).
Differences: one rank only (``dist_process_group`` must be None: the
vocabulary-parallel form is not built), a label outside [0, V) counts as
z = 0 (the reference leaves that entry unwritten), and d_hidden sums the
splits in fp32 (the reference adds each split's bf16 product into a bf16
d_hidden, kernels.py:1575-1582).
"""
from __future__ import annotations

import typing

import torch

from . import _capi

_REDUCTIONS = {"none": 0, "sum": 1, "mean": 2}

# bytes of bf16 logits gradient one vocabulary split of the backward may hold
SPLIT_BYTES = 128 << 20
# "library": logits of a vocabulary chunk from a plain fp32-output GEMM, then
# the statistics / gradient kernels; "fused": the GEMM kernel with the
# statistics (forward) or the gradient (backward) in its epilogue.  Forward
# and backward choose separately (measured at 8192 tokens x 201,088 entries:
# forward 9.0 ms library against 10.9 fused; the backward's logits gradient
# 9.2 ms fused against 9.9 library).
LOGITS_GEMM = "library"
DLOGITS_GEMM = "fused"
# bytes of fp32 logits one chunk of the library path may hold
CHUNK_BYTES = 128 << 20


def logits_chunk(M: int, V: int) -> int:
    """Vocabulary columns per chunk of the library path: [M, chunk] fp32
    within CHUNK_BYTES, a multiple of 256."""
    n = max(256, (CHUNK_BYTES // (4 * max(M, 1))) // 256 * 256)
    return min(n, V)


def vocab_split(M: int, V: int) -> int:
    """Vocabulary columns per backward split: the [M, split] bf16 gradient
    within SPLIT_BYTES, a multiple of the kernel's 256-column tile."""
    n = max(256, (SPLIT_BYTES // (2 * max(M, 1))) // 256 * 256)
    return min(n, V)


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
    if M > 0 and LOGITS_GEMM == "library":
        stream = _capi.stream_of(dev)
        ch = logits_chunk(M, V)
        zbuf = torch.empty(M * ch, dtype=torch.float32, device=dev)
        n_parts = (V + ch - 1) // ch
        zlab = ws.data_ptr() + n_parts * M * 16      # the label logits after the partials
        for j, v0 in enumerate(range(0, V, ch)):
            n = min(ch, V - v0)
            zc = zbuf[:M * n].view(M, n)
            torch.mm(h, w[v0:v0 + n].t(), out_dtype=torch.float32, out=zc)
            _capi.call("af3_lm_head_chunk_stats", zc.data_ptr(), n, M, v0, n, lab.data_ptr(), float(temperature),
                       ws.data_ptr() + j * M * 16, zlab, stream)
        _capi.call("af3_lm_head_reduce", ws.data_ptr(), M, n_parts, zlab, lab.data_ptr(), V,
                   *[o.data_ptr() for o in outs], stream)
        return tuple(outs)
    _capi.call("af3_lm_head_logprobs", h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), M, V, H, lab.data_ptr(),
               float(temperature), *[o.data_ptr() for o in outs], ws.data_ptr(), ws_n, _capi.stream_of(dev))
    return tuple(outs)


def lm_head_dlogits(hidden, weight, labels, temperature, lse, ez, dlogprobs, dentropy, reduction=0):
    """The bf16 logits gradient [M, V] for upstream gradients of logprobs /
    entropy: the values the backward forms split by split (library mode: from
    the same GEMM calls)."""
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
    if M > 0 and DLOGITS_GEMM == "library":
        # the logits of the backward's splits and chunks (the same GEMM calls)
        split = vocab_split(M, V)
        ch = min(logits_chunk(M, V), split)
        zbuf = torch.empty(M * ch, dtype=torch.float32, device=dev)
        stream = _capi.stream_of(dev)
        for v0 in range(0, V, split):
            n = min(split, V - v0)
            for c0 in range(0, n, ch):
                nc = min(ch, n - c0)
                zc = zbuf[:M * nc].view(M, nc)
                torch.mm(h, w[v0 + c0:v0 + c0 + nc].t(), out_dtype=torch.float32, out=zc)
                _capi.call("af3_lm_head_dz_chunk", zc.data_ptr(), nc, M, v0 + c0, nc, lab.data_ptr(),
                           float(temperature), lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), stride, scale,
                           dent.data_ptr(), dz.data_ptr() + 2 * (v0 + c0), dz.stride(0), stream)
        return dz
    _capi.call("af3_lm_head_dlogits", h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), M, V, H, lab.data_ptr(),
               float(temperature), lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), stride, scale, dent.data_ptr(),
               dz.data_ptr(), dz.stride(0), _capi.stream_of(dev))
    return dz


def lm_head_backward(hidden, weight, labels, temperature, lse, ez, dlogprobs, dentropy, reduction=0,
                     need_hidden=True, need_weight=True):
    """-> (d_hidden, d_weight) in bf16 (None where not needed), the logits
    gradient formed one vocabulary split at a time."""
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
    d_hidden = torch.zeros(M, H, dtype=torch.float32, device=dev) if need_hidden else None
    d_weight = torch.empty(V, H, dtype=torch.bfloat16, device=dev) if need_weight else None
    if M == 0 or not (need_hidden or need_weight):
        return (d_hidden.to(torch.bfloat16) if need_hidden else None), (d_weight.zero_() if need_weight else None)
    split = vocab_split(M, V)
    dz = torch.empty(M, split, dtype=torch.bfloat16, device=dev)
    stream = _capi.stream_of(dev)
    library = DLOGITS_GEMM == "library"
    if library:
        ch = min(logits_chunk(M, V), split)
        zbuf = torch.empty(M * ch, dtype=torch.float32, device=dev)
    for v0 in range(0, V, split):
        n = min(split, V - v0)
        dzc = dz[:, :n]
        if library:
            for c0 in range(0, n, ch):
                nc = min(ch, n - c0)
                zc = zbuf[:M * nc].view(M, nc)
                torch.mm(h, w[v0 + c0:v0 + c0 + nc].t(), out_dtype=torch.float32, out=zc)
                _capi.call("af3_lm_head_dz_chunk", zc.data_ptr(), nc, M, v0 + c0, nc, lab.data_ptr(),
                           float(temperature), lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), stride, scale,
                           dent.data_ptr(), dzc.data_ptr() + 2 * c0, dz.stride(0), stream)
        else:
            _capi.call("af3_lm_head_dlogits_range", h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0), M, v0, n,
                       H, lab.data_ptr(), float(temperature), lse.data_ptr(), ez.data_ptr(), dlp.data_ptr(), stride,
                       scale, dent.data_ptr(), dzc.data_ptr(), dz.stride(0), stream)
        if need_hidden:
            torch.addmm(d_hidden, dzc, w[v0:v0 + n], out_dtype=torch.float32, out=d_hidden)
        if need_weight:
            torch.mm(dzc.t(), h, out=d_weight[v0:v0 + n])
    return (d_hidden.to(torch.bfloat16) if need_hidden else None), d_weight


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
        d_hidden, d_weight = lm_head_backward(h, w, lab, ctx.temperature, lse, ez, dlp, dentropy, ctx.red,
                                              ctx.needs_input_grad[0], ctx.needs_input_grad[1])
        if d_hidden is not None:
            d_hidden = d_hidden.view(ctx.shape)
        return d_hidden, d_weight, None, None, None, None


linear_cross_entropy = LinearCrossEntropy.apply
