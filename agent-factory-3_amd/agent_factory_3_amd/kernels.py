"""Python launchers of the gfx950 dequant and SwiGLU kernels.

Mirrors the bf16-path functions of the reference's
``src/agent_factory_3/models/gpt_oss/kernels.py`` (same arguments, shapes,
dtypes and assertion behaviour), launching hand-written HIP kernels through
the C ABI on the caller's current stream:

=======================================  =====================================
this module                              reference (kernels.py)
=======================================  =====================================
``mxfp4_to_bf16_hip``                    ``mxfp4_to_bf16_triton`` 206-235
``swiglu_forward``                       ``_swiglu_forward_triton`` 451-490
``swiglu_backward``                      ``_swiglu_backward`` 556-582
``swiglu_backward_raw``                  (new: backward from the raw input)
``mxfp4_to_fp8_e5m2``                    ``mxfp4_to_fp8_e5m2_triton`` 20-108
``mxfp4_to_fp8_e5m2_colmajor``           ``mxfp4_to_fp8_e5m2_colmajor`` 238-312
``dynamic_quantize_per_token``           ``dynamic_quantize_per_token`` 319-388
``mxfp4_lora_merge``                     (new: expert-LoRA merge for weight sync,
                                         arithmetic of model_trainer.py:710-712)
=======================================  =====================================

The reference's names are provided as aliases so code that imports them keeps
working; nothing here uses Triton.
"""
from __future__ import annotations

import torch

from . import _capi


def _need_cuda(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (the MI355X path has no CPU implementation)")


def mxfp4_to_bf16_hip(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MXFP4 -> bf16, bit-exact with kernels.py:120-203.

    Args:
        blocks: [..., G, 16] uint8, two e2m1 values per byte (low nibble first)
        scales: [..., G] uint8 e8m0 block scales
    Returns:
        [..., G*32] bfloat16
    """
    _need_cuda(blocks, "blocks")
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("blocks and scales must be uint8")
    if blocks.shape[-1] != 16 or tuple(blocks.shape[:-1]) != tuple(scales.shape):
        raise ValueError(f"shape mismatch: blocks {tuple(blocks.shape)} scales {tuple(scales.shape)}")
    prefix = blocks.shape[:-2]
    G = blocks.shape[-2]
    n_groups = blocks.numel() // 16
    blocks_flat = blocks.reshape(n_groups, 16).contiguous()
    scales_flat = scales.reshape(n_groups).contiguous()
    if blocks_flat.data_ptr() % 16:
        blocks_flat = blocks_flat.clone()
    out = torch.empty(n_groups, 32, dtype=torch.bfloat16, device=blocks.device)
    _capi.call("af3_mxfp4_to_bf16", blocks_flat.data_ptr(), scales_flat.data_ptr(), out.data_ptr(),
               n_groups, _capi.stream_of(blocks.device))
    return out.reshape(*prefix, G * 32)


def _rows2d(t: torch.Tensor) -> torch.Tensor:
    """View as [M, last] keeping the row stride when possible."""
    if t.dim() == 2:
        return t
    try:
        return t.view(-1, t.shape[-1])
    except RuntimeError:
        return t.reshape(-1, t.shape[-1]).contiguous()


def swiglu_forward(gate_up_raw: torch.Tensor, alpha: float, limit: float, save_for_bwd: bool = False):
    """Clamped SwiGLU forward (kernels.py:451-490).

    Args:
        gate_up_raw: [..., 2*N] interleaved gate/up, bf16, stride(-1) == 1
        save_for_bwd: also return the clamped gate and up ([..., N] each)
    """
    assert gate_up_raw.shape[-1] % 2 == 0
    assert gate_up_raw.stride(-1) == 1
    _need_cuda(gate_up_raw, "gate_up_raw")
    if gate_up_raw.dtype != torch.bfloat16:
        raise TypeError("gate_up_raw must be bfloat16")
    prefix = gate_up_raw.shape[:-1]
    N = gate_up_raw.shape[-1] // 2
    x = _rows2d(gate_up_raw)
    M = x.shape[0]
    dev = gate_up_raw.device
    out = torch.empty(*prefix, N, dtype=torch.bfloat16, device=dev)
    g = u = None
    if save_for_bwd:
        g = torch.empty(*prefix, N, dtype=torch.bfloat16, device=dev)
        u = torch.empty(*prefix, N, dtype=torch.bfloat16, device=dev)
    _capi.call("af3_swiglu_fwd", x.data_ptr(), x.stride(0) if M > 1 else 2 * N, out.data_ptr(), N,
               _capi.ptr(g), _capi.ptr(u), N, M, N, float(alpha), float(limit), _capi.stream_of(dev))
    if save_for_bwd:
        return out, g, u
    return out


def swiglu_backward(grad_output: torch.Tensor, gate: torch.Tensor, up: torch.Tensor, alpha: float,
                    limit: float) -> torch.Tensor:
    """Clamped SwiGLU backward from saved clamped gate/up (kernels.py:556-582).

    Returns the interleaved [..., 2*N] gradient of the raw gate_up input.
    """
    assert grad_output.stride(-1) == 1
    _need_cuda(grad_output, "grad_output")
    prefix = grad_output.shape[:-1]
    N = grad_output.shape[-1]
    dO = _rows2d(grad_output.to(torch.bfloat16))
    g = _rows2d(gate.contiguous())
    u = _rows2d(up.contiguous())
    M = dO.shape[0]
    out = torch.empty(*prefix, 2 * N, dtype=torch.bfloat16, device=grad_output.device)
    _capi.call("af3_swiglu_bwd", dO.data_ptr(), dO.stride(0) if M > 1 else N, g.data_ptr(), u.data_ptr(), N,
               out.data_ptr(), 2 * N, M, N, float(alpha), float(limit), _capi.stream_of(grad_output.device))
    return out


def swiglu_backward_raw(grad_output: torch.Tensor, gate_up_raw: torch.Tensor, alpha: float,
                        limit: float) -> torch.Tensor:
    """SwiGLU backward from the raw interleaved pre-activation (clamped inside)."""
    assert grad_output.stride(-1) == 1 and gate_up_raw.stride(-1) == 1
    _need_cuda(grad_output, "grad_output")
    prefix = grad_output.shape[:-1]
    N = grad_output.shape[-1]
    dO = _rows2d(grad_output.to(torch.bfloat16))
    x = _rows2d(gate_up_raw)
    M = dO.shape[0]
    out = torch.empty(*prefix, 2 * N, dtype=torch.bfloat16, device=grad_output.device)
    _capi.call("af3_swiglu_bwd_raw", dO.data_ptr(), dO.stride(0) if M > 1 else N, x.data_ptr(),
               x.stride(0) if M > 1 else 2 * N, out.data_ptr(), 2 * N, M, N, float(alpha), float(limit),
               _capi.stream_of(grad_output.device))
    return out


def mxfp4_to_fp8_e5m2(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MXFP4 -> fp8 E5M2 bits, row-major [..., G*32] (kernels.py:20-108 rule
    and uint16 packing, bit for bit)."""
    _need_cuda(blocks, "blocks")
    if blocks.dtype != torch.uint8 or scales.dtype != torch.uint8:
        raise TypeError("blocks and scales must be uint8")
    if blocks.shape[-1] != 16 or tuple(blocks.shape[:-1]) != tuple(scales.shape):
        raise ValueError(f"shape mismatch: blocks {tuple(blocks.shape)} scales {tuple(scales.shape)}")
    prefix, G = blocks.shape[:-2], blocks.shape[-2]
    n_groups = blocks.numel() // 16
    bf = blocks.reshape(n_groups, 16).contiguous()
    sf = scales.reshape(n_groups).contiguous()
    out = torch.empty(n_groups, 32, dtype=torch.uint8, device=blocks.device)
    _capi.call("af3_mxfp4_to_fp8_e5m2", bf.data_ptr(), sf.data_ptr(), out.data_ptr(), n_groups,
               _capi.stream_of(blocks.device))
    return out.reshape(*prefix, G * 32).view(torch.float8_e5m2)


def mxfp4_to_fp8_e5m2_colmajor(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """MXFP4 [E, N, G, 16] -> fp8 E5M2 [E, K, N] (N contiguous), K = 32 G
    (kernels.py:238-312, values truncated to a byte as its stores do)."""
    _need_cuda(blocks, "blocks")
    if blocks.dim() != 4 or blocks.shape[-1] != 16:
        raise ValueError(f"blocks must be [E, N, G, 16], got {tuple(blocks.shape)}")
    E, N, G, _ = blocks.shape
    if tuple(scales.shape) != (E, N, G):
        raise ValueError(f"scales must be [{E}, {N}, {G}], got {tuple(scales.shape)}")
    out = torch.empty(E, G * 32, N, dtype=torch.uint8, device=blocks.device)
    _capi.call("af3_mxfp4_to_fp8_e5m2_colmajor", blocks.contiguous().data_ptr(), scales.contiguous().data_ptr(),
               out.data_ptr(), E, N, G, _capi.stream_of(blocks.device))
    return out.view(torch.float8_e5m2)


def mxfp4_lora_merge(blocks: torch.Tensor, scales: torch.Tensor, lora_A: torch.Tensor, lora_B: torch.Tensor,
                     scaling: float, layout: str = "hf") -> torch.Tensor:
    """bf16 expert weights with the LoRA delta folded in:
    ``W'[e] = bf16(float(deq(W[e])) + scaling * (B[e] @ A[e]))`` in fp32.

    blocks [E, N, G, 16] u8, scales [E, N, G] u8, lora_A [E, r, 32 G] bf16,
    lora_B [E, N, r] bf16.  ``layout="hf"`` returns [E, K, N] (transformers'
    GptOssExperts parameter layout), ``"rows"`` [E, N, K].
    """
    _need_cuda(blocks, "blocks")
    if blocks.dim() != 4 or blocks.shape[-1] != 16:
        raise ValueError(f"blocks must be [E, N, G, 16], got {tuple(blocks.shape)}")
    E, N, G, _ = blocks.shape
    K = 32 * G
    r = lora_A.shape[1] if lora_A.dim() == 3 else -1
    if tuple(scales.shape) != (E, N, G):
        raise ValueError(f"scales must be [{E}, {N}, {G}], got {tuple(scales.shape)}")
    if tuple(lora_A.shape) != (E, r, K) or tuple(lora_B.shape) != (E, N, r):
        raise ValueError(f"lora_A must be [E, r, {K}] and lora_B [E, {N}, r], got "
                         f"{tuple(lora_A.shape)} / {tuple(lora_B.shape)}")
    if lora_A.dtype != torch.bfloat16 or lora_B.dtype != torch.bfloat16:
        raise TypeError("LoRA factors must be bfloat16")
    if layout not in ("hf", "rows"):
        raise ValueError("layout must be 'hf' ([E, K, N]) or 'rows' ([E, N, K])")
    shape = (E, K, N) if layout == "hf" else (E, N, K)
    out = torch.empty(shape, dtype=torch.bfloat16, device=blocks.device)
    a, b = lora_A.contiguous(), lora_B.contiguous()
    _capi.call("af3_mxfp4_lora_merge", blocks.contiguous().data_ptr(), scales.contiguous().data_ptr(),
               a.data_ptr(), b.data_ptr(), float(scaling), out.data_ptr(), E, N, K, r,
               1 if layout == "hf" else 0, _capi.stream_of(blocks.device))
    return out


def quantize_per_token_e4m3(x: torch.Tensor, with_bf16: bool = False):
    """Per-row fp8 E4M3FN codes of ``x`` [M, K] bf16 and fp32 scales [M]:
    scale = max(amax, 1e-12) / 448, codes = E4M3(x / scale) (round to nearest
    even, saturating).  ``with_bf16`` also returns the codes' values as bf16."""
    _need_cuda(x, "x")
    if x.dtype != torch.bfloat16 or x.dim() != 2:
        raise TypeError("x must be a 2-D bfloat16 tensor")
    M, K = x.shape
    Kp = (K + 7) // 8 * 8
    if not (x.stride(-1) == 1 and (x.stride(0) % 8 == 0 or M == 1) and x.data_ptr() % 16 == 0):
        xp = torch.empty(M, Kp, dtype=x.dtype, device=x.device)   # rows 16-byte aligned
        xp[:, :K] = x
        x = xp[:, :K]
    codes = torch.empty(M, Kp, dtype=torch.uint8, device=x.device)[:, :K]
    scale = torch.empty(M, dtype=torch.float32, device=x.device)
    vals = torch.empty(M, Kp, dtype=torch.bfloat16, device=x.device)[:, :K] if with_bf16 else None
    _capi.call("af3_quantize_per_token_e4m3", x.data_ptr(), x.stride(0) if M > 1 else Kp, M, K, codes.data_ptr(),
               Kp, scale.data_ptr(), _capi.ptr(vals), Kp, _capi.stream_of(x.device))
    codes = codes.view(torch.float8_e4m3fn)
    return (codes, scale, vals) if with_bf16 else (codes, scale)


def dynamic_quantize_per_token(x: torch.Tensor):
    """BF16 -> (fp8 E4M3FN [M, K], fp32 per-row scale [M]) (kernels.py:375-388)."""
    codes, scale = quantize_per_token_e4m3(x)
    return codes.contiguous() if codes.stride(0) != codes.shape[1] else codes, scale


# the reference's names (kernels.py), for code that imports them directly
mxfp4_to_bf16_triton = mxfp4_to_bf16_hip
mxfp4_to_fp8_e5m2_triton = mxfp4_to_fp8_e5m2
_swiglu_forward_triton = swiglu_forward
_swiglu_backward = swiglu_backward
