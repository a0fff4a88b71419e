"""gpt-oss MoE experts with frozen MXFP4 weights on MI355X (drop-in module).

Same public API as the reference's ``src/agent_factory_3/models/gpt_oss/
quantization.py``, for both ``dequant_dtype`` modes:

================================  ===========================================
reference (quantization.py)       here
================================  ===========================================
``mxfp4_to_bf16`` 89-99           HIP dequant kernel (bit-exact)
``FP4_VALUES`` 131-134            same table (e2m1 code -> value)
``convert_moe_packed_tensors``    HIP dequant + transpose to [E, K, N]
  137-172
pack / unpack / store 232-287     same byte reinterpretation into bf16
                                  containers (FSDP2-shardable)
``DequantMoEMatmul`` 294-421      grouped GEMM with the MXFP4 -> bf16
                                  conversion fused into the tile load
                                  (no materialised bf16 weight), 15 inputs,
                                  gradient for ``x`` only
``SwiGLUFunction`` 424-444        HIP clamped SwiGLU fwd/bwd
``Mxfp4Bf16DequantGptOssExperts`` same parameters/attributes/forward
  451-544
``routing_torch_dist`` 551-590    top-k routing (world size 1)
``routing_replay`` 593-636        HIP routing kernels
``mlp_forward`` 639-668           same control flow
``replace_with_dequant_experts``  same module surgery
  675-699
================================  ===========================================

New (not in the reference, which puts LoRA on attention only): per-expert
LoRA on both projections (``enable_expert_lora``), with the PEFT convention
``W_eff = W + (lora_alpha / r) * B @ A`` (model_trainer.py:665,711) and bf16
adapters; its autograd function returns gradients for ``x``, ``A`` and ``B``.

``dequant_dtype="fp8"`` (quantization.py:332-357, 382-408) quantizes the
activation (forward) or the incoming gradient (backward) per token to fp8
E4M3FN and runs the same grouped GEMM on the codes' values (exact in bf16)
with the per-token scale applied to the fp32 accumulator; the reference's
E5M2 weights hold exactly the MXFP4 values, so the products are the same.
Expert LoRA is bf16-mode only.

Every compute call goes to ``libaf3_mi355x.so``; there is no CPU or eager
fallback.
"""
from __future__ import annotations

import math
from contextlib import contextmanager

import torch
from torch import nn

from . import _capi, kernels
from .kernels import mxfp4_to_bf16_hip, swiglu_backward_raw, swiglu_forward
from .routing import (  # noqa: F401  (re-exported names of the routing layer)
    ExptData, GatherIndx, RoutingData, ScatterIndx, compute_expt_data, compute_expt_data_torch,
    dense_routing, gemm_order_for, max_tiles, router_linear, routing, routing_replay,
)

GEMM_BLOCK_M = 128
# Grouped-GEMM tile selection (tuning knob): rows per tile (128 or 256) of
# explicitly selected configurations, and the C library's tile_cfg (0 =
# default).  The default kernels take the map of fwd_block_m (forward, tile_cfg
# 26) and dx_block_m (input gradient, tile_cfg 28), both 128; 256 there selects
# the 256 x 256 kernels (tile_cfg 22 / 23).  The LoRA row products always use
# the 128-row map.  x_off32: tell the library when x lies within 4 GiB (the
# forward then addresses it by a scalar base and 32-bit offsets).
GEMM_TILE = {"block_m": 256, "tile_cfg": 0, "fwd_block_m": 128, "dx_block_m": 128}

# The expert module's forward GEMMs read a tiled copy of each frozen
# projection's packed weights (af3_mxfp4_tile_fwd: the words one k-step of a
# wave needs from 32 weight rows are one contiguous KB), made on first use and
# kept per weight storage and version: one more copy of the packed blocks on
# the device (1.6 GB for a gpt-oss-120b layer's 128 experts).  The input
# gradient, the checkpoint format and the scales use the blocks as stored.
FWD_TILED_WEIGHTS = True
# The input-gradient GEMMs read a tiled copy of each projection's e8m0 scales
# (af3_mxfp4_tile_dx_scales: a wave's scale bytes of a k-step are 128
# contiguous bytes), made on first use and kept like the tiled weights (1/16
# of the packed blocks' size, ~0.1 GB for a gpt-oss-120b layer).
DX_TILED_SCALES = True

# Optional launch timer for the grouped GEMM (set by benchmark harnesses):
# callable(tag: str, flops: int, detail: str) -> context manager wrapping the launch.
KERNEL_TIMER = None

FP4_VALUES = [
    +0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
    -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0,
]


@contextmanager
def on_device(dev):
    if isinstance(dev, torch.Tensor):
        dev = dev.device
    elif isinstance(dev, str):
        dev = torch.device(dev)
    if getattr(dev, "type", None) == "cuda":
        with torch.cuda.device(dev):
            yield
            return
    yield


# ---------------------------------------------------------------------------
# dequant
# ---------------------------------------------------------------------------

def mxfp4_to_bf16(blocks, scales):
    """MXFP4 [..., G, 16] + scales [..., G] -> bf16 [..., G*32] (quantization.py:89-99)."""
    return mxfp4_to_bf16_hip(blocks, scales)


def convert_moe_packed_tensors(blocks, scales, *, dtype=torch.bfloat16, rows_per_chunk=None):
    """Dequantize to a full weight, transposed to [E, K, N] (quantization.py:137-172).

    Used by the dequantize-at-load fallback of the quantizer.  Scale bytes
    2..252 give the reference's LUT + ldexp values bit for bit; bytes 0, 1 and
    253..255 follow the kernels' flush-to-signed-zero rule (kernels.py:151-156)
    where ldexp would give bf16 subnormals, inf or NaN, so a loaded weight
    equals what the fused GEMMs compute with.
    """
    if dtype != torch.bfloat16:
        raise TypeError("only bf16 dequantisation is implemented")
    blocks, scales = blocks.to(torch.uint8), scales.to(torch.uint8)
    try:
        if not blocks.is_cuda:
            blocks, scales = blocks.cuda(), scales.cuda()
        return mxfp4_to_bf16_hip(blocks, scales).transpose(1, 2).contiguous()
    except torch.OutOfMemoryError:
        # quantization.py:166-172 retries on the CPU when the device runs out of
        # memory; here the HIP kernel dequantizes one expert at a time and the
        # weight is assembled in host memory (same values, returned on the CPU).
        return _convert_per_expert_to_host(blocks, scales)


def _convert_per_expert_to_host(blocks, scales):
    """[E, N, G, 16] + [E, N, G] -> CPU bf16 [E, G*32, N], one expert's weight on the GPU at a time."""
    dev = blocks.device if blocks.is_cuda else torch.device("cuda", torch.cuda.current_device())
    E, N, G = scales.shape
    out = torch.empty(E, G * 32, N, dtype=torch.bfloat16)
    for e in range(E):
        w = mxfp4_to_bf16_hip(blocks[e].to(dev), scales[e].to(dev)).t().contiguous()
        out[e].copy_(w)      # synchronous device-to-host copy; w is freed with the next expert
        del w
    return out


# ---------------------------------------------------------------------------
# FSDP-compatible storage of the packed bytes (quantization.py:232-287)
# ---------------------------------------------------------------------------

def _pack_uint8_as_bf16(tensor):
    """Reinterpret a uint8 tensor as bf16 (two bytes per element, odd length padded)."""
    flat = tensor.contiguous().reshape(-1)
    if flat.numel() % 2:
        flat = torch.cat([flat, flat.new_zeros(1)])
    return flat.view(torch.bfloat16)


def _unpack_bf16_as_uint8(packed, shape):
    """View bf16-packed bytes as a uint8 tensor of ``shape`` (no copy)."""
    numel = math.prod(shape)
    return packed.reshape(-1).view(torch.uint8)[:numel].reshape(shape)


def _store_mxfp4_weights(blocks, scales, module, proj, target_device):
    """Register ``{proj}_blocks`` / ``{proj}_scales`` as bf16-container Parameters."""
    if getattr(target_device, "type", target_device) == "cpu":
        target_device = "cuda"
    blocks = blocks.to(target_device).contiguous()
    scales = scales.to(target_device).contiguous()
    for attr in (f"{proj}_blocks", f"{proj}_scales", proj):
        if attr in module._parameters:
            del module._parameters[attr]
    setattr(module, f"_{proj}_shapes", (tuple(blocks.shape), tuple(scales.shape)))
    module.register_parameter(f"{proj}_blocks", nn.Parameter(_pack_uint8_as_bf16(blocks), requires_grad=False))
    module.register_parameter(f"{proj}_scales", nn.Parameter(_pack_uint8_as_bf16(scales), requires_grad=False))


# ---------------------------------------------------------------------------
# grouped GEMM (the matmul_ogs replacement)
# ---------------------------------------------------------------------------

def _expt_data(routing_data, n_rows, device):
    if routing_data is None:
        return dense_routing(n_rows, device), 1
    ed = routing_data.expt_data
    if ed is None or not all(bm in getattr(ed, "block_pid_map", {}) for bm in (128, 256, WGRAD_CHUNK)):
        ed = compute_expt_data(routing_data.expt_hist, routing_data.n_expts_tot, n_rows)
        routing_data = RoutingData(routing_data.gate_scal, routing_data.expt_hist, routing_data.n_expts_tot,
                                   routing_data.n_expts_act, ed)
    return routing_data, routing_data.n_expts_act


def _gather_ptr(gather_indx):
    if gather_indx is None:
        return None
    g = gather_indx.src_indx
    if g.dtype != torch.int32:
        g = g.to(torch.int32)
    return g.contiguous()


def _weight_dims(blocks, trans_w):
    """(E, N, K) of the GEMM from the MXFP4 block tensor [E, rows, G, 16]."""
    if blocks.dim() == 3:
        blocks = blocks.unsqueeze(0)
    E, rows, G, _ = blocks.shape
    return (E, G * 32, rows) if trans_w else (E, rows, G * 32)


def mxfp4_tile_fwd(blocks):
    """Forward-tiled copy of packed MXFP4 weights ``blocks`` [E, N, K/32, 16]
    (uint8, N % 32 == 0, K % 64 == 0): the same bytes permuted so that
    ``out.view(E, N/32, K/64, 2, 32, 16)[e, n // 32, kt, h, n % 32] ==
    blocks[e, n, 2 kt + h]``; ``moe_rows(..., w_tiled=out)`` reads it in the
    forward.  No counterpart in the reference (its matmul_ogs reads the stored
    layout, quantization.py:358-362)."""
    if not blocks.is_cuda:
        raise RuntimeError("blocks must be a GPU tensor (the MI355X path has no CPU implementation)")
    b = blocks if blocks.dim() == 4 else blocks.unsqueeze(0)
    if b.dtype != torch.uint8 or b.shape[-1] != 16:
        raise TypeError(f"blocks must be uint8 [E, N, K/32, 16] (got {b.dtype} {tuple(b.shape)})")
    E, N, G, _ = b.shape
    b = b if b.is_contiguous() and b.data_ptr() % 16 == 0 else b.contiguous()
    out = torch.empty(b.shape, dtype=torch.uint8, device=b.device)
    _capi.call("af3_mxfp4_tile_fwd", b.data_ptr(), E, N, G * 32, out.data_ptr(), _capi.stream_of(b.device))
    return out.view(blocks.shape)


def mxfp4_tile_dx_scales(scales):
    """Tiled copy of the e8m0 scales ``scales`` [E, K, N/32] of trans_w=True
    weights (K % 64 == 0) for the input-gradient kernel, flat uint8:
    ``out[:E*K/64*NT*512].view(E, K/64, NT, 8, 64)[e, k // 64, n // 256,
    (n // 32) % 8, k % 64] == scales[e, k, n // 32]`` (NT = ceil(N/256), 127
    past N/32), then ``out[-E*NT:].view(E, NT)``: 1 where a scale byte of the
    n-tile lies outside [2, 252]; ``moe_rows(..., trans_w=True, s_tiled=out)``
    reads it.  No counterpart in the reference."""
    if not scales.is_cuda:
        raise RuntimeError("scales must be a GPU tensor (the MI355X path has no CPU implementation)")
    s = scales if scales.dim() == 3 else scales.unsqueeze(0)
    if s.dtype != torch.uint8:
        raise TypeError(f"scales must be uint8 [E, K, N/32] (got {s.dtype})")
    E, K, G = s.shape
    s = s.contiguous()
    nt = (G * 32 + 255) // 256
    out = torch.empty(E * nt * ((K // 64) * 512 + 1), dtype=torch.uint8, device=s.device)
    _capi.call("af3_mxfp4_tile_dx_scales", s.data_ptr(), E, K, G * 32, out.data_ptr(), _capi.stream_of(s.device))
    return out


def moe_rows(x, blocks, scales, bias, routing_data, gather_indx=None, gammas=None, trans_w=False,
             lora_l=None, lora_b=None, swiglu=None, a_row_scale=None, w_tiled=None, s_tiled=None):
    """Expert-sorted output rows of the grouped GEMM (no scatter).

    ``trans_w=False``: ``Y[r] = X[a(r)] @ W[e]^T`` with W = dequant(blocks) [E, N, K]
    (matmul_ogs(x, w.transpose(-1, -2)), quantization.py:361).
    ``trans_w=True``:  ``Y[r] = X[a(r)] @ W[e]`` (matmul_ogs(grad, w), quantization.py:411).
    Then ``(+ bias[e]) * gammas[r]`` and bf16 rounding.  ``lora_l``/``lora_b``
    append the expert-LoRA term ``L[r] @ B[e]^T`` (trans 0) / ``L[r] @ B[e]``.

    ``swiglu=("fwd", alpha, limit)`` (trans 0) also returns the clamped SwiGLU
    of the bf16 rows, ``(Y, act)``; ``swiglu=("bwd", gate_up, alpha, limit)``
    (trans 1) returns the SwiGLU backward of the bf16 rows against the saved
    interleaved pre-activation ``gate_up`` [R, 2N], i.e. dGU [R, 2N].  Both are
    fused into the GEMM epilogue; None is returned when the selected kernel
    has no fused epilogue (the caller then runs the two steps separately).
    ``w_tiled``: the ``mxfp4_tile_fwd`` copy of ``blocks``, read instead of
    them by the default forward kernel (ignored by the others); ``s_tiled``:
    the ``mxfp4_tile_dx_scales`` copy of ``scales``, read instead of them by
    the default input-gradient kernel.
    """
    if not x.is_cuda:
        raise RuntimeError("x must be a GPU tensor (the MI355X path has no CPU implementation)")
    if x.dtype != torch.bfloat16:
        raise TypeError(f"x must be bfloat16 (got {x.dtype})")
    dev = x.device
    x = x if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0 else x.contiguous()
    E, N, K = _weight_dims(blocks, trans_w)
    if x.shape[-1] != K:
        raise ValueError(f"x has {x.shape[-1]} columns, weight reduction dim is {K}")
    g = _gather_ptr(gather_indx)
    R = g.shape[0] if g is not None else x.shape[0]
    routing_data, k_act = _expt_data(routing_data, R, dev)
    ed = routing_data.expt_data
    bm = GEMM_TILE["block_m"] if K % 64 == 0 else 128
    if K % 64 == 0 and a_row_scale is None:
        # the default kernels (tile_cfg 26 forward, 28 input gradient) run on the 128-row map
        if not trans_w and GEMM_TILE["tile_cfg"] % 100 in (0, 26):
            bm = GEMM_TILE.get("fwd_block_m", 128)
        elif trans_w and GEMM_TILE["tile_cfg"] % 100 in (0, 28):
            bm = GEMM_TILE.get("dx_block_m", 128)
    pid_map = gemm_order_for(ed, bm) if GEMM_TILE.get("order", True) else None
    if pid_map is None:
        pid_map = ed.block_pid_map[bm]
    offs = ed.token_offs_raw
    epi, glu, ld_glu, alpha, limit = 0, None, 0, 0.0, 0.0
    if swiglu is None:
        y = torch.empty(R, N, dtype=torch.bfloat16, device=dev)
    elif swiglu[0] == "fwd" and not trans_w:
        epi, alpha, limit = 2, float(swiglu[1]), float(swiglu[2])
        y = torch.empty(R, N, dtype=torch.bfloat16, device=dev)
        glu = torch.empty(R, N // 2, dtype=torch.bfloat16, device=dev)
        ld_glu = N // 2
    elif swiglu[0] == "bwd" and trans_w:
        epi, alpha, limit = 1, float(swiglu[2]), float(swiglu[3])
        glu = swiglu[1]
        if glu.shape != (R, 2 * N) or glu.stride(-1) != 1:
            raise ValueError(f"gate_up pre-activation must be [{R}, {2 * N}] with unit column stride")
        ld_glu = glu.stride(0) if R > 1 else 2 * N
        y = torch.empty(R, 2 * N, dtype=torch.bfloat16, device=dev)
    else:
        raise ValueError(f"bad swiglu epilogue request {swiglu[0]!r} for trans_w={trans_w}")
    if R == 0 or pid_map.numel() == 0:
        return y if epi == 0 else (y, glu) if epi == 2 else y
    blocks = blocks if blocks.data_ptr() % 16 == 0 else blocks.clone()
    if w_tiled is not None and (w_tiled.shape != blocks.shape or w_tiled.dtype != torch.uint8 or not w_tiled.is_contiguous()
                              or w_tiled.data_ptr() % 16):
        raise ValueError("w_tiled must be the mxfp4_tile_fwd copy of blocks (same shape, contiguous uint8)")
    b = None
    if bias is not None:
        b = bias.to(torch.float32).contiguous()
    gm, gm_f32 = None, 0
    if gammas is not None:
        if gammas.dtype == torch.float32:
            gm, gm_f32 = gammas.contiguous(), 1
        else:
            gm = gammas.to(torch.bfloat16).contiguous()
    lr = 0
    if lora_l is not None:
        lr = lora_l.shape[-1]
        lora_l = lora_l.contiguous()
        lora_b = lora_b.to(torch.bfloat16).contiguous()
    ldx = x.stride(0) if x.shape[0] > 1 else K
    # every row of x lies within 4 GiB of x: the kernels may address it by 32-bit offsets
    off32 = GEMM_TILE.get("x_off32", True) and ((x.shape[0] - 1) * ldx + K) * 2 <= 1 << 32
    cfg = GEMM_TILE["tile_cfg"] | (_capi.X_OFFSETS_32 if off32 else 0)
    args = (x.data_ptr(), ldx, _capi.ptr(g), k_act if g is not None else 1,
            blocks.data_ptr(), scales.data_ptr(), 1 if trans_w else 0, _capi.ptr(b), _capi.ptr(gm), gm_f32,
            _capi.ptr(lora_l), lr, _capi.ptr(lora_b), lr, offs.data_ptr(), pid_map.data_ptr(),
            ed.token_offs_pad[bm].data_ptr(), pid_map.numel(), bm, cfg, E, N, K, y.data_ptr(), y.shape[1])
    stream = _capi.stream_of(dev)

    if a_row_scale is not None:  # fp8 mode: (acc * a_row_scale[a(r)] + bias) * gammas
        if epi or lr:
            raise ValueError("a row scale cannot be combined with the LoRA segment or a fused SwiGLU")
        a_row_scale = a_row_scale.to(torch.float32).contiguous()

    # the tiled weights go to the default forward kernel, the tiled scales to
    # the default input-gradient kernel; any other selection declines them
    # (nothing launched) and the stored blocks / scales are used
    targs = None
    if w_tiled is not None and not trans_w and a_row_scale is None and bm == 128 \
            and GEMM_TILE["tile_cfg"] % 100 in (0, 26):
        targs = list(args)
        targs[4], targs[19] = w_tiled.data_ptr(), cfg | _capi.W_FWD_TILED
    if s_tiled is not None and trans_w and a_row_scale is None and bm == 128 \
            and GEMM_TILE["tile_cfg"] % 100 in (0, 28):
        if s_tiled.dtype != torch.uint8 or not s_tiled.is_contiguous() \
                or s_tiled.numel() != E * ((N + 255) // 256) * ((K // 64) * 512 + 1):
            raise ValueError("s_tiled must be the mxfp4_tile_dx_scales copy of scales")
        targs = list(args)
        targs[5], targs[19] = s_tiled.data_ptr(), cfg | _capi.S_DX_TILED

    def launch():
        if a_row_scale is not None:
            rargs = args[:10] + args[14:]   # without the LoRA operands
            if not _capi.try_call("af3_moe_gemm_rowscale", *rargs, a_row_scale.data_ptr(), stream):
                raise RuntimeError("moe_gemm: the A row scale needs the default tile configurations (20-23)")
            return True
        if targs is not None:
            if epi == 0 and _capi.try_call("af3_moe_gemm", *targs, stream):
                return True
            if epi and _capi.try_call("af3_moe_gemm_swiglu", *targs, epi, glu.data_ptr(), ld_glu, alpha, limit,
                                      stream):
                return True
        if epi == 0:
            _capi.call("af3_moe_gemm", *args, stream)
            return True
        return _capi.try_call("af3_moe_gemm_swiglu", *args, epi, glu.data_ptr(), ld_glu, alpha, limit, stream)

    if KERNEL_TIMER is None:
        ok = launch()
    else:
        detail = f"{'dX' if trans_w else 'fwd'} N={N} K={K}" + {0: "", 1: " +SwiGLU bwd", 2: " +SwiGLU fwd"}[epi]
        with KERNEL_TIMER("moe_gemm_dgrad" if trans_w else "moe_gemm_fwd", 2 * R * N * (K + lr), detail):
            ok = launch()
    if not ok:
        return None
    return (y, glu) if epi == 2 else y


def moe_combine(rows, scatter_indx, n_expts_act):
    """Sum each token's K expert rows (matmul_ogs scatter reduction)."""
    src = scatter_indx.src_indx
    src = (src if src.dtype == torch.int32 else src.to(torch.int32)).contiguous()
    n_tokens = src.shape[0] // n_expts_act
    N = rows.shape[-1]
    out = torch.empty(n_tokens, N, dtype=torch.bfloat16, device=rows.device)
    if n_tokens:
        _capi.call("af3_moe_combine", rows.data_ptr(), rows.stride(0), src.data_ptr(), n_tokens, n_expts_act, N,
                   out.data_ptr(), N, _capi.stream_of(rows.device))
    return out


def moe_rows_f8(codes, a_row_scale, blocks, scales, bias, routing_data, gather_indx=None, gammas=None,
                trans_w=False):
    """Rows of the fp8 mode on the block-scaled MFMA: per-token E4M3 ``codes``
    [Tx, K] (float8_e4m3fn, rows 16-byte aligned) times the MXFP4 weights
    (``trans_w`` as in ``moe_rows``: False for the forward, True for the input
    gradient, whose weights the kernel converts to E5M2), ``(acc *
    a_row_scale[a(r)] + bias[e]) * gammas`` in bf16.  None when the kernel's
    requirements do not hold (the caller then runs the bf16-operand form of
    the same arithmetic)."""
    dev = codes.device
    E, N, K = _weight_dims(blocks, trans_w)
    if codes.shape[-1] != K:
        raise ValueError(f"codes have {codes.shape[-1]} columns, weight reduction dim is {K}")
    g = _gather_ptr(gather_indx)
    R = g.shape[0] if g is not None else codes.shape[0]
    routing_data, k_act = _expt_data(routing_data, R, dev)
    ed = routing_data.expt_data
    bm = 256
    pid_map = gemm_order_for(ed, bm) if GEMM_TILE.get("order", True) else None
    if pid_map is None:
        pid_map = ed.block_pid_map[bm]
    y = torch.empty(R, N, dtype=torch.bfloat16, device=dev)
    if R == 0 or pid_map.numel() == 0:
        return y
    ld = codes.stride(0) if codes.shape[0] > 1 else K
    if (codes.stride(-1) != 1 or ld % 16 or codes.data_ptr() % 16 or K % 64 or (trans_w and N % 64)
            or GEMM_TILE["tile_cfg"] not in ((0, 23) if trans_w else (0, 22))):
        return None
    blocks = blocks if blocks.data_ptr() % 16 == 0 else blocks.clone()
    b = bias.to(torch.float32).contiguous() if bias is not None else None
    gm, gm_f32 = None, 0
    if gammas is not None:
        gm, gm_f32 = (gammas.contiguous(), 1) if gammas.dtype == torch.float32 else (
            gammas.to(torch.bfloat16).contiguous(), 0)
    s = a_row_scale.to(torch.float32).contiguous()

    def launch():
        return _capi.try_call("af3_moe_gemm_f8", codes.data_ptr(), ld, _capi.ptr(g),
                              k_act if g is not None else 1, blocks.data_ptr(), scales.data_ptr(), int(trans_w),
                              _capi.ptr(b),
                              _capi.ptr(gm), gm_f32, ed.token_offs_raw.data_ptr(), pid_map.data_ptr(),
                              ed.token_offs_pad[bm].data_ptr(), pid_map.numel(), bm, 0, E, N, K, y.data_ptr(), N,
                              s.data_ptr(), _capi.stream_of(dev))
    if KERNEL_TIMER is None:
        ok = launch()
    else:
        with KERNEL_TIMER("moe_gemm_dgrad_f8" if trans_w else "moe_gemm_fwd_f8", 2 * R * N * K):
            ok = launch()
    return y if ok else None


FP8_BLOCK_SCALED = True  # fp8 mode on the block-scaled MFMA (else: E4M3 values as bf16 operands)


def matmul_ogs(x, w_blocks_scales, bias, routing_data=None, gather_indx=None, scatter_indx=None, gammas=None,
               trans_w=False, a_row_scale=None):
    """matmul_ogs semantics over MXFP4 weights: rows, then the scatter-sum if any.
    ``a_row_scale`` (fp32, one per row of ``x``): the per-token scale of fp8
    activations (PrecisionConfig lhs ``scale_mode="per_token"``), applied to
    the accumulator before bias and gammas."""
    blocks, scales = w_blocks_scales
    y = moe_rows(x, blocks, scales, bias, routing_data, gather_indx, gammas, trans_w, a_row_scale=a_row_scale)
    if scatter_indx is None:
        return y
    k = routing_data.n_expts_act if routing_data is not None else 1
    return moe_combine(y, scatter_indx, k)


# ---------------------------------------------------------------------------
# Autograd functions
# ---------------------------------------------------------------------------

def _gamma_grad(d_act, act, dY, gather, k_act, bias, routing_data, gammas):
    """d gamma[r] = <dY[t(r)], y[r]> for the down projection's expert rows, from its
    gamma-scaled input gradient ``d_act`` (= gamma * dY W), its input ``act`` and the
    bias (``af3_gamma_grad``); returned in ``gammas``' dtype."""
    R, N = act.shape
    ed = routing_data.expt_data
    out = torch.empty(R, dtype=torch.float32, device=act.device)
    gam = _bf16c(gammas)
    b = bias.float().contiguous() if bias is not None else None
    dyc = dY.contiguous()
    gp = _gather_ptr(gather)
    _capi.call("af3_gamma_grad", d_act.data_ptr(), d_act.stride(0), act.data_ptr(), act.stride(0), N,
               dyc.data_ptr(), dyc.stride(0), gp.data_ptr() if gp is not None else None,
               k_act if gather is not None else 1,
               b.data_ptr() if b is not None else None, b.shape[1] if b is not None else 0,
               ed.token_offs_raw.data_ptr(), routing_data.n_expts_tot, gam.data_ptr(), R, out.data_ptr(),
               _capi.stream_of(act.device))
    return out.to(gammas.dtype)


class DequantMoEMatmul(torch.autograd.Function):
    """MXFP4 grouped GEMM (quantization.py:294-421), dequant fused into the GEMM.

    Weights are not saved: backward re-derives them from ``experts_module``
    (FSDP re-gathers them for backward).  Returns a gradient for ``x`` only.
    """

    @staticmethod
    def forward(ctx, x, blocks, scales, bias, routing_data, fwd_gather_indx, fwd_scatter_indx, fwd_gammas,
                bwd_gather_indx, bwd_scatter_indx, bwd_gammas, dequant_dtype="bf16", n_expts_act=1,
                experts_module=None, proj_name=None):
        if dequant_dtype not in ("bf16", "fp8"):
            raise NotImplementedError(f"dequant_dtype={dequant_dtype!r}: 'bf16' or 'fp8'")
        with on_device(x.device):
            if dequant_dtype == "fp8":
                # quantization.py:332-357: per-token E4M3 activations x MXFP4 weights (their E5M2
                # form has the same values), fp32 accumulation scaled per row, bf16 out
                y = None
                if FP8_BLOCK_SCALED:
                    xc, xs = kernels.quantize_per_token_e4m3(x.to(torch.bfloat16))
                    y = moe_rows_f8(xc, xs, blocks, scales, bias, routing_data, fwd_gather_indx, fwd_gammas)
                if y is None:
                    _, xs, xq = kernels.quantize_per_token_e4m3(x.to(torch.bfloat16), with_bf16=True)
                    y = moe_rows(xq, blocks, scales, bias, routing_data, fwd_gather_indx, fwd_gammas, False,
                                 a_row_scale=xs)
                k = routing_data.n_expts_act if routing_data is not None else 1
                out = y if fwd_scatter_indx is None else moe_combine(y, fwd_scatter_indx, k)
            else:  # matmul_ogs(x, (blocks, scales), ...) with the module's forward-tiled weights
                y = moe_rows(x, blocks, scales, bias, routing_data, fwd_gather_indx, fwd_gammas, False,
                             w_tiled=_fwd_weights(experts_module, proj_name))
                k = routing_data.n_expts_act if routing_data is not None else 1
                out = y if fwd_scatter_indx is None else moe_combine(y, fwd_scatter_indx, k)
        ctx.experts_module = experts_module
        ctx.proj_name = proj_name
        if experts_module is None:  # no module to re-derive from: keep the (view) tensors
            ctx.weights = (blocks, scales)
        if ctx.needs_input_grad[7]:  # routing-weight gradient (routing.GAMMA_GRAD)
            if fwd_gather_indx is not None or fwd_scatter_indx is None:
                raise NotImplementedError("routing-weight gradients are implemented for the down projection")
            ctx.save_for_backward(x, fwd_gammas)
            ctx.gamma_bias = bias
        ctx.routing_data = routing_data
        ctx.bwd_gather_indx = bwd_gather_indx
        ctx.bwd_scatter_indx = bwd_scatter_indx
        ctx.bwd_gammas = bwd_gammas
        ctx.dequant_dtype = dequant_dtype
        ctx.n_expts_act = n_expts_act
        return out

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.experts_module is not None:
            blocks, scales = ctx.experts_module._get_uint8_weights(ctx.proj_name)
        else:
            blocks, scales = ctx.weights
        with on_device(grad_output.device):
            g = grad_output.to(torch.bfloat16).contiguous()
            if ctx.dequant_dtype == "fp8":  # quantization.py:382-408
                grad_x = None
                if FP8_BLOCK_SCALED:
                    gc, gs = kernels.quantize_per_token_e4m3(g)
                    y = moe_rows_f8(gc, gs, blocks, scales, None, ctx.routing_data, ctx.bwd_gather_indx,
                                    ctx.bwd_gammas, trans_w=True)
                    if y is not None:
                        k = ctx.routing_data.n_expts_act if ctx.routing_data is not None else 1
                        grad_x = y if ctx.bwd_scatter_indx is None else moe_combine(y, ctx.bwd_scatter_indx, k)
                if grad_x is None:
                    _, gs, gq = kernels.quantize_per_token_e4m3(g, with_bf16=True)
                    grad_x = matmul_ogs(gq, (blocks, scales), None, ctx.routing_data, ctx.bwd_gather_indx,
                                        ctx.bwd_scatter_indx, ctx.bwd_gammas, trans_w=True, a_row_scale=gs)
            else:  # matmul_ogs(g, (blocks, scales), ..., trans_w=True) with the module's tiled scales
                y = moe_rows(g, blocks, scales, None, ctx.routing_data, ctx.bwd_gather_indx, ctx.bwd_gammas, True,
                             s_tiled=_dx_scales(ctx.experts_module, ctx.proj_name))
                k = ctx.routing_data.n_expts_act if ctx.routing_data is not None else 1
                grad_x = y if ctx.bwd_scatter_indx is None else moe_combine(y, ctx.bwd_scatter_indx, k)
            d_gam = None
            if ctx.needs_input_grad[7]:
                x, gam = ctx.saved_tensors
                d_gam = _gamma_grad(grad_x, _bf16c(x), g, ctx.bwd_gather_indx, ctx.n_expts_act, ctx.gamma_bias,
                                    ctx.routing_data, gam)
        return grad_x, None, None, None, None, None, None, d_gam, None, None, None, None, None, None, None


class SwiGLUFunction(torch.autograd.Function):
    """gpt-oss clamped SwiGLU (quantization.py:424-444).

    Saves the raw interleaved input (same bytes as the reference's clamped
    gate + up pair) and clamps again in backward, so the forward writes only
    its output.
    """

    @staticmethod
    def forward(ctx, gate_up_raw, alpha, limit):
        out = swiglu_forward(gate_up_raw, alpha, limit, save_for_bwd=False)
        ctx.save_for_backward(gate_up_raw)
        ctx.alpha = alpha
        ctx.limit = limit
        return out

    @staticmethod
    def backward(ctx, grad_output):
        (gate_up_raw,) = ctx.saved_tensors
        return swiglu_backward_raw(grad_output.contiguous(), gate_up_raw, ctx.alpha, ctx.limit), None, None


def _lora_rows(x, gather, k_act, wl, trans_b, scale, ed, n_out, K):
    dev = x.device
    R = gather.shape[0] if gather is not None else x.shape[0]
    out = torch.empty(R, n_out, dtype=torch.bfloat16, device=dev)
    # full tiles first: the tiles past one round of resident blocks are then the
    # partial ones, whose clamped rows are cache hits
    pid_map = gemm_order_for(ed, GEMM_BLOCK_M)
    if pid_map is None:
        pid_map = ed.block_pid_map[GEMM_BLOCK_M]
    if R and pid_map.numel():
        E = wl.shape[0]
        _capi.call("af3_lora_rows", x.data_ptr(), x.stride(0) if x.shape[0] > 1 else K, _capi.ptr(gather),
                   k_act if gather is not None else 1, wl.data_ptr(), trans_b, float(scale),
                   ed.token_offs_raw.data_ptr(), pid_map.data_ptr(), pid_map.numel(), E, n_out, K,
                   out.data_ptr(), n_out, _capi.stream_of(dev))
    return out


WGRAD_CHUNK = 512


def _wgrad_chunks(ed, R, E):
    """Entries of the WGRAD_CHUNK tile map the weight-gradient kernels visit:
    R expert-sorted rows over E experts make at most max_tiles(R, E,
    WGRAD_CHUNK) chunks, listed first (the map itself is sized for the smallest
    tile), so the grid and the fp32 partial workspace are sized by that bound."""
    return min(ed.block_pid_map[WGRAD_CHUNK].numel(), max_tiles(R, E, WGRAD_CHUNK))


def _lora_wgrad(a, a_gather, a_div, a_rowscale, b, b_gather, b_div, ed, E, M, N):
    dev = a.device
    g = torch.empty(E, M, N, dtype=torch.bfloat16, device=dev)
    cmap = ed.block_pid_map[WGRAD_CHUNK]
    coffs = ed.token_offs_pad[WGRAD_CHUNK]
    R = a_gather.shape[0] if a_gather is not None else (b_gather.shape[0] if b_gather is not None else a.shape[0])
    nch = _wgrad_chunks(ed, R, E)
    ws_n = int(_capi.load().af3_lora_wgrad_workspace_bytes(nch, M, N))
    ws = torch.empty(ws_n // 4, dtype=torch.float32, device=dev)
    _capi.call("af3_lora_wgrad", a.data_ptr(), a.stride(0) if a.shape[0] > 1 else M, _capi.ptr(a_gather), a_div,
               _capi.ptr(a_rowscale), b.data_ptr(), b.stride(0) if b.shape[0] > 1 else N, _capi.ptr(b_gather),
               b_div, 1.0, ed.token_offs_raw.data_ptr(), E, M, N, cmap.data_ptr(), coffs.data_ptr(), nch,
               WGRAD_CHUNK, ws.data_ptr(), ws_n, g.data_ptr(), _capi.stream_of(dev))
    return g


def _lora_u_and_dB(big, gather, gdiv, rowscale, L, Bw, scale, ed, E, W):
    """The two LoRA backward products that read the wide gradient ``big``:
    u[i] = scale * big[b(i)] @ Bw[e]  and  dB[e] = sum_i bf16(rs(i) big[b(i)])^T L[i],
    in one pass over ``big`` (af3_lora_u_wgrad); shapes it declines go through
    _lora_rows and _lora_wgrad."""
    dev = big.device
    R, r = L.shape
    u = torch.empty(R, r, dtype=torch.bfloat16, device=dev)
    g = torch.empty(E, W, r, dtype=torch.bfloat16, device=dev)
    cmap = ed.block_pid_map[WGRAD_CHUNK]
    coffs = ed.token_offs_pad[WGRAD_CHUNK]
    nch = _wgrad_chunks(ed, R, E)
    ws_n = int(_capi.load().af3_lora_u_wgrad_workspace_bytes(nch, R, W, r))
    ws = torch.empty(max(ws_n, 1), dtype=torch.uint8, device=dev)
    L = L.contiguous()
    Bw = Bw.contiguous()
    if _capi.try_call("af3_lora_u_wgrad", big.data_ptr(), big.stride(0) if big.shape[0] > 1 else W,
                      _capi.ptr(gather), gdiv, _capi.ptr(rowscale), L.data_ptr(), Bw.data_ptr(), float(scale),
                      ed.token_offs_raw.data_ptr(), E, R, W, r, cmap.data_ptr(), coffs.data_ptr(), nch,
                      WGRAD_CHUNK, ws.data_ptr(), ws_n, u.data_ptr(), g.data_ptr(), _capi.stream_of(dev)):
        return u, g
    del ws
    u = _lora_rows(big, gather, gdiv, Bw, 1, scale, ed, r, W)
    return u, _lora_wgrad(big, gather, gdiv, rowscale, L, None, 1, ed, E, W, r)


class LoraDequantMoEMatmul(torch.autograd.Function):
    """Frozen-MXFP4 grouped GEMM plus a trainable per-expert LoRA term.

    Forward (trans 0 weights ``W[e]`` = dequant(blocks[e]) of shape [N, K]):
        L[r]   = bf16(s * X[a(r)] @ A[e]^T)              A: [E, r, K]
        Y_r[r] = bf16(gamma[r] * (X[a(r)] @ W[e]^T + L[r] @ B[e]^T + bias[e]))   B: [E, N, r]
        Y      = scatter-sum(Y_r) if fwd_scatter_indx else Y_r
    Backward with dZ[r] = gamma_b[r] * dY[b(r)] (b = backward gather):
        u[r]  = s * dY[b(r)] @ B[e]                      (without gamma)
        dX_r  = gamma_b[r] * (dY[b(r)] @ W[e] + u[r] @ A[e]);  dX = scatter-sum(dX_r) if bwd scatter
        dA[e] = sum_r gamma_b[r] u[r]^T X[a(r)]
        dB[e] = sum_r gamma_b[r] dY[b(r)]^T L[r]
    which are the gradients of W_eff = W + s * B @ A.
    """

    @staticmethod
    def forward(ctx, x, lora_A, lora_B, scaling, blocks, scales, bias, routing_data, fwd_gather_indx,
                fwd_scatter_indx, fwd_gammas, bwd_gather_indx, bwd_scatter_indx, bwd_gammas, experts_module=None,
                proj_name=None):
        if ctx.needs_input_grad[10]:
            raise NotImplementedError("routing-weight gradients with expert LoRA need the fused SwiGLU path "
                                      "(quantization.FUSED_SWIGLU)")
        dev = x.device
        E, N, K = _weight_dims(blocks, False)
        xg = x if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0 else x.contiguous()
        g = _gather_ptr(fwd_gather_indx)
        R = g.shape[0] if g is not None else xg.shape[0]
        routing_data, k_act = _expt_data(routing_data, R, dev)
        ed = routing_data.expt_data
        A = lora_A.to(torch.bfloat16).contiguous()
        B = lora_B.to(torch.bfloat16).contiguous()
        r = A.shape[1]
        with on_device(dev):
            L = _lora_rows(xg, g, k_act, A, 0, scaling, ed, r, K)
            y = moe_rows(xg, blocks, scales, bias, routing_data, fwd_gather_indx, fwd_gammas, False, L, B,
                         w_tiled=_fwd_weights(experts_module, proj_name))
            if fwd_scatter_indx is not None:
                y = moe_combine(y, fwd_scatter_indx, k_act)
        ctx.save_for_backward(xg, A, B, L)
        ctx.scaling = float(scaling)
        ctx.experts_module = experts_module
        ctx.proj_name = proj_name
        if experts_module is None:
            ctx.weights = (blocks, scales)
        ctx.routing_data = routing_data
        ctx.fwd_gather = g
        ctx.k_act = k_act
        ctx.bwd_gather_indx = bwd_gather_indx
        ctx.bwd_scatter_indx = bwd_scatter_indx
        ctx.bwd_gammas = bwd_gammas
        ctx.lora_dtypes = (lora_A.dtype, lora_B.dtype)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        xg, A, B, L = ctx.saved_tensors
        if ctx.experts_module is not None:
            blocks, scales = ctx.experts_module._get_uint8_weights(ctx.proj_name)
        else:
            blocks, scales = ctx.weights
        E, N, K = _weight_dims(blocks, False)
        r = A.shape[1]
        ed = ctx.routing_data.expt_data
        k_act = ctx.k_act
        dY = grad_output.to(torch.bfloat16).contiguous()
        bg = _gather_ptr(ctx.bwd_gather_indx)
        gam = ctx.bwd_gammas
        if gam is not None:
            gam = gam.to(torch.bfloat16).contiguous()
        with on_device(dY.device):
            u, dB = _lora_u_and_dB(dY, bg, k_act if bg is not None else 1, gam, L, B, ctx.scaling, ed, E, N)
            dx = moe_rows(dY, blocks, scales, None, ctx.routing_data, ctx.bwd_gather_indx, gam, True, u, A,
                          s_tiled=_dx_scales(ctx.experts_module, ctx.proj_name))
            if ctx.bwd_scatter_indx is not None:
                dx = moe_combine(dx, ctx.bwd_scatter_indx, k_act)
            dA = _lora_wgrad(u, None, 1, gam, xg, ctx.fwd_gather, k_act if ctx.fwd_gather is not None else 1,
                             ed, E, r, K)
        dA = dA.to(ctx.lora_dtypes[0])
        dB = dB.to(ctx.lora_dtypes[1])
        return (dx, dA, dB) + (None,) * 13


# ---------------------------------------------------------------------------
# Expert projections composed with the SwiGLU fused into the GEMM epilogues
# ---------------------------------------------------------------------------

# The expert module composes gate_up -> SwiGLU -> down with these two
# functions: the SwiGLU forward rides on the gate_up epilogue, and (when
# FUSED_SWIGLU_BWD) its backward on the down projection's dX epilogue.  The
# values and gradients are those of the reference's DequantMoEMatmul ->
# SwiGLUFunction -> DequantMoEMatmul chain (quantization.py:507-544), bit for
# bit; FUSED_SWIGLU = False restores that chain of separate kernels.
# The fused backward replaces the separate SwiGLU backward pass (and the dI
# round trip through HBM) by loads of the saved pre-activation inside each dX
# work item's epilogue, issued in two batches ahead of their use.  With the
# routing-weight gradient on, dI itself is needed and the separate pass runs.
FUSED_SWIGLU = True
FUSED_SWIGLU_BWD = True


def _weights_of(ctx):
    if ctx.experts_module is not None:
        return ctx.experts_module._get_uint8_weights(ctx.proj_name)
    return ctx.weights


def _fwd_weights(experts_module, proj_name):
    """The module's forward-tiled copy of ``proj_name``'s packed weights (None
    without a module or with FWD_TILED_WEIGHTS off)."""
    if experts_module is None or not FWD_TILED_WEIGHTS:
        return None
    return experts_module._fwd_tiled(proj_name)


def _dx_scales(experts_module, proj_name):
    """The module's tiled copy of ``proj_name``'s scales for the input
    gradient (None without a module or with DX_TILED_SCALES off)."""
    if experts_module is None or not DX_TILED_SCALES:
        return None
    return experts_module._dx_tiled_scales(proj_name)


def _bf16c(t):
    return None if t is None else t.to(torch.bfloat16).contiguous()


class _GateUpSwiGLU(torch.autograd.Function):
    """gate_up projection (optional expert LoRA) returning the interleaved
    pre-activation and its clamped SwiGLU from the same epilogue.  The SwiGLU
    output carries no gradient here: the pre-activation's gradient comes from
    _SwiGLUDown.backward."""

    @staticmethod
    def forward(ctx, x, lora_A, lora_B, scaling, blocks, scales, bias, routing_data, gather_indx, scatter_indx,
                alpha, limit, experts_module=None, proj_name=None):
        dev = x.device
        E, N, K = _weight_dims(blocks, False)
        xg = x if x.stride(-1) == 1 and x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0 else x.contiguous()
        g = _gather_ptr(gather_indx)
        R = g.shape[0] if g is not None else xg.shape[0]
        routing_data, k_act = _expt_data(routing_data, R, dev)
        ed = routing_data.expt_data
        A, B, L = _bf16c(lora_A), _bf16c(lora_B), None
        with on_device(dev):
            if A is not None:
                L = _lora_rows(xg, g, k_act, A, 0, scaling, ed, A.shape[1], K)
            wf = _fwd_weights(experts_module, proj_name)
            res = moe_rows(xg, blocks, scales, bias, routing_data, gather_indx, None, False, L, B,
                           swiglu=("fwd", alpha, limit), w_tiled=wf)
            if res is None:
                gu = moe_rows(xg, blocks, scales, bias, routing_data, gather_indx, None, False, L, B, w_tiled=wf)
                act = swiglu_forward(gu, alpha, limit)
            else:
                gu, act = res
        ctx.mark_non_differentiable(act)
        ctx.set_materialize_grads(False)
        # the input is needed only for the LoRA weight gradient dA (the
        # reference's DequantMoEMatmul saves nothing, quantization.py:364-373)
        ctx.save_for_backward(xg if A is not None else None, A, B, L)
        ctx.scaling = float(scaling)
        ctx.experts_module = experts_module
        ctx.proj_name = proj_name
        if experts_module is None:
            ctx.weights = (blocks, scales)
        ctx.routing_data = routing_data
        ctx.fwd_gather = g
        ctx.k_act = k_act
        ctx.scatter_indx = scatter_indx
        ctx.lora_dtypes = (lora_A.dtype, lora_B.dtype) if lora_A is not None else None
        return gu, act

    @staticmethod
    def backward(ctx, grad_gu, grad_act):
        xg, A, B, L = ctx.saved_tensors
        blocks, scales = _weights_of(ctx)
        E, N, K = _weight_dims(blocks, False)
        ed = ctx.routing_data.expt_data
        k_act = ctx.k_act
        dGU = grad_gu.to(torch.bfloat16).contiguous()
        dA = dB = u = None
        with on_device(dGU.device):
            if A is not None:
                u, dB = _lora_u_and_dB(dGU, None, 1, None, L, B, ctx.scaling, ed, E, N)
                dB = dB.to(ctx.lora_dtypes[1])
            dx = moe_rows(dGU, blocks, scales, None, ctx.routing_data, None, None, True, u, A,
                          s_tiled=_dx_scales(ctx.experts_module, ctx.proj_name))
            if ctx.scatter_indx is not None:
                dx = moe_combine(dx, ctx.scatter_indx, k_act)
            if A is not None:
                r = A.shape[1]
                dA = _lora_wgrad(u, None, 1, None, xg, ctx.fwd_gather,
                                 k_act if ctx.fwd_gather is not None else 1, ed, E, r, K).to(ctx.lora_dtypes[0])
        return (dx, dA, dB) + (None,) * 11


class _SwiGLUDown(torch.autograd.Function):
    """Down projection (optional expert LoRA, gammas, scatter-sum) of the
    SwiGLU output ``act`` of the pre-activation ``gate_up``; backward returns
    the gradient w.r.t. ``gate_up`` straight from the fused dX + SwiGLU
    backward epilogue (``act`` itself gets none: it is a function of
    ``gate_up``)."""

    @staticmethod
    def forward(ctx, gate_up, act, lora_A, lora_B, scaling, blocks, scales, bias, routing_data, scatter_indx,
                gammas, bwd_gather_indx, alpha, limit, experts_module=None, proj_name=None):
        dev = act.device
        E, N, K = _weight_dims(blocks, False)
        R = act.shape[0]
        routing_data, k_act = _expt_data(routing_data, R, dev)
        ed = routing_data.expt_data
        A, B, L = _bf16c(lora_A), _bf16c(lora_B), None
        with on_device(dev):
            if A is not None:
                L = _lora_rows(act, None, 1, A, 0, scaling, ed, A.shape[1], K)
            y = moe_rows(act, blocks, scales, bias, routing_data, None, gammas, False, L, B,
                         w_tiled=_fwd_weights(experts_module, proj_name))
            if scatter_indx is not None:
                y = moe_combine(y, scatter_indx, k_act)
        # gate_up (the SwiGLU's input, the same bytes as the reference's saved
        # clamped gate / up pair, quantization.py:434-436) is always needed;
        # act only for the LoRA weight gradient dA and the routing-weight gradient
        keep_act = A is not None or ctx.needs_input_grad[10]
        ctx.save_for_backward(gate_up, act if keep_act else None, A, B, L)
        ctx.scaling = float(scaling)
        ctx.experts_module = experts_module
        ctx.proj_name = proj_name
        if experts_module is None:
            ctx.weights = (blocks, scales)
        ctx.routing_data = routing_data
        ctx.k_act = k_act
        ctx.gammas = gammas
        ctx.gamma_bias = bias if ctx.needs_input_grad[10] else None
        ctx.bwd_gather_indx = bwd_gather_indx
        ctx.alpha, ctx.limit = float(alpha), float(limit)
        ctx.lora_dtypes = (lora_A.dtype, lora_B.dtype) if lora_A is not None else None
        return y

    @staticmethod
    def backward(ctx, grad_output):
        gate_up, act, A, B, L = ctx.saved_tensors
        blocks, scales = _weights_of(ctx)
        E, N, K = _weight_dims(blocks, False)
        ed = ctx.routing_data.expt_data
        k_act = ctx.k_act
        dY = grad_output.to(torch.bfloat16).contiguous()
        bg = _gather_ptr(ctx.bwd_gather_indx)
        gam = _bf16c(ctx.gammas)
        dA = dB = u = None
        with on_device(dY.device):
            if A is not None:
                u, dB = _lora_u_and_dB(dY, bg, k_act if bg is not None else 1, gam, L, B, ctx.scaling, ed, E, N)
                dB = dB.to(ctx.lora_dtypes[1])
            dgu = d_gam = None
            want_gam = ctx.needs_input_grad[10]  # routing-weight gradient (routing.GAMMA_GRAD)
            if FUSED_SWIGLU_BWD and not want_gam:
                dgu = moe_rows(dY, blocks, scales, None, ctx.routing_data, ctx.bwd_gather_indx, gam, True, u, A,
                               swiglu=("bwd", gate_up, ctx.alpha, ctx.limit),
                               s_tiled=_dx_scales(ctx.experts_module, ctx.proj_name))
            if dgu is None:
                d_act = moe_rows(dY, blocks, scales, None, ctx.routing_data, ctx.bwd_gather_indx, gam, True, u, A,
                                 s_tiled=_dx_scales(ctx.experts_module, ctx.proj_name))
                if want_gam:
                    d_gam = _gamma_grad(d_act, act, dY, ctx.bwd_gather_indx, k_act, ctx.gamma_bias,
                                        ctx.routing_data, ctx.gammas)
                dgu = swiglu_backward_raw(d_act, gate_up, ctx.alpha, ctx.limit)
            if A is not None:
                r = A.shape[1]
                dA = _lora_wgrad(u, None, 1, gam, act, None, 1, ed, E, r, K).to(ctx.lora_dtypes[0])
        return (dgu, None, dA, dB) + (None,) * 6 + (d_gam,) + (None,) * 5


# ---------------------------------------------------------------------------
# Expert module
# ---------------------------------------------------------------------------

class Mxfp4Bf16DequantGptOssExperts(nn.Module):
    """MoE experts with frozen MXFP4 weights (quantization.py:451-544)."""

    def __init__(self, config):
        super().__init__()
        self.num_experts = config.num_local_experts
        self.intermediate_size = config.intermediate_size
        self.hidden_size = config.hidden_size
        self.gate_up_proj = nn.Parameter(
            torch.zeros(self.num_experts, 2 * self.intermediate_size, self.hidden_size // 32, 16,
                        dtype=torch.uint8), requires_grad=False)
        self.gate_up_proj_bias = nn.Parameter(
            torch.zeros(self.num_experts, 2 * self.intermediate_size, dtype=torch.bfloat16), requires_grad=False)
        self.down_proj = nn.Parameter(
            torch.zeros(self.num_experts, self.hidden_size, self.intermediate_size // 32, 16, dtype=torch.uint8),
            requires_grad=False)
        self.down_proj_bias = nn.Parameter(
            torch.zeros(self.num_experts, self.hidden_size, dtype=torch.bfloat16), requires_grad=False)
        self.alpha = 1.702
        self.limit = getattr(config, "swiglu_limit", 7.0)
        self.dequant_dtype = getattr(config, "dequant_dtype", "bf16")
        self.expert_lora_r = 0
        self.expert_lora_scaling = 0.0

    def _get_uint8_weights(self, proj):
        """uint8 views of the bf16-packed blocks/scales (valid while FSDP has them gathered)."""
        shapes = getattr(self, f"_{proj}_shapes", None)
        blocks_param = getattr(self, f"{proj}_blocks")
        scales_param = getattr(self, f"{proj}_scales")
        if shapes is not None:
            blocks_shape, scales_shape = shapes
            return _unpack_bf16_as_uint8(blocks_param, blocks_shape), _unpack_bf16_as_uint8(scales_param,
                                                                                            scales_shape)
        return blocks_param, scales_param

    def _proj(self, x, proj, bias, routing_data, fg, fs, fgam, bg, bs, bgam):
        blocks, scales = self._get_uint8_weights(proj)
        if self.expert_lora_r and self.dequant_dtype != "bf16":
            raise NotImplementedError("expert LoRA is implemented for dequant_dtype='bf16' only")
        if self.expert_lora_r:
            return LoraDequantMoEMatmul.apply(
                x, getattr(self, f"{proj}_lora_A"), getattr(self, f"{proj}_lora_B"), self.expert_lora_scaling,
                blocks, scales, bias, routing_data, fg, fs, fgam, bg, bs, bgam, self, proj)
        return DequantMoEMatmul.apply(x, blocks, scales, bias, routing_data, fg, fs, fgam, bg, bs, bgam,
                                      self.dequant_dtype, routing_data.n_expts_act, self, proj)

    def _bias_f32(self, proj):
        """The projection's bias in fp32 (the GEMM epilogue's operand), cast once
        per parameter storage and version instead of every call (the expert
        biases are frozen: the grouped GEMMs return no bias gradient)."""
        b = getattr(self, f"{proj}_bias")
        cache = self.__dict__.setdefault("_bias_f32_cache", {})
        hit = cache.get(proj)
        # same tensor object (held by the cache, so its storage cannot be reused
        # by another one), same storage, no in-place change since
        if hit is None or hit[0] is not b or hit[1] != (b.data_ptr(), b._version):
            hit = cache[proj] = (b, (b.data_ptr(), b._version), b.detach().float())
        return hit[2]

    def _fwd_tiled(self, proj):
        """The forward-tiled copy of the projection's packed weights
        (``mxfp4_tile_fwd``), made once per weight storage and version (the
        expert weights are frozen); None where the forward cannot read one."""
        blocks, _ = self._get_uint8_weights(proj)
        if not blocks.is_cuda or blocks.dim() != 4 or blocks.shape[1] % 32 or blocks.shape[2] % 2:
            return None
        src = getattr(self, f"{proj}_blocks", None)
        if src is None:
            return None
        cache = self.__dict__.setdefault("_fwd_tiled_cache", {})
        key = (blocks.data_ptr(), src._version, tuple(blocks.shape))
        hit = cache.get(proj)
        # same parameter object (held by the cache, so its storage cannot be
        # reused by another one), same storage, no in-place change since
        if hit is None or hit[0] is not src or hit[1] != key:
            cache.pop(proj, None)  # the old copy goes before the new one is made
            with torch.no_grad():
                hit = cache[proj] = (src, key, mxfp4_tile_fwd(blocks))
        return hit[2]

    def _dx_tiled_scales(self, proj):
        """The input gradient's tiled copy of the projection's scales
        (``mxfp4_tile_dx_scales``), made once per scale storage and version;
        None where the input-gradient kernel cannot read one."""
        _, scales = self._get_uint8_weights(proj)
        if not scales.is_cuda or scales.dim() != 3 or scales.shape[1] % 64:
            return None
        src = getattr(self, f"{proj}_scales", None)
        if src is None:
            return None
        cache = self.__dict__.setdefault("_dx_scales_cache", {})
        key = (scales.data_ptr(), src._version, tuple(scales.shape))
        hit = cache.get(proj)
        if hit is None or hit[0] is not src or hit[1] != key:
            cache.pop(proj, None)
            with torch.no_grad():
                hit = cache[proj] = (src, key, mxfp4_tile_dx_scales(scales))
        return hit[2]

    def forward(self, hidden_states: torch.Tensor, routing_data, gather_idx, scatter_idx) -> torch.Tensor:
        if FUSED_SWIGLU and self.dequant_dtype == "bf16":
            lora = self.expert_lora_r > 0
            la = (lambda proj, ab: getattr(self, f"{proj}_lora_{ab}") if lora else None)  # noqa: E731
            gu_blocks, gu_scales = self._get_uint8_weights("gate_up_proj")
            gate_up, act = _GateUpSwiGLU.apply(
                hidden_states, la("gate_up_proj", "A"), la("gate_up_proj", "B"), self.expert_lora_scaling,
                gu_blocks, gu_scales, self._bias_f32("gate_up_proj"), routing_data, gather_idx, scatter_idx,
                self.alpha, self.limit, self, "gate_up_proj")
            dn_blocks, dn_scales = self._get_uint8_weights("down_proj")
            return _SwiGLUDown.apply(
                gate_up, act, la("down_proj", "A"), la("down_proj", "B"), self.expert_lora_scaling, dn_blocks,
                dn_scales, self._bias_f32("down_proj"), routing_data, scatter_idx, routing_data.gate_scal,
                gather_idx, self.alpha, self.limit, self, "down_proj")
        gate_up_raw = self._proj(hidden_states, "gate_up_proj", self._bias_f32("gate_up_proj"), routing_data,
                                 gather_idx, None, None, None, scatter_idx, None)
        intermediate = SwiGLUFunction.apply(gate_up_raw, self.alpha, self.limit)
        return self._proj(intermediate, "down_proj", self._bias_f32("down_proj"), routing_data,
                          None, scatter_idx, routing_data.gate_scal, gather_idx, None, routing_data.gate_scal)


def enable_expert_lora(experts: Mxfp4Bf16DequantGptOssExperts, r: int = 16, lora_alpha: float = 32.0,
                       init: str = "peft", generator: torch.Generator | None = None,
                       a_std: float = 0.1, b_std: float = 0.0316):
    """Attach trainable bf16 LoRA adapters to both expert projections.

    Parameters (per expert e): ``gate_up_proj_lora_A [E, r, H]``,
    ``gate_up_proj_lora_B [E, 2I, r]`` (rows in the interleaved gate/up order
    of the frozen weight), ``down_proj_lora_A [E, r, I]``,
    ``down_proj_lora_B [E, H, r]``.  Scaling ``lora_alpha / r``.
    ``init="peft"``: A kaiming-uniform(a=sqrt(5)), B = 0 (PEFT default);
    ``init="normal"``: A ~ N(0, a_std^2), B ~ N(0, b_std^2).
    """
    if r % 8 or r <= 0 or r > 64:
        raise ValueError("expert LoRA rank must be a positive multiple of 8, at most 64")
    dev = experts.gate_up_proj_bias.device
    E, H, I2 = experts.num_experts, experts.hidden_size, 2 * experts.intermediate_size
    I = experts.intermediate_size
    shapes = {"gate_up_proj_lora_A": (E, r, H), "gate_up_proj_lora_B": (E, I2, r),
              "down_proj_lora_A": (E, r, I), "down_proj_lora_B": (E, H, r)}
    for name, shp in shapes.items():
        t = torch.empty(shp, dtype=torch.float32)
        if name.endswith("_A"):
            if init == "peft":
                bound = 1.0 / math.sqrt(shp[-1])  # kaiming_uniform_(a=sqrt(5)) on [r, fan_in]
                t.uniform_(-bound, bound, generator=generator)
            else:
                t.normal_(0.0, a_std, generator=generator)
        else:
            if init == "peft":
                t.zero_()
            else:
                t.normal_(0.0, b_std, generator=generator)
        experts.register_parameter(name, nn.Parameter(t.to(device=dev, dtype=torch.bfloat16)))
    experts.expert_lora_r = r
    experts.expert_lora_scaling = float(lora_alpha) / r
    return experts


EXPERT_LORA_PARAMS = ("gate_up_proj_lora_A", "gate_up_proj_lora_B", "down_proj_lora_A", "down_proj_lora_B")


def _full(t):
    """The whole tensor of a (possibly FSDP2-sharded) parameter: DTensor.full_tensor() is a collective."""
    return t.full_tensor() if hasattr(t, "full_tensor") else t


def expert_lora_state_dict(model, to_cpu: bool = True) -> dict:
    """The expert-LoRA adapters of every experts module, for saving with the
    attention adapters.

    The reference saves adapters through PEFT (``get_peft_model_state_dict``,
    model_trainer.py:573, or ``save_pretrained``), which keeps only keys that
    name the adapter, so these parameters, registered on the experts module,
    would be left out.  Keys are the module path plus the parameter name, the
    form PEFT gives its own saved keys (adapter name removed); each module also
    stores ``<path>.expert_lora_scaling`` (lora_alpha / r) as a 0-d fp32 tensor.
    Merge the result into the adapter dict before writing it (safetensors /
    ``torch.save``); ``load_expert_lora_state_dict`` restores it.  Under FSDP2
    every rank must call this (``full_tensor`` is a collective)."""
    out = {}
    for name, mod in model.named_modules():
        if isinstance(mod, Mxfp4Bf16DequantGptOssExperts) and getattr(mod, "expert_lora_r", 0):
            for p in EXPERT_LORA_PARAMS:
                t = _full(getattr(mod, p)).detach()
                out[f"{name}.{p}"] = t.cpu().contiguous() if to_cpu else t
            out[f"{name}.expert_lora_scaling"] = torch.tensor(float(mod.expert_lora_scaling), dtype=torch.float32)
    return out


def load_expert_lora_state_dict(model, state_dict: dict, strict: bool = True) -> list:
    """Restore expert-LoRA adapters saved by ``expert_lora_state_dict``: each
    experts module whose path has adapters in ``state_dict`` gets expert LoRA
    at the saved rank and scaling (``enable_expert_lora`` if it has none yet)
    and the saved tensors copied in.  Keys may carry PEFT's
    ``base_model.model.`` prefix.  Returns the paths restored; with ``strict``
    a module path in the dict that the model does not have raises."""
    def strip(k):
        return k[len("base_model.model."):] if k.startswith("base_model.model.") else k
    sd = {strip(k): v for k, v in state_dict.items()}
    paths = sorted({k.rsplit(".", 1)[0] for k in sd if k.rsplit(".", 1)[-1] in EXPERT_LORA_PARAMS})
    modules = dict(model.named_modules())
    done = []
    for path in paths:
        mod = modules.get(path)
        if not isinstance(mod, Mxfp4Bf16DequantGptOssExperts):
            if strict:
                raise KeyError(f"{path}: no experts module at this path to load expert LoRA into")
            continue
        A = sd[f"{path}.gate_up_proj_lora_A"]
        r = A.shape[1]
        scaling = float(sd[f"{path}.expert_lora_scaling"]) if f"{path}.expert_lora_scaling" in sd else None
        if getattr(mod, "expert_lora_r", 0) != r:
            enable_expert_lora(mod, r=r, lora_alpha=(scaling if scaling is not None else 1.0) * r)
        elif scaling is not None:
            mod.expert_lora_scaling = scaling
        with torch.no_grad():
            for p in EXPERT_LORA_PARAMS:
                dst = getattr(mod, p)
                src = sd[f"{path}.{p}"]
                if tuple(src.shape) != tuple(dst.shape):
                    raise ValueError(f"{path}.{p}: saved shape {tuple(src.shape)}, module {tuple(dst.shape)}")
                dst.copy_(src.to(device=dst.device, dtype=dst.dtype))
        done.append(path)
    return done


def merge_expert_lora(experts: Mxfp4Bf16DequantGptOssExperts, proj: str, layout: str = "hf") -> torch.Tensor:
    """bf16 weight of ``proj`` with the expert LoRA folded in, for weight sync.

    ``W'[e] = bf16(float(deq(W[e])) + s * (B[e] @ A[e]))`` with fp32 base and
    delta — the arithmetic of the reference's LoRA merge
    (model_trainer.py:710-712) — in one HIP kernel over the packed weight.
    ``layout="hf"``: [E, K, N] as transformers' GptOssExperts holds
    ``gate_up_proj`` / ``down_proj``; ``"rows"``: [E, N, K].
    """
    if not experts.expert_lora_r:
        raise ValueError("the experts module has no expert LoRA (enable_expert_lora)")
    shapes = getattr(experts, f"_{proj}_shapes", None)
    blocks_p, scales_p = _full(getattr(experts, f"{proj}_blocks")), _full(getattr(experts, f"{proj}_scales"))
    if shapes is not None:
        blocks, scales = _unpack_bf16_as_uint8(blocks_p, shapes[0]), _unpack_bf16_as_uint8(scales_p, shapes[1])
    else:
        blocks, scales = blocks_p, scales_p
    A = _full(getattr(experts, f"{proj}_lora_A")).detach()
    B = _full(getattr(experts, f"{proj}_lora_B")).detach()
    with torch.no_grad():
        return kernels.mxfp4_lora_merge(blocks, scales, A, B, experts.expert_lora_scaling, layout)


def build_merged_expert_state_dict(model, to_cpu: bool = True) -> dict:
    """Merged expert weights of every experts module carrying expert LoRA.

    The expert-side counterpart of the reference's ``_build_merged_state_dict``
    (model_trainer.py:653-719) for sglang's ``update_weights_from_disk``: keys
    are the module path plus ``.gate_up_proj`` / ``.down_proj`` with PEFT's
    ``base_model.model.`` prefix removed (the names of a bf16 gpt-oss
    checkpoint), values [E, K, N] bf16.  Only the tensors the adapters change
    are included; biases stay as they are.
    """
    merged = {}
    for name, mod in model.named_modules():
        if not isinstance(mod, Mxfp4Bf16DequantGptOssExperts) or not mod.expert_lora_r:
            continue
        prefix = name.removeprefix("base_model.model.")
        for proj in ("gate_up_proj", "down_proj"):
            w = merge_expert_lora(mod, proj, "hf")
            merged[f"{prefix}.{proj}"] = w.cpu() if to_cpu else w
    return merged


# ---------------------------------------------------------------------------
# Routing entry points and the MLP forward
# ---------------------------------------------------------------------------

def routing_torch_dist(logits, n_expts_act):
    """Top-k routing under torch.distributed (quantization.py:551-590).

    Expert-parallel masking is not part of this single-GPU build: at world
    size 1 this is plain top-k routing.
    """
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized() and dist.get_world_size() > 1:
        raise NotImplementedError("expert-parallel routing (world size > 1) is not implemented")
    return routing(logits, n_expts_act)


def mlp_forward(self, hidden_states, router_indices=None):
    """MoE MLP forward with optional routing replay (quantization.py:639-668)."""
    import torch.distributed as dist
    if dist.is_available() and dist.is_initialized() and hasattr(self, "_is_hooked"):
        route = routing_torch_dist
    else:
        route = routing
    if router_indices is None:  # indices set by enable_routing_replay's decoder wrapper
        from .routing_replay import current_router_indices
        router_indices = current_router_indices(self)
    batch_size = hidden_states.shape[0]
    hidden_states = hidden_states.reshape(-1, self.router.hidden_dim)
    with on_device(hidden_states.device):
        # router GEMM on the HIP kernel (the reference's nn.functional.linear, quantization.py:654)
        router_logits = router_linear(hidden_states, self.router.weight, self.router.bias)
        if router_indices is not None:
            expt_indx = router_indices.reshape(-1, self.router.top_k).to(device=router_logits.device,
                                                                         dtype=torch.int32)
            routing_data, gather_idx, scatter_idx = routing_replay(router_logits, expt_indx, self.router.top_k)
        else:
            routing_data, gather_idx, scatter_idx = route(router_logits, self.router.top_k)
    routed_out = self.experts(hidden_states, routing_data, gather_idx, scatter_idx=scatter_idx)
    routed_out = routed_out.reshape(batch_size, -1, self.router.hidden_dim)
    return routed_out, router_logits


def replace_with_dequant_experts(model, quantization_config=None, modules_to_not_convert=None):
    """Swap GptOssExperts for the MXFP4 module and re-bind GptOssMLP.forward (quantization.py:675-699)."""
    if quantization_config is not None and getattr(quantization_config, "dequantize", False):
        return model
    dequant_dtype = getattr(quantization_config, "dequant_dtype", "bf16")
    model.config.dequant_dtype = dequant_dtype
    try:
        from transformers.quantizers.quantizers_utils import should_convert_module
    except ImportError:  # pragma: no cover - transformers always ships it
        def should_convert_module(name, patterns=None):
            return not patterns or not any(p in name for p in patterns)
    from types import MethodType
    replaced = False
    for module_name, module in list(model.named_modules()):
        if not should_convert_module(module_name, modules_to_not_convert):
            continue
        if module.__class__.__name__ == "GptOssExperts":
            with torch.device("meta"):
                model.set_submodule(module_name, Mxfp4Bf16DequantGptOssExperts(model.config))
            replaced = True
        if module.__class__.__name__ == "GptOssMLP":
            module.forward = MethodType(mlp_forward, module)
    if not replaced:
        import warnings
        warnings.warn("No expert modules found for MXFP4 dequant conversion.")
    return model


# ---------------------------------------------------------------------------
# transformers weight-loading conversions (quantization.py:175-221)
# ---------------------------------------------------------------------------
try:
    from transformers.core_model_loading import ConversionOps as _ConversionOps
    from transformers.quantizers.quantizers_utils import get_module_from_name as _get_module_from_name
except ImportError:  # pragma: no cover - only the HF loading integration needs these
    _ConversionOps = object
    _get_module_from_name = None


def _first(v):
    return v[0] if isinstance(v, list) else v


class Mxfp4Fp8DequantQuantize(_ConversionOps):
    """Quantize-on-load is not supported (checkpoints are pre-quantized)."""

    def __init__(self, hf_quantizer):
        self.hf_quantizer = hf_quantizer

    def convert(self, input_dict, model=None, missing_keys=None, full_layer_name=None, **kwargs):
        return {}


class Mxfp4Fp8DequantDequantize(_ConversionOps):
    """dequantize=True fallback: load the full bf16 weight ([E, K, N], transposed)."""

    def __init__(self, hf_quantizer):
        self.hf_quantizer = hf_quantizer

    def convert(self, input_dict, model=None, full_layer_name=None, missing_keys=None, **kwargs):
        blocks = _first(input_dict["_blocks"])
        scales = _first(input_dict["_scales"])
        return {full_layer_name: convert_moe_packed_tensors(blocks, scales)}


class Mxfp4Fp8DequantDeserialize(_ConversionOps):
    """Keep the checkpoint's MXFP4 blocks/scales as-is (bf16-container Parameters)."""

    def __init__(self, hf_quantizer):
        self.hf_quantizer = hf_quantizer

    def convert(self, input_dict, model=None, full_layer_name=None, missing_keys=None, **kwargs):
        blocks = _first(input_dict["_blocks"])
        scales = _first(input_dict["_scales"])
        module, _ = _get_module_from_name(model, full_layer_name)
        proj = "gate_up_proj" if "gate_up_proj" in full_layer_name else "down_proj"
        _store_mxfp4_weights(blocks, scales, module, proj, blocks.device)
        if missing_keys is not None:
            missing_keys.discard(f"{full_layer_name}")
        module._is_hf_initialized = True
        return {}
