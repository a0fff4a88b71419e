"""MXFP4 -> bf16 dequant restated on the CPU (test infrastructure only).

Two independent restatements:

* ``nibble_to_bf16_bits`` / ``dequant_bits`` — the integer bit assembly of
  kernels.py:120-158 (_convert_nibble_to_bf16) with the block layout of
  kernels.py:189-200 (byte j -> elements 2j (low nibble), 2j+1 (high nibble)).
* ``dequant_lut_ldexp`` — the transformers-style LUT + ldexp form of
  quantization.py:102-122 (_mxfp4_to_bf16_pytorch) / 137-163.

They agree bit for bit for scale bytes S in [2, 252]; outside it the Triton
form flushes to signed zero (exponent < 1 or > 254) while ldexp yields bf16
subnormals / inf.  The product kernel follows the Triton form everywhere.
"""
from __future__ import annotations

import numpy as np
import torch

# kernels.py / quantization.py:131-134 — e2m1 code -> value
FP4_VALUES = [+0.0, +0.5, +1.0, +1.5, +2.0, +3.0, +4.0, +6.0,
              -0.0, -0.5, -1.0, -1.5, -2.0, -3.0, -4.0, -6.0]


def nibble_to_bf16_bits(nib, scale):
    """kernels.py:137-158, vectorised over numpy int arrays; returns uint16 bits."""
    nib = np.asarray(nib, dtype=np.int64)
    scale = np.asarray(scale, dtype=np.int64)
    sign = (nib >> 3) & 1
    ee = (nib >> 1) & 3
    m = nib & 1
    n_abs = nib & 7
    exp = np.where(ee > 0, ee - 1 + scale, scale - 1)
    mant = np.where(ee > 0, m << 6, 0)
    result = (sign << 15) | (exp << 7) | mant
    result = np.where(n_abs == 0, sign << 15, result)
    result = np.where((n_abs > 0) & (exp > 254), sign << 15, result)
    result = np.where((n_abs > 0) & (exp < 1), sign << 15, result)
    return (result & 0xFFFF).astype(np.uint16)


def dequant_bits(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """blocks [..., G, 16] u8, scales [..., G] u8 -> bf16 bits [..., G*32] u16 (kernels.py:189-200)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    lo = nibble_to_bf16_bits(blocks & 0xF, scales[..., None])
    hi = nibble_to_bf16_bits(blocks >> 4, scales[..., None])
    out = np.empty(blocks.shape[:-1] + (32,), dtype=np.uint16)
    out[..., 0::2] = lo
    out[..., 1::2] = hi
    return out.reshape(blocks.shape[:-2] + (blocks.shape[-2] * 32,))


def dequant_lut_ldexp(blocks: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """quantization.py:102-122: LUT of e2m1 values, then ldexp by (S - 127), in bf16."""
    lut = torch.tensor(FP4_VALUES, dtype=torch.bfloat16)
    prefix = blocks.shape[:-2]
    G, B = blocks.shape[-2], blocks.shape[-1]
    blk = blocks.to(torch.uint8)
    exp = (scales.to(torch.int32) - 127).unsqueeze(-1)
    out = torch.empty(*prefix, G, B * 2, dtype=torch.bfloat16)
    out[..., 0::2] = lut[(blk & 0x0F).long()]
    out[..., 1::2] = lut[(blk >> 4).long()]
    torch.ldexp(out, exp.expand_as(out), out=out)
    return out.reshape(*prefix, G * B * 2)


def exact_value(nib: int, scale: int) -> float:
    """Mathematical value of one e2m1 code times 2^(S-127) (float64, exact)."""
    return float(np.ldexp(FP4_VALUES[nib], scale - 127))


def bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)


def exhaustive_table() -> np.ndarray:
    """[256 scales, 16 nibbles] uint16 bf16 bits of the Triton rule."""
    s = np.arange(256)[:, None]
    n = np.arange(16)[None, :]
    return nibble_to_bf16_bits(n, s)


def dequant_f32(blocks, scales) -> torch.Tensor:
    """float32 weight [..., G*32] from MXFP4 (via the bit formula)."""
    b = blocks.numpy() if isinstance(blocks, torch.Tensor) else blocks
    s = scales.numpy() if isinstance(scales, torch.Tensor) else scales
    return torch.from_numpy(bits_to_f32(dequant_bits(b, s)).copy())


_TABLE_F32 = None


def dequant_f32_table(blocks, scales) -> torch.Tensor:
    """float32 weight [..., G*32]: the values of ``dequant_f32`` looked up in the
    exhaustive [256 scales x 16 nibbles] table of ``nibble_to_bf16_bits``
    (same rule and layout, fast enough for whole experts at gpt-oss size)."""
    global _TABLE_F32
    if _TABLE_F32 is None:
        _TABLE_F32 = torch.from_numpy(bits_to_f32(exhaustive_table()).reshape(-1).copy())
    b = torch.as_tensor(blocks).to(torch.int64)
    s = torch.as_tensor(scales).to(torch.int64).unsqueeze(-1) * 16
    out = torch.empty(*b.shape, 2, dtype=torch.float32)
    out[..., 0] = _TABLE_F32[s + (b & 15)]
    out[..., 1] = _TABLE_F32[s + (b >> 4)]
    return out.reshape(*b.shape[:-2], b.shape[-2] * 32)
