"""fp8 mode of the expert path restated on the CPU (test infrastructure only).

* ``nibble_to_e5m2`` / ``e5m2_rows`` / ``e5m2_colmajor`` — the int32 rule of
  kernels.py:20-37 (_convert_nibble_to_fp8, exponent field ee + S - 113) with
  the two output layouts of kernels.py:52-108 (row-major: the uint16
  ``lo | hi << 8`` stores of 80-84) and kernels.py:238-312 (column-major
  [E, K, N], one byte per store).  Both reproduce what the reference stores
  for scale bytes whose exponent leaves E5M2 (S > 140: the exponent field
  spills past 8 bits and is truncated the way each store truncates).
* ``f32_to_e4m3`` — fp32 -> fp8 E4M3FN, round to nearest even, saturating at
  +-448 (the conversion at kernels.py:383 for the values it receives).
* ``quantize_per_token`` — kernels.py:343-388: per-row amax, scale =
  max(amax, 1e-12) / 448, codes = E4M3(x * (1 / scale)), in float32 with
  IEEE division.
* ``e4m3_to_f32`` / ``e5m2_to_f32`` — the value of a code (for checks).

Pinning (tests/test_oracle_fp8.py): in-format E5M2 codes decode to the MXFP4
values of oracle/mxfp4.py, the two layouts agree, E4M3 rounding equals torch's
float8_e4m3fn cast below 464.  Parity unpinned: the out-of-format E5M2 bytes
(S > 140; restated from the reference's expression only) and the last ulp of
the scale and its reciprocal (the reference divides with Triton's fp32 division
on its own GPU, this restatement with IEEE division).
"""
from __future__ import annotations

import numpy as np


def nibble_to_e5m2(nib, scale):
    """kernels.py:21-37 in int32 (numpy int64 here), returned untruncated."""
    nib = np.asarray(nib, dtype=np.int64)
    scale_adj = np.asarray(scale, dtype=np.int64) - 113
    sign = (nib >> 3) & 1
    ee = (nib >> 1) & 3
    m = nib & 1
    n_abs = nib & 7
    exp = ee + scale_adj
    mant = np.where(ee > 0, m << 1, 0)
    result = (sign << 7) | (exp << 2) | mant
    result = np.where(n_abs == 0, sign << 7, result)
    result = np.where((n_abs > 0) & (exp < 1), sign << 7, result)
    return result


def e5m2_rows(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """blocks [..., G, 16] u8, scales [..., G] u8 -> [..., G*32] u8 (kernels.py:52-108)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    lo = nibble_to_e5m2(blocks & 0xF, scales[..., None])
    hi = nibble_to_e5m2(blocks >> 4, scales[..., None])
    combined = ((lo | (hi << 8)) & 0xFFFF).astype(np.uint16)       # .to(tl.uint16), little-endian bytes
    out = np.empty(blocks.shape[:-1] + (32,), dtype=np.uint8)
    out[..., 0::2] = (combined & 0xFF).astype(np.uint8)
    out[..., 1::2] = (combined >> 8).astype(np.uint8)
    return out.reshape(blocks.shape[:-2] + (blocks.shape[-2] * 32,))


def e5m2_colmajor(blocks: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """blocks [E, N, G, 16], scales [E, N, G] -> [E, G*32, N] u8 (kernels.py:262-285)."""
    blocks = np.asarray(blocks, dtype=np.uint8)
    scales = np.asarray(scales, dtype=np.uint8)
    E, N, G, _ = blocks.shape
    lo = nibble_to_e5m2(blocks & 0xF, scales[..., None]) & 0xFF    # .to(tl.uint8) per value
    hi = nibble_to_e5m2(blocks >> 4, scales[..., None]) & 0xFF
    vals = np.empty((E, N, G, 32), dtype=np.uint8)
    vals[..., 0::2] = lo
    vals[..., 1::2] = hi
    return np.ascontiguousarray(vals.reshape(E, N, G * 32).transpose(0, 2, 1))


def e5m2_to_f32(code) -> np.ndarray:
    """Value of E5M2 codes (bias 15; exponent 31 = inf / NaN)."""
    c = np.asarray(code, dtype=np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    ex = (c >> 2) & 0x1F
    m = c & 3
    val = np.where(ex == 0, m / 4.0 * 2.0 ** -14, (1 + m / 4.0) * 2.0 ** (ex - 15.0))
    val = np.where(ex == 31, np.where(m == 0, np.inf, np.nan), val)
    return (sign * val).astype(np.float64)


def e4m3_to_f32(code) -> np.ndarray:
    """Value of E4M3FN codes (bias 7, no infinities, 0x7F / 0xFF = NaN)."""
    c = np.asarray(code, dtype=np.int64)
    sign = np.where(c & 0x80, -1.0, 1.0)
    ex = (c >> 3) & 0xF
    m = c & 7
    val = np.where(ex == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (ex - 7.0))
    val = np.where((ex == 15) & (m == 7), np.nan, val)
    return (sign * val).astype(np.float64)


def f32_to_e4m3(v) -> np.ndarray:
    """float32 -> E4M3FN codes: round to nearest even, |v| >= 464 (incl. inf) -> +-448, NaN -> 0x7F."""
    v = np.asarray(v, dtype=np.float32)
    u = v.view(np.uint32).astype(np.int64)
    sign = (u >> 24) & 0x80
    a = u & 0x7FFFFFFF
    # normal range [2^-6, 464): drop 20 mantissa bits of the pattern with round-to-nearest-even, rebias 127 -> 7
    r = ((a + 0x7FFFF + ((a >> 20) & 1)) >> 20) - (120 << 3)
    # below 2^-6: multiples of 2^-9 (0..8; 8 is the smallest normal 0x08)
    small = np.minimum(np.nan_to_num(np.abs(v.astype(np.float64)), nan=0.0, posinf=1.0), 1.0)
    sub = np.rint(small * 512.0).astype(np.int64)
    code = np.where(a < 0x3C800000, sub, r)
    code = np.where(a >= 0x43E80000, 0x7E, code)
    code = np.where(a > 0x7F800000, 0x7F, code)
    return (sign | code).astype(np.uint8)


def quantize_per_token(x: np.ndarray):
    """x [M, K] (bf16 values as float32) -> (codes [M, K] u8, scale [M] f32)  (kernels.py:343-388)."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.abs(x).max(axis=1) if x.shape[1] else np.zeros(x.shape[0], np.float32)
    scale = (np.maximum(amax, np.float32(1e-12)) / np.float32(448.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    codes = f32_to_e4m3((x * inv[:, None]).astype(np.float32))
    return codes, scale
