"""Pins oracle.mxfp4 (CPU): exhaustive table, LUT+ldexp cross-check, layout."""
import numpy as np
import torch
from pathlib import Path

from oracle import mxfp4

GOLDEN = Path(__file__).parent / "golden" / "mxfp4_table.npy"


def test_exhaustive_table_matches_golden():
    assert (mxfp4.exhaustive_table() == np.load(GOLDEN, allow_pickle=False)).all()


def test_bit_formula_equals_lut_ldexp_in_normal_scale_range():
    # all 16 codes x scales 2..252, where both reference forms are defined identically
    s = np.arange(2, 253, dtype=np.uint8)
    blocks = np.tile(np.arange(256, dtype=np.uint8), (s.size, 1)).reshape(s.size, 16, 16)  # [S, G=16, 16]
    scales = np.repeat(s[:, None], 16, axis=1)
    a = mxfp4.dequant_bits(blocks, scales)
    b = mxfp4.dequant_lut_ldexp(torch.from_numpy(blocks), torch.from_numpy(scales))
    assert (a == b.view(torch.int16).numpy().view(np.uint16)).all()


def test_flush_rules_outside_normal_range():
    t = mxfp4.exhaustive_table()
    # S = 0: every non-zero code would need exponent <= 1 -> codes 1 (0.5) and 2,3 (1, 1.5 -> exp 0) flush
    assert t[0, 1] == 0 and t[0, 9] == 0x8000
    # S = 255: 6.0 * 2^128 overflows -> signed zero, not inf
    assert t[255, 7] == 0 and t[255, 15] == 0x8000
    # -0 keeps its sign at every scale
    assert (t[:, 8] == 0x8000).all() and (t[:, 0] == 0).all()


def test_values_match_exact_arithmetic():
    t = mxfp4.exhaustive_table()
    for s in (118, 124, 127, 130):
        for code in range(16):
            assert mxfp4.bits_to_f32(t[s, code]) == np.float32(mxfp4.exact_value(code, s))


def test_layout_low_nibble_first():
    blocks = np.zeros((1, 16), dtype=np.uint8)
    blocks[0, 3] = 0x72          # low nibble 2 (1.0) -> element 6, high nibble 7 (6.0) -> element 7
    scales = np.array([127], dtype=np.uint8)
    out = mxfp4.bits_to_f32(mxfp4.dequant_bits(blocks, scales))
    assert out[6] == 1.0 and out[7] == 6.0 and np.count_nonzero(out) == 2
