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


def _f32_bits(t):
    return t.contiguous().view(torch.int32).numpy()


def test_table_dequant_equals_bit_formula_for_every_byte_and_scale():
    """dequant_f32_table (the fast lookup the full-size GPU checks use) against
    dequant_f32 (the bit formula) and against the golden table (float64 MX
    arithmetic), for all 256 packed bytes under all 256 scale bytes."""
    blocks = np.tile(np.arange(256, dtype=np.uint8), (256, 1)).reshape(256, 16, 16)  # [S, G=16, 16]
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 16, axis=1)
    fast = mxfp4.dequant_f32_table(torch.from_numpy(blocks), torch.from_numpy(scales))
    slow = mxfp4.dequant_f32(blocks, scales)
    assert fast.shape == (256, 512) and (_f32_bits(fast) == _f32_bits(slow)).all()
    gold = np.load(GOLDEN, allow_pickle=False).astype(np.uint32)          # [scale, nibble] bf16 bits
    b = blocks.reshape(256, 256).astype(np.int64)
    s = np.arange(256)[:, None]
    want = np.empty((256, 512), dtype=np.uint32)
    want[:, 0::2] = gold[s, b & 15]
    want[:, 1::2] = gold[s, b >> 4]
    assert (_f32_bits(fast).view(np.uint32) == want << 16).all()


def test_table_dequant_equals_bit_formula_on_random_expert_weights():
    g = torch.Generator().manual_seed(31)
    blocks = torch.randint(0, 256, (3, 40, 5, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(0, 256, (3, 40, 5), generator=g, dtype=torch.uint8)
    fast = mxfp4.dequant_f32_table(blocks, scales)
    assert fast.shape == (3, 40, 160)
    assert (_f32_bits(fast) == _f32_bits(mxfp4.dequant_f32(blocks, scales))).all()
    # one expert's slice (how the full-size checks call it) is the same slice of the whole
    assert (_f32_bits(mxfp4.dequant_f32_table(blocks[1], scales[1])) == _f32_bits(fast[1])).all()
