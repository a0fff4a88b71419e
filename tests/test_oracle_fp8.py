"""The fp8-mode oracle (oracle/fp8.py) against independent references:
E5M2 codes decode to exactly the MXFP4 values wherever they fit the format,
the row- and column-major layouts agree, E4M3 rounding matches torch's
float8_e4m3fn conversion, and per-token quantization meets its error bound
with each row's largest magnitude mapped to 448."""
import numpy as np
import torch

from oracle import fp8, mxfp4

NIB = np.arange(16)[:, None]
SC = np.arange(256)[None, :]


def test_e5m2_values_are_the_mxfp4_values_in_format():
    code = fp8.nibble_to_e5m2(NIB, SC)
    val = fp8.e5m2_to_f32(code & 0xFF)
    want = np.array(mxfp4.FP4_VALUES)[:, None] * 2.0 ** (SC - 127.0)
    # every (nibble, scale) whose E5M2 exponent field is in 1..30, or whose value is 0
    ee = (NIB >> 1) & 3
    exp = ee + SC - 113
    inside = ((exp >= 1) & (exp <= 30)) | ((NIB & 7) == 0)
    assert np.array_equal(val[inside], want[inside])
    # signs survive, also on zeros
    assert np.array_equal((code[inside] >> 7) & 1, np.broadcast_to(NIB >> 3, code.shape)[inside])
    # exponent below the format: flushed to a signed zero (the reference does not round to E5M2 subnormals)
    below = (exp < 1) & ((NIB & 7) != 0)
    assert below.any() and np.all((code[below] & 0x7F) == 0)
    # in-format rows for the BASELINE scale range 118..130: everything
    assert inside[:, 118:131].all()


def test_e5m2_row_and_column_layouts_agree():
    g = np.random.default_rng(0)
    blocks = g.integers(0, 256, (3, 40, 5, 16), dtype=np.uint8)
    scales = g.integers(100, 141, (3, 40, 5), dtype=np.uint8)
    rows = fp8.e5m2_rows(blocks, scales)            # [E, N, K]
    cols = fp8.e5m2_colmajor(blocks, scales)        # [E, K, N]
    assert np.array_equal(rows.transpose(0, 2, 1), cols)
    # byte 2j / 2j+1 of a group hold the low / high nibble of block byte j
    lo = fp8.nibble_to_e5m2(blocks[0, 0, 0] & 0xF, scales[0, 0, 0])
    assert np.array_equal(rows[0, 0, 0:32:2], lo.astype(np.uint8))


def test_e5m2_packing_outside_the_format():
    # S = 200: exponent field 87..90 spills past 8 bits; the row-major store keeps
    # (lo | hi << 8) & 0xFFFF, the column-major store each value's low byte
    b = np.array([[[0x53] + [0] * 15]], dtype=np.uint8)       # lo nibble 3 (1.5), hi nibble 5 (3.0)
    s = np.array([[200]], dtype=np.uint8)
    lo = (0 << 7) | ((1 + 200 - 113) << 2) | 2
    hi = (0 << 7) | ((2 + 200 - 113) << 2) | 2
    row = fp8.e5m2_rows(b, s)[0, :2]
    assert row[0] == ((lo | hi << 8) & 0xFF) and row[1] == (((lo | hi << 8) >> 8) & 0xFF)
    col = fp8.e5m2_colmajor(b[None], s[None])[0, :2, 0]
    assert col[0] == (lo & 0xFF) and col[1] == (hi & 0xFF)


def test_e4m3_rounding_matches_torch():
    g = np.random.default_rng(1)
    parts = [g.uniform(-463.9, 463.9, 20000), g.uniform(-0.05, 0.05, 20000), g.normal(0, 1, 20000),
             g.uniform(-2 ** -6, 2 ** -6, 20000)]
    # exact ties between neighbouring codes (round to even) and the subnormal / normal edge
    codes = np.arange(0, 0x7E)
    v = fp8.e4m3_to_f32(codes)
    mids = (v[:-1] + v[1:]) / 2
    parts += [mids, -mids, v, np.array([2 ** -6, 2 ** -7, 2 ** -9, 2 ** -10, 3 * 2 ** -11, 0.0, -0.0])]
    x = np.concatenate(parts).astype(np.float32)
    ours = fp8.f32_to_e4m3(x)
    theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def test_e4m3_saturation_and_nan():
    x = np.array([448.0, 463.99, 464.0, 1e6, np.inf, -np.inf, -500.0, np.nan], dtype=np.float32)
    assert fp8.f32_to_e4m3(x).tolist() == [0x7E, 0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE, 0x7F]


def test_quantize_per_token_bounds():
    g = torch.Generator().manual_seed(2)
    x = (torch.randn(64, 300, generator=g) * torch.logspace(-3, 3, 64)[:, None]).to(torch.bfloat16)
    x[5] = 0
    xf = x.float().numpy()
    codes, scale = fp8.quantize_per_token(xf)
    amax = np.abs(xf).max(axis=1)
    assert np.array_equal(scale, (np.maximum(amax, np.float32(1e-12)) / np.float32(448)).astype(np.float32))
    dec = fp8.e4m3_to_f32(codes) * scale[:, None]
    err = np.abs(dec - xf)
    # half an E4M3 step: 2^-4 relative for normals, 2^-10 * scale absolute for subnormals
    assert np.all(err <= np.maximum(np.abs(xf) * 2.0 ** -4, 2.0 ** -10 * scale[:, None]) * (1 + 1e-6))
    nz = amax > 0
    assert np.all(np.abs(fp8.e4m3_to_f32(codes[nz])).max(axis=1) == 448.0)
    assert np.all(codes[5] == 0)
