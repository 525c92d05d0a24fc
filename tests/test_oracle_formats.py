"""Pins the format oracle (oracle/formats.py, oracle/c/oracle.c) — CPU only.

Known-answer vectors come from the reference's Swift tests
(Tests/DeepSeekRepackTests/DeepSeekRepackTests.swift:336-412), kept as data in
tests/golden/reference_kats.json; the rest are closed forms and an independent
library decoder (torch.float8_e4m3fn).
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import formats as F
from oracle import c_oracle as C


def _bf16_bits(values):
    return (np.asarray(values, np.float32).view(np.uint32) >> 16).astype(np.uint16)


KATS = json.loads((Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def _kat4_source():
    idx = np.arange(128 * 128)
    v = ((idx * 37 + 11) & 0xFF).astype(np.uint8)
    return np.where((v & 0x7F) == 0x7F, v ^ 1, v).astype(np.uint8)


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_kat_fixed_vector(impl):
    kat = KATS["mxfp4_fixed_vector"]
    q = F.quantize_mxfp4_bf16 if impl == "numpy" else C.quantize_bf16
    w, s = q(_bf16_bits(kat["values"]), kat["rows"], kat["columns"])
    assert list(w.ravel()) == kat["weights"]
    assert list(s.ravel()) == kat["scales"]


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_kat_bf16_rows(impl):
    kat = KATS["mxfp4_bf16_rows"]
    q = F.quantize_mxfp4_bf16 if impl == "numpy" else C.quantize_bf16
    w, s = q(np.array(kat["bf16_bits"], np.uint16), kat["rows"], kat["columns"])
    assert list(w.ravel()) == kat["weights"]
    assert list(s.ravel()) == kat["scales"]


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_kat_official_fp8_blocks(impl):
    kat = KATS["fp8_official_blocks"]
    first = kat["first_bytes"]
    src = np.array(first + [0] * (kat["rows"] * kat["columns"] - len(first)), np.uint8)
    q = F.quantize_mxfp4_fp8 if impl == "numpy" else C.quantize_fp8
    w, s = q(src, np.array([kat["inverse_scale_bf16"]], np.uint16), kat["rows"], kat["columns"])
    assert list(w.ravel()[:16]) == kat["weights_head"]
    assert list(s.ravel()[:4]) == kat["scales_head"]


@pytest.mark.parametrize("impl", ["numpy", "c"])
def test_kat_fp8_sha256(impl):
    # Pins e4m3 decode, x scale, bf16 RNE and the encoder end to end.
    kat = KATS["fp8_pattern_sha256"]
    q = F.quantize_mxfp4_fp8 if impl == "numpy" else C.quantize_fp8
    w, s = q(_kat4_source(), np.array([kat["inverse_scale_bf16"]], np.uint16), kat["rows"], kat["columns"])
    assert hashlib.sha256(w.tobytes()).hexdigest() == kat["weights_sha256"]
    assert hashlib.sha256(s.tobytes()).hexdigest() == kat["scales_sha256"]


def test_encoders_reject_incomplete_plans():
    with pytest.raises(ValueError):
        F.quantize_mxfp4_bf16(np.zeros(31, np.uint16), 1, 31)
    with pytest.raises(ValueError):
        F.quantize_mxfp4_fp8(np.zeros(64 * 128, np.uint8), np.zeros(1, np.uint16), 64, 128)


def test_numpy_and_c_encoders_agree_on_random_rows():
    rng = np.random.default_rng(5)
    for scale in (1e-3, 1.0, 300.0):
        bits = _bf16_bits(rng.standard_normal((16, 256)).astype(np.float32) * scale)
        a = F.quantize_mxfp4_bf16(bits, 16, 256)
        b = C.quantize_bf16(bits, 16, 256)
        np.testing.assert_array_equal(a[0], b[0])
        np.testing.assert_array_equal(a[1], b[1])


def test_e2m1_e8m0_closed_form_every_code_and_scale():
    # Every (scale byte, code) pair: value = sign * magnitude * 2**(b - 127); 255 is NaN.
    codes = np.arange(16, dtype=np.uint8)
    words = np.zeros((256, 4), np.uint32)
    for j in range(4):
        words[:, j] = sum(((int(codes[(2 * j * 4 + n) % 16])) << (4 * n)) for n in range(8))
    packed = np.tile(words, (1, 1))  # [256, 4] -> 32 values per row, codes cycling
    scales = np.arange(256, dtype=np.uint8).reshape(256, 1)
    got = F.dequant_mxfp4(packed, scales)
    mags = [0, 0.5, 1, 1.5, 2, 3, 4, 6]
    for b in range(256):
        for i in range(32):
            code = (int(packed[b, i // 8]) >> (4 * (i % 8))) & 15
            m = mags[code & 7] * (-1 if code & 8 else 1)
            want = np.nan if b == 255 else np.float32(m) * np.float32(2.0 ** (b - 127))
            if b == 255:
                assert np.isnan(got[b, i])
            else:
                assert got[b, i] == want, (b, i, code)
    np.testing.assert_array_equal(got, C.dequant_mxfp4(packed, scales))


def test_mxfp4_round_trip_on_exact_values():
    # Values already on the MXFP4 grid encode and decode to themselves.
    rng = np.random.default_rng(9)
    codes = rng.integers(0, 16, size=(8, 64)).astype(np.uint8)
    codes[:, ::32] = 7  # each group holds +6, so the encoder picks exponent(6) - 2 = 0 relative
    exps = rng.integers(-8, 3, size=(8, 2))
    vals = F.e2m1_value(codes).reshape(8, 2, 32) * (2.0 ** exps)[..., None]
    vals = vals.reshape(8, 64).astype(np.float32)
    w, s = F.quantize_mxfp4_bf16(F.bf16_round(vals), 8, 64)
    back = F.dequant_mxfp4(np.ascontiguousarray(w).view(np.uint32), s)
    np.testing.assert_array_equal(back, vals)


def test_e4m3_matches_torch_float8_every_byte():
    b = np.arange(256, dtype=np.uint8)
    ours = F.e4m3_value(b)
    theirs = torch.from_numpy(b).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(theirs)
    assert list(np.flatnonzero(nan)) == [0x7F, 0xFF]
    np.testing.assert_array_equal(np.isnan(ours), nan)
    np.testing.assert_array_equal(ours[~nan], theirs[~nan])
    c = np.array([C.e4m3(int(v)) for v in b], np.float32)
    np.testing.assert_array_equal(c[~nan], theirs[~nan])


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 10000),
                        np.array([0.0, -0.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8], np.float32)]).astype(np.float32)
    ours = F.bf16_round(v)
    theirs = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(ours, theirs)


def test_fp8_blocks_crop_and_reject():
    rng = np.random.default_rng(1)
    w = rng.integers(0, 256, size=(130, 200)).astype(np.uint8)
    w = np.where((w & 0x7F) == 0x7F, w ^ 1, w).astype(np.uint8)
    s = rng.random((2, 2)).astype(np.float32)
    out = F.dequant_fp8_blocks(w, s)
    assert out.shape == (130, 200)
    # Ragged edge: row 129 / column 199 use block (1, 1).
    assert out[129, 199] == F.e4m3_value(w[129, 199]) * s[1, 1]
    assert out[127, 127] == F.e4m3_value(w[127, 127]) * s[0, 0]
    assert out[128, 5] == F.e4m3_value(w[128, 5]) * s[1, 0]
    bad = w.copy()
    bad[3, 3] = 0x7F
    with pytest.raises(ValueError):
        F.dequant_fp8_blocks(bad, s)
    with pytest.raises(ValueError):
        F.dequant_fp8_blocks(w, np.array([[1, -1], [1, 1]], np.float32))
    with pytest.raises(ValueError):
        F.dequant_fp8_blocks(w, np.ones((1, 2), np.float32))
    with pytest.raises(ValueError):
        F.dequant_fp8_blocks(w, s.astype(np.float64))


# ---- E2M3 activation terms of the prefill GEMMs -------------------------------------------

def test_e2m3_is_the_ocp_format():
    # OCP MX v1.0 E2M3: 1 sign, 2 exponent (bias 1), 3 mantissa bits, no inf / NaN. Checked
    # through its shape, not its formula: 8 values per binade, the spacing of each binade,
    # subnormals down to 1/8, maximum 7.5, and the sign bit negating.
    m = F.E2M3_MAGNITUDES.astype(np.float64)
    assert m[0] == 0 and np.all(np.diff(m) > 0) and m[-1] == 7.5
    spacing = np.diff(m)
    assert np.all(spacing[:16] == 0.125)          # up to 2: subnormals and the first binade
    assert np.all(spacing[16:24] == 0.25)         # [2, 4]
    assert np.all(spacing[24:] == 0.5)            # [4, 7.5]
    assert list(m[[8, 16, 24]]) == [1.0, 2.0, 4.0]
    np.testing.assert_array_equal(F.e2m3_value(np.arange(32) | 32), -F.E2M3_MAGNITUDES)


def test_e2m3_encode_is_nearest_with_ties_to_even_and_saturates():
    rng = np.random.default_rng(3)
    v = np.concatenate([rng.uniform(-9, 9, 20000), (F.E2M3_MAGNITUDES[1:] + F.E2M3_MAGNITUDES[:-1]) / 2,
                        -(F.E2M3_MAGNITUDES[1:] + F.E2M3_MAGNITUDES[:-1]) / 2, [7.74, 7.76, 100.0, -0.0, -0.01]])
    codes = F.e2m3_encode(v)
    got = np.abs(F.e2m3_value(codes).astype(np.float64))
    a = np.minimum(np.abs(v), 7.5)
    dist = np.abs(a[:, None] - F.E2M3_MAGNITUDES[None, :].astype(np.float64))
    assert np.all(np.abs(a - got) == dist.min(1))                       # a nearest value
    mid = np.isin(np.abs(v), (F.E2M3_MAGNITUDES[1:] + F.E2M3_MAGNITUDES[:-1]) / 2)
    assert np.all((codes[mid] & 1) == 0)                                 # ties to the even code
    assert F.e2m3_value(F.e2m3_encode(np.array([100.0])))[0] == 7.5        # saturation
    assert np.all((codes & 32) == np.where(np.signbit(v), 32, 0))        # the sign always kept
    np.testing.assert_array_equal(F.e2m3_encode(F.e2m3_value(np.arange(64))), np.arange(64))


def test_split_rows_reconstruct_within_a_256th_of_the_block_maximum():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((6, 256)) * np.exp2(rng.integers(-30, 30, (6, 1)))).astype(np.float32)
    x[1, :32] = 0.0
    rec = F.split_rows_value(F.split_rows_e2m3(x), 256)
    for r in range(6):
        for b in range(8):
            blk = x[r, 32 * b:32 * b + 32].astype(np.float64)
            err = np.abs(rec[r, 32 * b:32 * b + 32] - blk).max()
            assert err <= np.abs(blk).max() / 256.0
    # a single term would miss by up to 1/16 of the block maximum: the lo term carries weight
    one = F.split_rows_e2m3(x)
    one[:, :, 24:48] = one[:, :, 72:96] = one[:, :, 120:144] = one[:, :, 168:192] = 0
    assert np.abs(F.split_rows_value(one, 256) - x).max() > np.abs(x).max() / 256.0


def test_split_rows_exact_and_zero_blocks():
    # values on the E2M3 grid at the block's scale are the hi term alone (lo fields 0)
    blk = np.concatenate([F.E2M3_MAGNITUDES[16:], -F.E2M3_MAGNITUDES[16:]]) * np.float32(2.0 ** -3)
    x = np.zeros((1, 128), np.float32)
    x[0, :32] = blk
    s = F.split_rows_e2m3(x)[0, 0]
    hi, lo, s_hi, s_lo = F.e2m3_terms(blk)
    assert s_hi == 127 - 3 and s_lo == 1 and not np.any(lo & 31)
    np.testing.assert_array_equal(F.e2m3_value(hi) * np.float32(2.0 ** -3), blk)
    assert list(s[192:200]) == [124, 1, 1, 1, 1, 1, 1, 1] and not np.any(s[48:192])   # zero blocks: exponent 1


def test_fp8_e8m0_dequant_closed_form_and_crop():
    """dequant_fp8 of the V4.1 release (deepseek_v41/dequant.py:45-50): every E4M3 value (torch's
    float8_e4m3fn decoder, independent of the oracle's table) times 2^(b - 127) of its 32 x 32
    block, computed in float64, with the ceil overhang of ragged edges cropped (:39-42); the
    products are exact, so the comparison is equality."""
    rng = np.random.default_rng(3)
    rows, cols = 70, 100
    w = rng.integers(0, 256, size=(rows, cols), dtype=np.uint8)
    w[(w & 127) == 127] = 0                       # reserved NaN codes
    s = rng.integers(100, 155, size=(3, 4), dtype=np.uint8)
    s[0, 0], s[2, 3] = 1, 254
    out = F.dequant_fp8_e8m0(w, s)
    vals = torch.from_numpy(w).view(torch.float8_e4m3fn).to(torch.float64).numpy()
    r, c = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    want = vals * np.exp2(s[r // 32, c // 32].astype(np.float64) - 127)
    assert out.dtype == np.float32
    np.testing.assert_array_equal(out.astype(np.float64), want.astype(np.float32).astype(np.float64))
    assert out[69, 99] == F.e4m3_value(w[69, 99]) * np.float32(2.0 ** (int(s[2, 3]) - 127))
    with pytest.raises(ValueError):
        F.dequant_fp8_e8m0(w, s[:2])


def test_e4m3_encode_matches_torch_rounding():
    """The oracle's E4M3 encoder (nearest, ties to the even code, signed zero) against torch's
    float8_e4m3fn conversion, over a wide sample, every representable value, every midpoint
    between neighbours (the ties) and tiny negatives."""
    rng = np.random.default_rng(9)
    grid = F.e4m3_value(np.arange(127, dtype=np.uint8)).astype(np.float64)
    mids = (grid[:-1] + grid[1:]) / 2
    v = np.concatenate([rng.standard_normal(50000) * 60, grid, -grid, mids, -mids, -rng.random(500) * 1e-4,
                        [0.0, -0.0, 448.0, -448.0]]).astype(np.float32)
    got = F.e4m3_encode(v)
    want = torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(got, want)


def test_split_rows_e4m3_is_bf16_exact():
    """Two E4M3 terms per 32-value block reproduce every bf16 value at or above 2^-13 of the
    block's maximum exactly (hi: the top 4 significant bits, lo: the residual times 16), over
    rows whose blocks span many binades; the hi scale puts the block maximum in [128, 256)."""
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((6, 512)) * np.exp2(rng.integers(-30, 30, (6, 16))).repeat(32, axis=1)).astype(np.float32)
    x[0, :32] = 0.0
    xb = F.bf16_round_f32(x).astype(np.float64)
    terms, scales = F.split_rows_e4m3(xb.astype(np.float32))
    back = F.split_rows_e4m3_value(terms, scales)
    blk = np.abs(xb).reshape(6, -1, 32).max(-1, keepdims=True)
    keep = (np.abs(xb).reshape(6, -1, 32) >= blk * 2.0 ** -13).reshape(6, 512)
    np.testing.assert_array_equal(back[keep], xb[keep])
    assert np.all(np.abs(back - xb) <= blk.repeat(32, axis=-1).reshape(6, 512) * 2.0 ** -20)
    hi = F.e4m3_value(terms[:, :, :128].reshape(6, -1, 32)).astype(np.float64)
    top = np.abs(hi).max(-1)
    assert np.all((top == 0) | ((top >= 128) & (top <= 256)))
