"""Weight formats of the expert path, restated in numpy (test oracle only).

Pinning (how each function here is checked, see tests/test_oracle_formats.py):

* ``quantize_mxfp4_bf16`` / ``quantize_mxfp4_fp8`` — the reference's four Swift
  known-answer tests (Tests/DeepSeekRepackTests/DeepSeekRepackTests.swift:336-412),
  bytes and SHA-256, plus the C restatement in ``oracle/c/oracle.c``.
* ``e2m1_value`` / ``e8m0_value`` / ``dequant_mxfp4`` — closed form over all
  16 codes x 256 scale bytes, and the round trip encode -> decode on exact values.
* ``e4m3_value`` — all 256 bytes against torch.float8_e4m3fn (an independent
  library decoder), NaN codes included.
* ``dequant_fp8_blocks`` — closed form on hand-built blocks (crop at ragged
  edges, NaN-code and bad-scale rejection).
* ``bf16_round`` — against torch's float32 -> bfloat16 conversion.
"""
from __future__ import annotations

import numpy as np

# E2M1 magnitudes, code & 7 -> value; bit 3 is the sign.
# deepseek_v41/dequant.py:29-30, Native/QwenNative/kernels.metal:140-144.
E2M1_MAGNITUDES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)
E2M1_VALUES = np.concatenate([E2M1_MAGNITUDES, -E2M1_MAGNITUDES]).astype(np.float32)

GROUP = 32          # MXFP4: values per E8M0 scale (deepseek_v41/dequant.py:27)
FP8_BLOCK = 128     # FP8 checkpoint: 128 x 128 blocks per fp32 scale (mimo/weights.py:27-41)


def e2m1_value(codes: np.ndarray) -> np.ndarray:
    """E2M1 nibble -> float32. Code 8 ("negative zero") decodes to -0.0, which
    compares equal to +0.0 (deepseek_v41/dequant.py:29-30 maps it to +0.0; the
    Metal table at Native/QwenNative/kernels.metal:701-702 gives -0.0)."""
    return E2M1_VALUES[np.asarray(codes) & 15]


def e8m0_value(scale_bytes: np.ndarray) -> np.ndarray:
    """E8M0 byte b -> 2**(b-127) as float32 (deepseek_v41/dequant.py:33-36).

    Edge bytes, fixed for this build: b == 0 is 2**-127 exactly (a float32
    denormal: what dequant.py's fp32 ``power`` gives and what OCP MX defines;
    the Metal bit trick at Native/QwenNative/kernels.metal:727 gives 0 instead),
    and b == 255 is NaN (OCP MX; dequant.py's fp32 power would give inf). The
    gfx950 scaled FP4 converts decode the same way, measured over all bytes.
    """
    b = np.asarray(scale_bytes).astype(np.int32)
    out = np.ldexp(np.ones(b.shape, np.float32), b - 127).astype(np.float32)
    return np.where(b == 255, np.float32(np.nan), out).astype(np.float32)


def unpack_mxfp4_codes(packed: np.ndarray) -> np.ndarray:
    """[O, K/8] uint32 (or [O, K/2] uint8) -> [O, K] codes; value i of a word is
    nibble i % 8, low nibble first (deepseek_v41/dequant.py:53-60,
    Native/QwenNative/kernels.metal:157-165)."""
    b = np.ascontiguousarray(packed).view(np.uint8)
    lo = b & 0x0F
    hi = b >> 4
    return np.stack([lo, hi], axis=-1).reshape(*b.shape[:-1], b.shape[-1] * 2)


def pack_mxfp4_codes(codes: np.ndarray) -> np.ndarray:
    """[O, K] codes -> [O, K/8] uint32 words (inverse of ``unpack_mxfp4_codes``)."""
    c = np.asarray(codes, np.uint8)
    pairs = c.reshape(*c.shape[:-1], c.shape[-1] // 2, 2)
    bytes_ = (pairs[..., 0] & 15) | ((pairs[..., 1] & 15) << 4)
    return np.ascontiguousarray(bytes_.astype(np.uint8)).view(np.uint32)


def dequant_mxfp4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Packed E2M1 [O, K/8] u32 + E8M0 [O, K/32] u8 -> float32 [O, K].

    w[o, i] = e2m1(nibble) * 2**(scale[o, i // 32] - 127), exact in fp32
    (deepseek_v41/dequant.py:63-68, Native/QwenNative/kernels.metal:511-518).
    """
    codes = unpack_mxfp4_codes(packed)
    values = e2m1_value(codes)
    s = e8m0_value(np.asarray(scales, np.uint8))
    return (values.reshape(*values.shape[:-1], -1, GROUP) * s[..., None]).reshape(values.shape)


def e4m3_value(bytes_: np.ndarray) -> np.ndarray:
    """FP8 E4M3FN byte -> float32 (Sources/DeepSeekRepack/MXFP4.swift:96-107).

    exponent 0: sign * m * 2**-9; (exponent, mantissa) == (15, 7): NaN;
    else sign * (1 + m/8) * 2**(e - 7).
    """
    b = np.asarray(bytes_, np.uint8).astype(np.int32)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0x0F
    m = b & 0x07
    sub = sign * m * 2.0 ** -9
    norm = sign * (1.0 + m / 8.0) * np.exp2(e - 7.0)
    out = np.where(e == 0, sub, norm)
    out = np.where((e == 15) & (m == 7), np.nan, out)
    return out.astype(np.float32)


def dequant_fp8_blocks(weight: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """FP8 E4M3 [rows, cols] bytes + fp32 [ceil(rows/128), ceil(cols/128)] -> fp32.

    Restates runtime/deepseek_v4_ssd/mimo/weights.py:17-43 with one source shard:
    shape checks, reserved NaN codes rejected (:33-34), non-finite or negative
    scales rejected (:35-36), each value times its block's scale, blocks cropped
    at ragged edges (:41). The reference then rounds to bf16; the expert path
    keeps fp32 (the MoE oracle's ``dequant-then-matmul`` is fp32).
    """
    w = np.asarray(weight)
    s = np.asarray(scales)
    if w.ndim != 2 or s.ndim != 2 or w.dtype != np.uint8:
        raise ValueError("FP8 weights must be a 2-D uint8 tensor with 2-D scales")
    if s.dtype != np.float32:
        raise ValueError("FP8 block scales must be float32")
    rows, cols = w.shape
    if rows < 1 or cols < 1:
        raise ValueError("FP8 tensor cannot be empty")
    if s.shape != (-(-rows // FP8_BLOCK), -(-cols // FP8_BLOCK)):
        raise ValueError("FP8 scale shape does not match 128x128 block padding")
    if np.any((w & 127) == 127):
        raise ValueError("FP8 checkpoint contains reserved NaN codes")
    if np.any(~np.isfinite(s) | (s < 0)):
        raise ValueError("FP8 checkpoint contains invalid block scales")
    expanded = np.repeat(np.repeat(s, FP8_BLOCK, axis=0), FP8_BLOCK, axis=1)[:rows, :cols]
    return (e4m3_value(w) * expanded).astype(np.float32)


FP8_E8M0_BLOCK = 32  # V4.1 release: one E8M0 byte per 32 x 32 block (deepseek_v41/dequant.py:25)


def dequant_fp8_e8m0(weight: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """FP8 E4M3 [rows, cols] bytes + E8M0 u8 [ceil(rows/32), ceil(cols/32)] -> fp32.

    Restates dequant_fp8 of runtime/deepseek_v4_ssd/deepseek_v41/dequant.py:45-50: every
    value times 2^(b - 127) of its 32 x 32 block (_expand_blocks crops the ceil overhang,
    :39-42), exact in fp32; the reference then casts to its output dtype (bf16 by default),
    which the expert path does not (the oracle's dequant-then-matmul is fp32). The native
    decoders compute the same products (fp8x4 x e8m0_256, Native/DeepSeekNative/kernels.metal:
    17-28). Byte 255 is NaN (OCP MX), byte 0 is 2^-127.
    """
    w = np.asarray(weight)
    s = np.asarray(scales)
    if w.ndim != 2 or s.ndim != 2 or w.dtype != np.uint8 or s.dtype != np.uint8:
        raise ValueError("FP8 weights and E8M0 scales must be 2-D uint8 tensors")
    rows, cols = w.shape
    if rows < 1 or cols < 1:
        raise ValueError("FP8 tensor cannot be empty")
    if s.shape != (-(-rows // FP8_E8M0_BLOCK), -(-cols // FP8_E8M0_BLOCK)):
        raise ValueError("E8M0 scale shape does not match 32x32 block padding")
    expanded = np.repeat(np.repeat(e8m0_value(s), FP8_E8M0_BLOCK, axis=0), FP8_E8M0_BLOCK, axis=1)[:rows, :cols]
    return (e4m3_value(w) * expanded).astype(np.float32)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def bf16_round(values: np.ndarray) -> np.ndarray:
    """float32 -> bf16 bits by round-to-nearest-even of the bit pattern
    (Sources/DeepSeekRepack/MXFP4.swift:109-113; NaN not special-cased, as there)."""
    bits = np.ascontiguousarray(values, np.float32).view(np.uint32).astype(np.uint64)
    rounded = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return (rounded >> 16).astype(np.uint16)


def bf16_round_f32(values: np.ndarray) -> np.ndarray:
    """float32 rounded to the nearest bf16, returned as float32."""
    return bf16_bits_to_f32(bf16_round(values))


def _fp4_code(values: np.ndarray) -> np.ndarray:
    """Nearest E2M1 code with ties to the even index, sign from the sign bit
    (Sources/DeepSeekRepack/MXFP4.swift:115-131). Magnitudes above 6 clamp to 6;
    a NaN magnitude keeps code 0 (no candidate compares less)."""
    v = np.asarray(values, np.float32)
    negative = np.signbit(v)
    magnitude = np.minimum(np.abs(v), np.float32(6.0))
    selected = np.zeros(v.shape, np.uint8)
    best = np.full(v.shape, np.inf, np.float32)
    for index, candidate in enumerate(E2M1_MAGNITUDES):
        d = np.abs(magnitude - candidate)
        take = (d < best) | ((d == best) & (index % 2 == 0))
        selected = np.where(take, np.uint8(index), selected)
        best = np.where(take, d, best)
    return selected | np.where(negative, np.uint8(8), np.uint8(0))


def _quantize_groups(values: np.ndarray, rows: int, columns: int) -> tuple[np.ndarray, np.ndarray]:
    """Shared tail of both Swift encoders (MXFP4.swift:22-37 and :68-85):
    per 32-value group, scale exponent = exponent(max|v|) - 2 clamped to
    [-127, 128]; an all-zero group keeps scale byte 0 and zero codes."""
    g = values.reshape(rows, columns // GROUP, GROUP).astype(np.float32)
    maximum = np.abs(g).max(axis=-1)
    zero = maximum == 0
    _, exp = np.frexp(np.where(zero, np.float32(1.0), maximum))
    exponent = np.clip(exp.astype(np.int32) - 1 - 2, -127, 128)   # Float.exponent == frexp - 1
    scales = np.where(zero, 0, exponent + 127).astype(np.uint8)
    factor = np.ldexp(np.float32(1.0), -exponent).astype(np.float32)
    codes = _fp4_code((g * factor[..., None]).astype(np.float32))
    codes = np.where(zero[..., None], np.uint8(0), codes)
    packed = (codes[..., 0::2] | (codes[..., 1::2] << 4)).astype(np.uint8)
    return packed.reshape(rows, columns // 2), scales


def quantize_mxfp4_bf16(bf16_bits: np.ndarray, rows: int, columns: int) -> tuple[np.ndarray, np.ndarray]:
    """BF16 [rows, columns] -> (MXFP4 bytes [rows, columns/2], E8M0 [rows, columns/32]).

    Restates MXFP4.quantizeBF16 (Sources/DeepSeekRepack/MXFP4.swift:4-40).
    """
    if rows <= 0 or columns <= 0 or columns % GROUP or np.size(bf16_bits) != rows * columns:
        raise ValueError("MXFP4 source must contain complete BF16 rows")
    values = bf16_bits_to_f32(np.asarray(bf16_bits, np.uint16).reshape(rows, columns))
    return _quantize_groups(values, rows, columns)


def quantize_mxfp4_fp8(fp8: np.ndarray, inverse_scales_bf16: np.ndarray,
                       rows: int, columns: int) -> tuple[np.ndarray, np.ndarray]:
    """FP8 E4M3 [rows, columns] with BF16 128x128 inverse scales -> MXFP4.

    Restates MXFP4.quantizeFP8 (Sources/DeepSeekRepack/MXFP4.swift:42-88): each
    value is e4m3 * scale rounded to bf16 (:66), then encoded as quantizeBF16.
    """
    if (rows <= 0 or columns <= 0 or rows % FP8_BLOCK or columns % FP8_BLOCK
            or np.size(fp8) != rows * columns
            or np.size(inverse_scales_bf16) != (rows // FP8_BLOCK) * (columns // FP8_BLOCK)):
        raise ValueError("MXFP4 FP8 source must contain complete 128 by 128 scale blocks")
    w = e4m3_value(np.asarray(fp8, np.uint8).reshape(rows, columns))
    s = bf16_bits_to_f32(np.asarray(inverse_scales_bf16, np.uint16).reshape(rows // FP8_BLOCK, columns // FP8_BLOCK))
    s = np.repeat(np.repeat(s, FP8_BLOCK, axis=0), FP8_BLOCK, axis=1)
    values = bf16_round_f32((w * s).astype(np.float32))
    return _quantize_groups(values, rows, columns)


# ---- E2M3 activation terms of the prefill GEMMs (no reference counterpart) ---------------
# The grouped GEMMs feed bf16 activations to the scaled MFMA as two E2M3 (fp6) terms per
# 32-value block, each with its own E8M0 exponent. This restates the device's split
# (whallm_amd/csrc/grouped_mfma.hip split6_rows_kernel / fp6_terms32) byte for byte.
# Pinned by the OCP MX definition of E2M3 (spacing and range, tests/test_oracle_formats.py),
# brute-force nearest-value rounding, reconstruction bounds, and the device bytes on MI355X.

SPLIT_STEP = 208   # bytes per row and 128-wide K step


def e2m3_value(codes: np.ndarray) -> np.ndarray:
    """6-bit E2M3 code -> float32: bit 5 sign, bits 3-4 exponent (bias 1), bits 0-2
    mantissa; exponent 0 is subnormal (m / 8). Max 7.5, no inf or NaN (OCP MX v1.0)."""
    c = np.asarray(codes, np.int64) & 63
    e, m = (c >> 3) & 3, c & 7
    mag = np.where(e == 0, m / 8.0, (1.0 + m / 8.0) * np.exp2(e - 1.0))
    return np.where(c & 32, -mag, mag).astype(np.float32)


E2M3_MAGNITUDES = e2m3_value(np.arange(32))


def e2m3_encode(values: np.ndarray) -> np.ndarray:
    """float -> E2M3 code: nearest magnitude, ties to the even code, saturating at 7.5;
    the sign bit follows the value's sign, also when the magnitude rounds to 0."""
    v = np.asarray(values, np.float64)
    if np.isnan(v).any():
        raise ValueError("E2M3 has no NaN")
    mag = np.minimum(np.abs(v), 7.5)
    d = np.abs(mag[..., None] - E2M3_MAGNITUDES.astype(np.float64))
    best = d.min(-1, keepdims=True)
    tie_codes = np.where(d == best, np.arange(32), 99)
    even = np.where(tie_codes % 2 == 0, tie_codes, 99).min(-1)
    code = np.where(even != 99, even, tie_codes.min(-1))
    return (code | np.where(np.signbit(v), 32, 0)).astype(np.uint8)


def e8m0_fp6_exponent(amax: np.ndarray) -> np.ndarray:
    """Biased exponent s putting a block maximum into [4, 8) at scale 2^(s - 127), at least 1."""
    e = (np.asarray(amax, np.float32).view(np.uint32) >> 23) & 0xFF
    return np.maximum(e.astype(np.int64) - 2, 1)


def e2m3_terms(block: np.ndarray) -> tuple[np.ndarray, np.ndarray, int, int]:
    """One 32-value fp32 block -> (hi codes, lo codes, s_hi, s_lo): hi = e2m3(x / 2^(s_hi-127));
    the residual r = x - value(hi) 2^(s_hi-127) (exact in fp32) gets its own exponent."""
    x = np.asarray(block, np.float32)
    s_hi = int(e8m0_fp6_exponent(np.abs(x).max()))
    sc_hi = np.float32(2.0 ** (s_hi - 127))
    hi = e2m3_encode(x / sc_hi)
    r = (x - e2m3_value(hi) * sc_hi).astype(np.float32)
    s_lo = int(e8m0_fp6_exponent(np.abs(r).max()))
    lo = e2m3_encode(r / np.float32(2.0 ** (s_lo - 127)))
    return hi, lo, s_hi, s_lo


def pack_e2m3_fields(codes: np.ndarray) -> np.ndarray:
    """32 six-bit codes -> 24 bytes, code k at bits 6k .. 6k + 5 (little-endian)."""
    bits = 0
    for k, c in enumerate(np.asarray(codes, np.uint8).reshape(32)):
        bits |= int(c) << (6 * k)
    return np.frombuffer(bits.to_bytes(24, "little"), np.uint8)


def split_rows_e2m3(x: np.ndarray) -> np.ndarray:
    """fp32 rows [R, H] (H a multiple of 128) -> [R, H/128, 208] bytes: per 128-wide step, the
    4 blocks' hi fields (24 B) and lo fields (24 B) in turn, then the 4 hi exponents, the 4 lo
    exponents; bytes 200-207 are padding (left unwritten by the device, zero here)."""
    x = np.asarray(x, np.float32)
    R, H = x.shape
    if H % 128:
        raise ValueError("split rows need H a multiple of 128")
    out = np.zeros((R, H // 128, SPLIT_STEP), np.uint8)
    for r in range(R):
        for b in range(H // 32):
            hi, lo, s_hi, s_lo = e2m3_terms(x[r, 32 * b:32 * b + 32])
            st, o = out[r, b // 4], (b % 4) * 48
            st[o:o + 24] = pack_e2m3_fields(hi)
            st[o + 24:o + 48] = pack_e2m3_fields(lo)
            st[192 + b % 4] = s_hi
            st[196 + b % 4] = s_lo
    return out


# ---- bf16-exact activation terms: two E4M3 terms per 32 values --------------------------

_E4M3_MAG = None


def e4m3_encode(v: np.ndarray) -> np.ndarray:
    """fp32 values with |v| <= 448 -> E4M3FN bytes, rounded to nearest, ties to the even code;
    a negative value that rounds to zero keeps its sign (0x80)."""
    global _E4M3_MAG
    if _E4M3_MAG is None:
        _E4M3_MAG = e4m3_value(np.arange(127, dtype=np.uint8)).astype(np.float64)  # codes 0..126 ascend
    v = np.asarray(v, np.float64)
    a = np.abs(v)
    if np.any(a > 448) or np.any(~np.isfinite(v)):
        raise ValueError("e4m3_encode takes finite values up to 448")
    hi = np.clip(np.searchsorted(_E4M3_MAG, a, side="left"), 0, 126)   # first code >= a
    lo = np.clip(hi - 1, 0, 126)
    d_lo, d_hi = a - _E4M3_MAG[lo], _E4M3_MAG[hi] - a
    code = np.where(d_lo < d_hi, lo, np.where(d_hi < d_lo, hi, np.where(lo % 2 == 0, lo, hi)))
    code = np.where(a == _E4M3_MAG[hi], hi, code)
    return (code | np.where(np.signbit(v), 0x80, 0)).astype(np.uint8)


def e4m3_term_exponent(amax) -> int:
    """E8M0 exponent of a block's hi term: e(amax) - 7 (biased), at least 5."""
    e = int((np.float32(amax).view(np.uint32) >> 23) & 0xFF)
    return max(e - 7, 5)


def e4m3_terms(block: np.ndarray) -> tuple[np.ndarray, np.ndarray, int]:
    """One 32-value block -> (hi bytes, lo bytes, s): hi = e4m3(x / 2^(s-127)) and lo =
    e4m3((x / 2^(s-127) - value(hi)) * 16), the lo scale being 2^(s-131)."""
    x = np.asarray(block, np.float32)
    s = e4m3_term_exponent(np.abs(x).max())
    h = (x * np.float32(2.0 ** (127 - s))).astype(np.float32)
    hi = e4m3_encode(h)
    lo = e4m3_encode(((h - e4m3_value(hi)) * np.float32(16.0)).astype(np.float32))
    return hi, lo, s


def split_rows_e4m3(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp32 rows [R, H] (H a multiple of 128) -> (terms [R, H/128, 256] bytes: per 128-wide step
    the hi terms of K 0..127, then the lo terms; scales [R, H/128] uint32: the step's 4 hi
    exponents, byte b for block b)."""
    x = np.asarray(x, np.float32)
    R, H = x.shape
    if H % 128:
        raise ValueError("split rows need H a multiple of 128")
    terms = np.zeros((R, H // 128, 256), np.uint8)
    scales = np.zeros((R, H // 128), np.uint32)
    for r in range(R):
        for b in range(H // 32):
            hi, lo, sc = e4m3_terms(x[r, 32 * b:32 * b + 32])
            st = terms[r, b // 4]
            st[32 * (b % 4):32 * (b % 4) + 32] = hi
            st[128 + 32 * (b % 4):128 + 32 * (b % 4) + 32] = lo
            scales[r, b // 4] |= np.uint32(sc) << np.uint32(8 * (b % 4))
    return terms, scales


def split_rows_e4m3_value(terms: np.ndarray, scales: np.ndarray) -> np.ndarray:
    """Inverse view of split_rows_e4m3: hi 2^(s-127) + lo 2^(s-131) per value, float64."""
    t = np.asarray(terms, np.uint8)
    R, steps = t.shape[:2]
    sc = np.asarray(scales).astype(np.uint32)
    out = np.zeros((R, steps * 128), np.float64)
    for b in range(steps * 4):
        s = ((sc[:, b // 4] >> np.uint32(8 * (b % 4))) & np.uint32(0xFF)).astype(np.float64)[:, None]
        hi = e4m3_value(t[:, b // 4, 32 * (b % 4):32 * (b % 4) + 32]).astype(np.float64)
        lo = e4m3_value(t[:, b // 4, 128 + 32 * (b % 4):160 + 32 * (b % 4)]).astype(np.float64)
        out[:, 32 * b:32 * b + 32] = hi * np.exp2(s - 127) + lo * np.exp2(s - 131)
    return out


def split_rows_value(split: np.ndarray, H: int) -> np.ndarray:
    """Inverse view of split_rows_e2m3: hi 2^(s_hi-127) + lo 2^(s_lo-127) per value, float64."""
    s = np.asarray(split, np.uint8)
    R = s.shape[0]
    out = np.zeros((R, H), np.float64)
    for r in range(R):
        for b in range(H // 32):
            st, o = s[r, b // 4], (b % 4) * 48
            for part, off, sb in ((0, o, 192), (1, o + 24, 196)):
                bits = int.from_bytes(bytes(st[off:off + 24]), "little")
                codes = np.array([(bits >> (6 * k)) & 63 for k in range(32)])
                out[r, 32 * b:32 * b + 32] += e2m3_value(codes).astype(np.float64) * 2.0 ** (int(st[sb + b % 4]) - 127)
    return out
