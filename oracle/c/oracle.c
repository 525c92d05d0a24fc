/* CPU oracle, plain C — TEST INFRASTRUCTURE ONLY (never linked into the product).
 *
 * A second restatement, independent of oracle/formats.py, of the byte-level
 * arithmetic of the expert path:
 *   - MXFP4 encoders  (Sources/DeepSeekRepack/MXFP4.swift:4-40, :42-88, helpers :90-131)
 *   - E2M1 / E8M0 decode (runtime/deepseek_v4_ssd/deepseek_v41/dequant.py:24-68)
 *   - E4M3 decode      (MXFP4.swift:96-107)
 *   - top-k by value, ties to the lower index (Native/DeepSeekNative/engine.mm:1881)
 *   - the fp32 dequant-then-matmul expert FFN (qwen4_exp.py:815-818)
 * Pinned by the reference's Swift known-answer vectors
 * (Tests/DeepSeekRepackTests/DeepSeekRepackTests.swift:336-412) through
 * tests/test_oracle_formats.py, and cross-checked against the numpy oracle.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float bf16_to_f32(uint16_t bits) {
  uint32_t u = (uint32_t)bits << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static float round_bf16(float v) { /* MXFP4.swift:109-113 */
  uint32_t bits;
  memcpy(&bits, &v, 4);
  uint32_t r = (bits + 0x7fffu + ((bits >> 16) & 1u)) & 0xffff0000u;
  float f;
  memcpy(&f, &r, 4);
  return f;
}

float wm_oracle_e4m3(uint8_t b) { /* MXFP4.swift:96-107 */
  float sign = (b & 0x80) ? -1.0f : 1.0f;
  int exponent = (b >> 3) & 0x0f, mantissa = b & 0x07;
  if (exponent == 0) return sign * (float)mantissa * ldexpf(1.0f, -9);
  if (exponent == 15 && mantissa == 7) return NAN;
  return sign * (1.0f + (float)mantissa / 8.0f) * ldexpf(1.0f, exponent - 7);
}

static const float E2M1[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

static uint8_t fp4_code(float value) { /* MXFP4.swift:115-131 */
  int negative = signbit(value) != 0;
  float a = fabsf(value);
  float magnitude = (6.0f < a) ? 6.0f : a; /* Swift min(a, 6): NaN stays NaN */
  int selected = 0;
  float distance = INFINITY;
  for (int i = 0; i < 8; ++i) {
    float d = fabsf(magnitude - E2M1[i]);
    if (d < distance || (d == distance && (i % 2) == 0)) {
      selected = i;
      distance = d;
    }
  }
  return (uint8_t)(selected | (negative ? 8 : 0));
}

static int float_exponent(float m) { /* Swift Float.exponent for a finite nonzero value */
  int e;
  frexpf(m, &e);
  return e - 1;
}

/* One 32-value group -> 16 bytes + 1 scale byte (MXFP4.swift:22-37). */
static void encode_group(const float* values, uint8_t* weights, uint8_t* scale) {
  float maximum = 0.0f;
  for (int i = 0; i < 32; ++i) {
    float a = fabsf(values[i]);
    maximum = a > maximum ? a : maximum; /* Swift max(maximum, a) */
  }
  if (maximum == 0.0f) return; /* group stays zero, scale byte 0 */
  int exponent = float_exponent(maximum) - 2;
  if (exponent < -127) exponent = -127;
  if (exponent > 128) exponent = 128;
  *scale = (uint8_t)(exponent + 127);
  float factor = ldexpf(1.0f, -exponent);
  for (int p = 0; p < 16; ++p) {
    uint8_t lo = fp4_code(values[2 * p] * factor);
    uint8_t hi = fp4_code(values[2 * p + 1] * factor);
    weights[p] = (uint8_t)(lo | (hi << 4));
  }
}

/* Returns 0 on success, 1 on an invalid plan (MXFP4.swift:9-14). */
int wm_oracle_quantize_bf16(const uint16_t* source, int64_t rows, int64_t columns, uint8_t* weights,
                            uint8_t* scales) {
  if (rows <= 0 || columns <= 0 || columns % 32) return 1;
  int64_t groups = columns / 32;
  memset(weights, 0, (size_t)(rows * columns / 2));
  memset(scales, 0, (size_t)(rows * groups));
  float values[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t g = 0; g < groups; ++g) {
      for (int i = 0; i < 32; ++i) values[i] = bf16_to_f32(source[r * columns + g * 32 + i]);
      encode_group(values, weights + r * columns / 2 + g * 16, scales + r * groups + g);
    }
  return 0;
}

int wm_oracle_quantize_fp8(const uint8_t* source, const uint16_t* inverse_scales, int64_t rows,
                           int64_t columns, uint8_t* weights, uint8_t* scales) {
  if (rows <= 0 || columns <= 0 || rows % 128 || columns % 128) return 1;
  int64_t groups = columns / 32, scale_columns = columns / 128;
  memset(weights, 0, (size_t)(rows * columns / 2));
  memset(scales, 0, (size_t)(rows * groups));
  float values[32];
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t g = 0; g < groups; ++g) {
      float s = bf16_to_f32(inverse_scales[(r / 128) * scale_columns + g / 4]);
      for (int i = 0; i < 32; ++i) values[i] = round_bf16(wm_oracle_e4m3(source[r * columns + g * 32 + i]) * s);
      encode_group(values, weights + r * columns / 2 + g * 16, scales + r * groups + g);
    }
  return 0;
}

/* w[o, i] = e2m1(nibble i % 8 of word i / 8) * 2^(scale - 127); scale byte 0 -> 2^-127
   (an fp32 denormal), 255 -> NaN (OCP MX). */
void wm_oracle_dequant_mxfp4(const uint32_t* packed, const uint8_t* scales, int64_t rows, int64_t columns,
                             float* out) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t i = 0; i < columns; ++i) {
      uint32_t word = packed[r * (columns / 8) + i / 8];
      uint32_t code = (word >> (4 * (i % 8))) & 15u;
      int b = scales[r * (columns / 32) + i / 32];
      float s = b == 255 ? NAN : ldexpf(1.0f, b - 127);
      float v = E2M1[code & 7];
      out[r * columns + i] = ((code & 8) ? -v : v) * s;
    }
}

/* Indices of the k largest values of each row, descending, ties to the lower index. */
void wm_oracle_topk(const float* scores, int64_t rows, int64_t columns, int64_t k, int32_t* indices) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* row = scores + r * columns;
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t c = 0; c < columns; ++c) {
        int taken = 0;
        for (int64_t q = 0; q < j; ++q) taken |= indices[r * k + q] == c;
        if (taken) continue;
        if (best < 0 || row[c] > row[best]) best = c;
      }
      indices[r * k + j] = (int32_t)best;
    }
  }
}

/* y[t] = (silu(x Wg^T) * (x Wu^T)) Wd^T in fp32 for one expert; Wgu [2I, H], Wd [H, I] dense fp32. */
void wm_oracle_ffn(const float* x, int64_t tokens, int64_t hidden, int64_t inter, const float* wgu,
                   const float* wd, float* act, float* y) {
  for (int64_t t = 0; t < tokens; ++t) {
    for (int64_t i = 0; i < inter; ++i) {
      float g = 0.0f, u = 0.0f;
      for (int64_t h = 0; h < hidden; ++h) {
        g += x[t * hidden + h] * wgu[i * hidden + h];
        u += x[t * hidden + h] * wgu[(inter + i) * hidden + h];
      }
      act[t * inter + i] = g / (1.0f + expf(-g)) * u;
    }
    for (int64_t o = 0; o < hidden; ++o) {
      float s = 0.0f;
      for (int64_t i = 0; i < inter; ++i) s += act[t * inter + i] * wd[o * inter + i];
      y[t * hidden + o] = s;
    }
  }
}
