// Shared device/host helpers of libwhallm_moe (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <stdexcept>
#include <string>

#include "../../include/whallm_moe.h"

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 wm_bf16x2;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 wm_bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float wm_f32x4;
typedef __attribute__((__vector_size__(2 * sizeof(float)))) float wm_f32x2;

namespace wm {

// ------------------------------------------------------------------ host error state
void set_error(const std::string& message);
void clear_error();

// Thrown when a caller's cancel callback asks to stop; the entry point returns 2
// (Native/QwenNative/capi.h:1-5: 0 ok, 1 error, 2 cancelled).
struct Cancelled : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// Runs `body`; a thrown std::exception becomes status 1 with its message, Cancelled
// status 2 (Native/QwenNative/capi.mm:20-37 turns exceptions into a status the same way).
template <typename Body>
int guarded(Body body) {
  try {
    clear_error();
    body();
    return 0;
  } catch (const Cancelled& e) {
    set_error(e.what());
    return 2;
  } catch (const std::exception& e) {
    set_error(e.what());
    return 1;
  } catch (...) {
    set_error("unknown error");
    return 1;
  }
}

[[noreturn]] void fail(const std::string& message);
void check_hip(hipError_t status, const char* what);
// Raises if the last launch failed (bad configuration, missing code object).
void check_launch(const char* kernel);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// ------------------------------------------------------------------ device helpers
// Load through a pointer known to address global memory. Pointers read from LDS or
// from memory are generic to the compiler, which then emits FLAT accesses; those
// also count against the LDS wait counter, so every LDS wait would wait for them.
template <typename T>
__device__ __forceinline__ T gload(const void* p) {
  return *(const __attribute__((address_space(1))) T*)(p);
}
typedef uint32_t wm_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 gload16(const void* p) {
  wm_u32x4 v = *(const __attribute__((address_space(1))) wm_u32x4*)(p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
// The same with the non-temporal hint (global_load ... nt), for data read once per call
// (weights streamed through a decode step).
__device__ __forceinline__ uint4 gload16_nt(const void* p) {
  wm_u32x4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) wm_u32x4*)(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) { return __uint_as_float(bits16 << 16); }

// float -> bf16 bits, round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// E8M0 byte -> 2^(b - 127) as the float whose exponent field is b. Used only as
// the scale operand of the gfx950 scaled converts, which read its exponent field:
// byte 0 decodes to 2^-127 and 255 to NaN (OCP MX), bit-exact with
// oracle/formats.py e8m0_value over all 256 bytes.
__device__ __forceinline__ float e8m0_scale_operand(uint32_t b) { return __uint_as_float(b << 23); }

// E8M0 byte -> its value 2^(b - 127) as a float to multiply by: byte 0 is the denormal
// 2^-127, 255 NaN (OCP MX), every other byte the normal float with exponent field b.
__device__ __forceinline__ float e8m0_value(uint32_t b) {
  return b == 0u ? __uint_as_float(0x00400000u) : (b == 255u ? __uint_as_float(0x7fc00000u) : __uint_as_float(b << 23));
}

// E2M1 magnitude table as fp32 bit patterns, index = code & 7.
__device__ __forceinline__ float e2m1_to_f32(uint32_t code) {
  // 0, .5, 1, 1.5, 2, 3, 4, 6: exponent/mantissa built from the 3 magnitude bits.
  uint32_t m = code & 7u;
  uint32_t e = m >> 1, man = m & 1u;
  // e == 0: subnormal E2M1 (0 or 0.5); else (1 + man/2) * 2^(e-1).
  uint32_t bits = e ? (((e + 126u) << 23) | (man << 22)) : (man ? 0x3f000000u : 0u);
  return __uint_as_float(bits | ((code & 8u) << 28));
}

// Eight E2M1 nibbles of one word as four bf16 pairs (nibbles 2j, 2j+1 in pair j),
// each times `scale` (a power of two). gfx950 V_CVT_SCALEF32_PK_BF16_FP4.
__device__ __forceinline__ void fp4x8_to_bf16(uint32_t word, float scale, wm_bf16x2 out[4]) {
  out[0] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 0);
  out[1] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 1);
  out[2] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 2);
  out[3] = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(word, scale, 3);
}

// bf16 pair . bf16 pair + acc (fp32), gfx950 V_DOT2_F32_BF16.
__device__ __forceinline__ float dot2_bf16(wm_bf16x2 a, wm_bf16x2 b, float acc) {
  return __builtin_amdgcn_fdot2_f32_bf16(a, b, acc, false);
}

__device__ __forceinline__ wm_bf16x2 bits_to_bf16x2(uint32_t u) { return __builtin_bit_cast(wm_bf16x2, u); }
__device__ __forceinline__ uint32_t bf16x2_to_bits(wm_bf16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// E4M3FN byte -> fp32 (Sources/DeepSeekRepack/MXFP4.swift:96-107): built from bits,
// subnormals exact; 0x7f / 0xff -> NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  uint32_t e = (b >> 3) & 15u, m = b & 7u;
  float mag;
  if (e == 0) mag = (float)m * (1.0f / 512.0f);
  else if (e == 15 && m == 7) mag = __uint_as_float(0x7fc00000u);
  else mag = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return (b & 0x80u) ? -mag : mag;
}

// DPP move of a float within 16-lane rows (gfx9 DPP controls).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over `WIDTH` consecutive lanes (a power of two <= 64), result in every lane of
// the segment. 16- and 64-lane sums use DPP (quad permutes and row mirrors) and,
// across rows, lane reads into scalar registers; no LDS round trips.
template <int WIDTH>
__device__ __forceinline__ float segment_sum(float v) {
  if constexpr (WIDTH == 16 || WIDTH == 64) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]: pairs
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]: quads
    v += dpp_f<0x141>(v);  // row_half_mirror: 8 lanes
    v += dpp_f<0x140>(v);  // row_mirror: 16 lanes
    if constexpr (WIDTH == 64) {
      float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
      float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
      float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
      float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
      v = (r0 + r1) + (r2 + r3);
    }
    return v;
  } else {
#pragma unroll
    for (int offset = WIDTH / 2; offset > 0; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
  }
}

// Maximum over each aligned group of WIDTH lanes (16 or 64); every lane of the group
// receives it. Same DPP steps as segment_sum.
template <int WIDTH>
__device__ __forceinline__ float segment_max(float v) {
  static_assert(WIDTH == 16 || WIDTH == 64, "segment_max: width 16 or 64");
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  if constexpr (WIDTH == 64) {
    float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    v = fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
  }
  return v;
}

// x * sigmoid(x) with the native exp2 and reciprocal (each ~1 ulp): large negative x gives
// exp2 -> inf, rcp -> 0, result -0; large positive x gives x; NaN stays NaN.
__device__ __forceinline__ float silu(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-1.4426950408889634f * x));
}

}  // namespace wm
