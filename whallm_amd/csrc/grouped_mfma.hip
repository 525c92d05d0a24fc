// Prefill-time expert FFN on gfx950 scaled MFMA (v_mfma_scale_f32_32x32x64_f8f6f4):
// grouped GEMMs over the row tiles of the permute kernel, for MXFP4 weights (E2M1 codes
// with an E8M0 scale per 32, fed to the MFMA as stored) and for FP8-E4M3 weights with
// fp32 128 x 128 block scales or with E8M0 32 x 32 block scales (the V4.1 release; the
// E8M0 bytes ride on the MFMA's A scales like MXFP4's).
//
// Replaces gather_rows16 + expert_gemm_sg (gate_up) + expert_act + expert_gemm_sg (down) +
// moe_combine_rows (Native/QwenNative/kernels.metal:691-765, engine.mm:2104-2162) and
// mx.gather_qmm (qwen4_exp.py:857-897, model.py:435-501):
//
//   split   : every token row of x (bf16) becomes two E2M3 (fp6) terms, hi and lo, each
//             with an E8M0 scale per 32 values, stored as the MFMA's B operand reads them
//             (the GEMMs copy them to LDS unchanged).
//   gate_up : tile = 128 permuted rows x (TW / 2 gate + the matching up weight rows); per
//             128-wide K step each wave runs its weight tiles x 2 row tiles x 2 halves of
//             the step x 2 terms MFMAs. SwiGLU is the epilogue, which writes act straight
//             back as E2M3 terms (the down GEMM's B operand).
//   down    : tile = 128 permuted rows x TW output columns over K = intermediate; bf16
//             rows in permuted order, unweighted.
//   combine : y[t] = sum of the token's K rows times their routing weights in k order,
//             plus the shared row times its gate.
//
// The shared expert is one more row group after the routed ones (rows P .. P+T-1). Work
// tiles are mapped XCD-major so the column tiles of one row tile share an L2.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <mutex>

#include "wm_common.h"
#include "moe_internal.h"

namespace wm {
namespace mf {

constexpr int BM = 128;     // permuted rows per tile
constexpr int XCDS = 8;
constexpr int FMT_FP8 = 0;
constexpr int FMT_FP4 = 4;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

struct Lists {
  const int32_t* order;       // [P] pair of each permuted row
  const int32_t* offsets;     // [E + 1]
  const int32_t* tiles;       // [n][2] (expert, first row)
  const int32_t* tile_count;  // [1]
  const float* shared_gate;   // [T] gate of the shared rows
  int pairs;                  // P = T * K
  int tokens;
  int k;
  int has_shared;
};

__device__ __forceinline__ int active_row_tiles(const Lists& L) {
  return L.tile_count[0] + (L.has_shared ? (L.tokens + BM - 1) / BM : 0);
}

__device__ __forceinline__ float pow2_biased(int e) { return __uint_as_float((uint32_t)e << 23); }

// ---------------------------------------------------------------------------------
// Loads and the persistent K loop.

// Direct global -> LDS loads, lane i writing LDS address lds + size * i. Written as inline
// assembly so the compiler does not treat them as LDS stores it must wait for before every
// LDS read (it cannot tell the ring's stages apart); the K loop's explicit vmcnt waits and
// barriers order them instead. M0 carries the wave-uniform LDS address (nothing else in
// these kernels uses M0); an M0 write needs wait states before an LDS DMA reads it.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) uint8_t*)p;
}
// The global address is a wave-uniform base in scalar registers plus a 32-bit per-lane
// offset, so no 64-bit addresses occupy vector registers.
__device__ __forceinline__ void dma16(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dwordx4 %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory");
}
__device__ __forceinline__ void dma4(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\ts_nop 1\n\tglobal_load_lds_dword %1, %2" ::"s"(lds), "v"(off), "s"(base)
               : "memory");
}
// A pointer every lane holds, moved to scalar registers and read through the constant
// address space, so the loads through it are scalar loads (waited for through lgkmcnt,
// outside the vmcnt count of the ring's loads). For data the kernel never writes.
typedef const __attribute__((address_space(4))) float* const_f32_ptr;
__device__ __forceinline__ const_f32_ptr uniform_ptr(const float* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return (const_f32_ptr)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ const uint8_t* uniform_u8(const uint8_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// Wait until this wave's loads have landed and its LDS reads have returned, then let every
// wave see every wave's loads. One asm statement, so no LDS access is scheduled across
// it, and no memory fence.
__device__ __forceinline__ void ring_wait_all() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The tiles of this workgroup in a persistent launch: XCD x takes the contiguous range
// [x * share, (x + 1) * share) of the (row tile, column tile) list, and its workgroups
// take every (gridDim / 8)-th tile of it, so the column tiles of a row tile (which read
// the same rows) and the row tiles of an expert (the same weights) meet in one L2.
struct TileRange {
  int first, stride, count;
};
__device__ __forceinline__ TileRange tile_range(int active) {
  const int xcd = blockIdx.x % XCDS, local = blockIdx.x / XCDS, per = gridDim.x / XCDS;
  const int share = (active + XCDS - 1) / XCDS;
  const int hi = min(xcd * share + share, active);
  TileRange t{xcd * share + local, per, 0};
  if (t.first < hi) t.count = (hi - t.first + per - 1) / per;
  return t;
}

// ---------------------------------------------------------------------------------
// Expert regions of a tile.

struct TileWeights {
  const uint8_t* w13;     // gate/up rows (MXFP4 words or E4M3 bytes)
  const uint8_t* w13s;    // MXFP4: E8M0 [2I, H/32]; FP8: fp32 [2I/128, H/128]
  const uint8_t* w2;
  const uint8_t* w2s;
  int up_first;
  float limit;
};

// ---------------------------------------------------------------------------------
// Activations as two E2M3 (fp6) terms. On v_mfma_scale_f32_32x32x64_f8f6f4 fp4 x fp6 runs
// at twice the rate of any fp8 operand (measured on MI355X: 32 against 64 cycles per
// instruction), and fp8 x fp6 at the fp8 rate (the 16x16x128 shape runs every format at
// the fp8 rate).
//
// Terms: a 32-value block gets hi = e2m3(x / 2^(s - 127)) with s = e(max |x|) - 2, so the
// block maximum lands in [4, 8); the residual x - hi (exact in fp32) gets its own block
// exponent the same way, lo = e2m3(residual / 2^(t - 127)). Rounding is to nearest even,
// saturating at 7.5 (the hardware conversion's behaviour). Per element the pair keeps an
// absolute error within about 2^-7 of the block maximum's binade.
//
// Split rows (x, and act for the down GEMM): per row, per 128-wide K step, 208 bytes: the
// 4 blocks' terms (hi fields 24 bytes, lo fields 24 bytes, each), then the 4 blocks' hi
// E8M0 bytes, their lo bytes, and 8 bytes of padding. The GEMMs load a row's step as 13
// pieces of 16 bytes.

constexpr int FMT_FP6 = 2;
constexpr int XSTEP = 208;

// E8M0 exponent that maps a block maximum into [4, 8) (never below 1, so 2^(127 - s) stays
// a normal float).
__device__ __forceinline__ int fp6_exponent(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xff);
  return e - 2 > 1 ? e - 2 : 1;
}

typedef float v16f_t __attribute__((ext_vector_type(16)));
typedef unsigned v6u_t __attribute__((ext_vector_type(6)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f2_t __attribute__((ext_vector_type(2)));

// Two floats to packed bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f2_t){a, b}, bf16x2_t));
}

// The two wide scaled conversions, written as assembly with early-clobber outputs. Both
// read their source and write their result over several passes, so a result register
// that overlaps a source register still to be read corrupts that source: the compiler's
// register allocator (ROCm 7.2) does allocate e.g. v[2:7] over a v[0:15] source, and on
// MI355X that cleared bits of field 5 in most blocks. "=&v" keeps the result apart.
__device__ __forceinline__ v6u_t cvt_2xpk16_fp6(const v16f_t& a, const v16f_t& b, float scale) {
  v6u_t r;
  asm("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, %3" : "=&v"(r) : "v"(a), "v"(b), "v"(scale));
  return r;
}
typedef float v32f_t __attribute__((ext_vector_type(32)));
__device__ __forceinline__ v32f_t cvt_pk32_f32_fp6(const v6u_t& f, float scale) {
  v32f_t r;
  asm("v_cvt_scalef32_pk32_f32_fp6 %0, %1, %2" : "=&v"(r) : "v"(f), "v"(scale));
  return r;
}

// The hi and lo E2M3 terms of one 32-value block (v in K order) with the hardware
// conversions: v_cvt_scalef32_2xpk16_fp6_f32 packs e2m3(x / scale) of its two 16-value
// operands interleaved (field 2i from the first, 2i + 1 from the second), rounding to
// nearest even and saturating at 7.5 (a negative value that rounds to zero keeps its sign
// bit); v_cvt_scalef32_pk32_f32_fp6 gives field * scale back, so the residual v - hi is exact.
__device__ __forceinline__ void fp6_terms32(const float (&v)[32], v6u_t& hi, v6u_t& lo, int& s_hi, int& s_lo) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  s_hi = fp6_exponent(amax);
  const float sc_hi = pow2_biased(s_hi);
  v16f_t ev, od;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    ev[m] = v[2 * m];
    od[m] = v[2 * m + 1];
  }
  hi = cvt_2xpk16_fp6(ev, od, sc_hi);
  const v32f_t back = cvt_pk32_f32_fp6(hi, sc_hi);
  float rmax = 0.0f;
#pragma unroll
  for (int m = 0; m < 16; ++m) {
    ev[m] = v[2 * m] - back[2 * m];
    od[m] = v[2 * m + 1] - back[2 * m + 1];
    rmax = fmaxf(rmax, fmaxf(fabsf(ev[m]), fabsf(od[m])));
  }
  s_lo = fp6_exponent(rmax);
  lo = cvt_2xpk16_fp6(ev, od, pow2_biased(s_lo));
}

// x [rows, H] bf16 -> split rows [rows][H/128][208 bytes]. One lane per 32-value block.
// With g (bf16 [H]) the kernel also writes gate[row] = sigmoid(x[row] . g), the shared
// expert's gate: a row's H/32 lanes are contiguous and aligned (H/32 a power of two <= 64),
// so their partial dots meet in a butterfly inside the group.
__global__ void __launch_bounds__(256) split6_rows_kernel(const uint16_t* __restrict__ x, int rows, int hidden,
                                                          uint8_t* __restrict__ x6, const uint16_t* __restrict__ g,
                                                          float* __restrict__ gate) {
  const int blocks = hidden / 32;
  const int64_t job = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (row, block)
  if (job >= (int64_t)rows * blocks) return;
  const int64_t row = job / blocks;
  const int blk = (int)(job % blocks);
  const uint4* src = reinterpret_cast<const uint4*>(x + row * hidden + blk * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 u = src[q];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * q + 2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
      v[8 * q + 2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
    }
  }
  v6u_t hi, lo;
  int s_hi, s_lo;
  fp6_terms32(v, hi, lo, s_hi, s_lo);
  uint8_t* step = x6 + (row * (hidden / 128) + blk / 4) * XSTEP;
  uint4* dst = reinterpret_cast<uint4*>(step + (blk % 4) * 48);
  dst[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  dst[1] = make_uint4(hi[4], hi[5], lo[0], lo[1]);
  dst[2] = make_uint4(lo[2], lo[3], lo[4], lo[5]);
  // the step's four blocks are lanes 4q .. 4q + 3 (blocks is a multiple of 4): the first
  // lane of the quad gathers their scale bytes and stores them as two words
  const uint32_t sc = (uint32_t)s_hi | ((uint32_t)s_lo << 8);
  const uint32_t q1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0x55, 0xf, 0xf, false);  // quad_perm [1,1,1,1]
  const uint32_t q2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0xAA, 0xf, 0xf, false);  // [2,2,2,2]
  const uint32_t q3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0xFF, 0xf, 0xf, false);  // [3,3,3,3]
  if (blk % 4 == 0) {
    const uint32_t w_hi = (sc & 0xffu) | ((q1 & 0xffu) << 8) | ((q2 & 0xffu) << 16) | ((q3 & 0xffu) << 24);
    const uint32_t w_lo = (sc >> 8) | ((q1 >> 8) << 8) | ((q2 >> 8) << 16) | ((q3 >> 8) << 24);
    *reinterpret_cast<uint2*>(step + 192) = make_uint2(w_hi, w_lo);
  }
  if (g) {
    const uint4* gs = reinterpret_cast<const uint4*>(g + blk * 32);
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 u = gs[q];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dot = fmaf(v[8 * q + 2 * j], bf16_bits_to_f32(w[j] & 0xffffu), dot);
        dot = fmaf(v[8 * q + 2 * j + 1], bf16_bits_to_f32(w[j] >> 16), dot);
      }
    }
    if (blocks == 64) {
      dot = segment_sum<64>(dot);  // the row is the whole wave: DPP and lane reads, no LDS
    } else {
      for (int off = 1; off < blocks; off <<= 1) dot += __shfl_xor(dot, off, 64);
    }
    if (blk == 0) gate[row] = 1.0f / (1.0f + __expf(-dot));
  }
}

// ---------------------------------------------------------------------------------
// Activations as two E4M3 terms (the bf16-exact form). A 32-value block gets hi =
// e4m3(x / 2^(s - 127)) with s = max(e(max |x|) - 7, 5), so the block maximum lands in
// [128, 256) (E4M3's largest finite is 448), and lo = e4m3((x / 2^(s - 127) - hi) * 16)
// under the scale 2^(s - 131), rounded to nearest even (the hardware conversion; both terms
// stay below 448, so nothing saturates). hi + lo reproduces every bf16 x with |x| >= 2^-13
// of its block's maximum exactly (hi keeps x's top 4 significant bits, the residual the
// other 4, and the residual times 16 stays on E4M3's grid down to 2^-13), the precision of
// the reference's bf16 activations (Native/QwenNative/kernels.metal:706-751 multiplies
// fp32 activations, qwen4_exp.py:774-783 feeds bf16 into quantized_matmul). An fp8 operand
// runs the 32x32x64 MFMA at the FP8 rate: fp4 x fp8 takes 64 cycles against fp4 x fp6's 32.
//
// Split rows: per row and 128-wide K step, 256 term bytes (hi for K 0..127, then lo, each in
// K order) in one array and the step's 4 hi scale bytes as one dword in another ([rows][steps]);
// the lo scale is the hi scale minus 4.
constexpr int XSTEP8 = 256;

// E8M0 exponent of a block's hi term: e(max) - 7, at least 5 so that the lo scale (s - 4)
// stays a normal power of two.
__device__ __forceinline__ int fp8_term_exponent(float amax) {
  const int e = (int)((__float_as_uint(amax) >> 23) & 0xff);
  return e - 7 > 5 ? e - 7 : 5;
}

// The hi and lo E4M3 terms of one 32-value block (v in K order) as 8 words each (byte i of
// the 32 = value i), and the hi scale byte.
__device__ __forceinline__ void fp8_terms32(const float (&v)[32], uint32_t (&hi)[8], uint32_t (&lo)[8], int& s_hi) {
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i]));
  s_hi = fp8_term_exponent(amax);
  const float f = pow2_biased(254 - s_hi);  // 2^(127 - s): exact
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    float h[4], l[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) h[j] = v[4 * q + j] * f;
    const uint32_t w01 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(h[0], h[1], 0, false);
    const uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(h[2], h[3], (int)w01, true);
    l[0] = (h[0] - __builtin_amdgcn_cvt_f32_fp8((int)w, 0)) * 16.0f;
    l[1] = (h[1] - __builtin_amdgcn_cvt_f32_fp8((int)w, 1)) * 16.0f;
    l[2] = (h[2] - __builtin_amdgcn_cvt_f32_fp8((int)w, 2)) * 16.0f;
    l[3] = (h[3] - __builtin_amdgcn_cvt_f32_fp8((int)w, 3)) * 16.0f;
    const uint32_t u01 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(l[0], l[1], 0, false);
    hi[q] = w;
    lo[q] = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(l[2], l[3], (int)u01, true);
  }
}

// x [rows, H] bf16 -> E4M3 split rows: terms [rows][H/128][256 bytes], scales
// [rows][H/128] dwords. One lane per 32-value block. With g (bf16 [H]) also gate[row] =
// sigmoid(x[row] . g) as in split6_rows_kernel.
__global__ void __launch_bounds__(256) split8_rows_kernel(const uint16_t* __restrict__ x, int rows, int hidden,
                                                          uint8_t* __restrict__ x8, uint32_t* __restrict__ x8s,
                                                          const uint16_t* __restrict__ g, float* __restrict__ gate) {
  const int blocks = hidden / 32;
  const int64_t job = (int64_t)blockIdx.x * 256 + threadIdx.x;  // (row, block)
  if (job >= (int64_t)rows * blocks) return;
  const int64_t row = job / blocks;
  const int blk = (int)(job % blocks);
  const uint4* src = reinterpret_cast<const uint4*>(x + row * hidden + blk * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const uint4 u = src[q];
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[8 * q + 2 * j] = bf16_bits_to_f32(w[j] & 0xffffu);
      v[8 * q + 2 * j + 1] = bf16_bits_to_f32(w[j] >> 16);
    }
  }
  uint32_t hi[8], lo[8];
  int s_hi;
  fp8_terms32(v, hi, lo, s_hi);
  uint8_t* step = x8 + (row * (hidden / 128) + blk / 4) * XSTEP8;
  uint4* dh = reinterpret_cast<uint4*>(step + (blk % 4) * 32);
  uint4* dl = reinterpret_cast<uint4*>(step + 128 + (blk % 4) * 32);
  dh[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
  dh[1] = make_uint4(hi[4], hi[5], hi[6], hi[7]);
  dl[0] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
  dl[1] = make_uint4(lo[4], lo[5], lo[6], lo[7]);
  // the step's four blocks are lanes 4q .. 4q + 3: the quad's first lane stores their bytes
  const uint32_t sc = (uint32_t)s_hi;
  const uint32_t q1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0x55, 0xf, 0xf, false);
  const uint32_t q2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0xAA, 0xf, 0xf, false);
  const uint32_t q3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)sc, 0xFF, 0xf, 0xf, false);
  if (blk % 4 == 0) x8s[row * (hidden / 128) + blk / 4] = sc | (q1 << 8) | (q2 << 16) | (q3 << 24);
  if (g) {
    const uint4* gs = reinterpret_cast<const uint4*>(g + blk * 32);
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 u = gs[q];
      const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dot = fmaf(v[8 * q + 2 * j], bf16_bits_to_f32(w[j] & 0xffffu), dot);
        dot = fmaf(v[8 * q + 2 * j + 1], bf16_bits_to_f32(w[j] >> 16), dot);
      }
    }
    if (blocks == 64) {
      dot = segment_sum<64>(dot);
    } else {
      for (int off = 1; off < blocks; off <<= 1) dot += __shfl_xor(dot, off, 64);
    }
    if (blk == 0) gate[row] = 1.0f / (1.0f + __expf(-dot));
  }
}

// ---------------------------------------------------------------------------------
// Prefill tile layout of expert weights (one expert region; rows R, K values per row, P
// 16-byte pieces per row and 128-wide K step: MXFP4 4, FP8 8):
//   weights [K/128 steps][R/16 groups][P pieces][16 rows][16 bytes]: piece p of a row's step
//           is its bytes [16p, 16p + 16) of the 16 P the step takes in the row layout;
//   MXFP4 scales [K/128 steps][R rows][4 bytes]: the row's 4 E8M0 bytes of the step;
//   FP8 block scales copied unchanged: fp32 [R/128][K/128], or E8M0 bytes [R/32][K/32].
// One 16-byte piece (or one 4-byte scale word) per thread.
template <int P>
__global__ void __launch_bounds__(256) repack_prefill_kernel(const uint8_t* __restrict__ src,
                                                             const uint8_t* __restrict__ src_s, int64_t stride,
                                                             int64_t stride_s, const int32_t* __restrict__ slots,
                                                             int experts, int rows, int k, int64_t words,
                                                             uint8_t* __restrict__ dst, uint8_t* __restrict__ dst_s) {
  const int64_t row_pieces = (int64_t)(k / 128) * P;   // 16-byte pieces per row
  const int64_t row_bytes = 16 * row_pieces;
  const int64_t pieces = (int64_t)rows * row_pieces;   // per expert; `words`: scale words per expert
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= (int64_t)experts * (pieces + words)) return;
  const int e = (int)(i / (pieces + words));
  const int64_t j = i - (int64_t)e * (pieces + words);
  int64_t slot = slots ? slots[e] : e;
  if (slot < 0) slot = 0;
  if (j < pieces) {
    const int64_t row = j / row_pieces;
    const int64_t pr = j % row_pieces;
    const int64_t step = pr / P, p = pr % P;
    const uint4 v = *reinterpret_cast<const uint4*>(src + slot * stride + row * row_bytes + 16 * pr);
    *reinterpret_cast<uint4*>(dst + (int64_t)e * rows * row_bytes + step * rows * (16 * P) + (row / 16) * (256 * P) +
                              p * 256 + (row % 16) * 16) = v;
  } else if (P == 4) {
    const int64_t w = j - pieces;
    const int64_t row = w / (k / 128);
    const int step = (int)(w % (k / 128));
    const uint32_t v = *reinterpret_cast<const uint32_t*>(src_s + slot * stride_s + row * (k / 32) + 4 * step);
    *reinterpret_cast<uint32_t*>(dst_s + (int64_t)e * rows * (k / 32) + (int64_t)step * rows * 4 + row * 4) = v;
  } else {
    const int64_t w = j - pieces;
    const uint32_t v = *reinterpret_cast<const uint32_t*>(src_s + slot * stride_s + 4 * w);
    *reinterpret_cast<uint32_t*>(dst_s + 4 * ((int64_t)e * words + w)) = v;
  }
}

// A uniform int32 read through the scalar cache (data written by an earlier launch).
__device__ __forceinline__ int32_t scalar_i32(const int32_t* p, int idx) {
  typedef const __attribute__((address_space(4))) int32_t* cptr;
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return ((cptr)(((uint64_t)hi << 32) | lo))[idx];
}

// Row range and expert of logical row tile m through scalar loads only (a per-lane vector
// load would make the compiler wait for every load in flight, the ring's included).
__device__ __forceinline__ bool resolve_tile_s(const Lists& L, int m, int& expert, int& begin, int& end) {
  const int routed_tiles = scalar_i32(L.tile_count, 0);
  if (m < routed_tiles) {
    expert = scalar_i32(L.tiles, 2 * m);
    begin = scalar_i32(L.tiles, 2 * m + 1);
    end = min(begin + BM, scalar_i32(L.offsets, expert + 1));
    return true;
  }
  const int j = m - routed_tiles;
  if (!L.has_shared || j * BM >= L.tokens) return false;
  expert = -1;
  begin = L.pairs + j * BM;
  end = min(begin + BM, L.pairs + L.tokens);
  return true;
}

// (row tile, column tile) of logical work tile `logical`. With more than 4 column tiles
// the list is blocked by expert (the shared expert's row tiles are one more block) and
// column-major inside a block, so the row tiles that read the same weight columns run
// together on one XCD (one L2 fetch of the weights; C4: 11.8 -> 9.6 GB of gate_up HBM
// reads). With 4 or fewer it is row-major: a row tile's column tiles run together (its
// split rows stay in L2) while the W workgroups of an XCD still cover W / n_tiles row tiles
// of an expert at a time (measured faster for C3's down GEMM). Scalar loads only.
__device__ __forceinline__ void order_tile(const Lists& L, int logical, int n_tiles, int& mt, int& nt) {
  const int m0 = logical / n_tiles;
  if (n_tiles <= 4) {
    mt = m0;
    nt = logical - m0 * n_tiles;
    return;
  }
  const int routed = scalar_i32(L.tile_count, 0);
  int t0, c;
  if (m0 < routed) {
    const int e = scalar_i32(L.tiles, 2 * m0);
    const int begin = scalar_i32(L.tiles, 2 * m0 + 1);
    const int lo = scalar_i32(L.offsets, e), hi = scalar_i32(L.offsets, e + 1);
    t0 = m0 - (begin - lo) / BM;
    c = (hi - lo + BM - 1) / BM;
  } else {
    t0 = routed;
    c = (L.tokens + BM - 1) / BM;
  }
  const int local = logical - t0 * n_tiles;
  nt = local / c;
  mt = t0 + (local - nt * c);
}

__device__ __forceinline__ TileWeights tile_weights_s(const wm_mxfp4_experts& routed, const wm_mxfp4_experts& shared,
                                                      int expert) {
  const wm_mxfp4_experts& t = expert < 0 ? shared : routed;
  const int e = expert < 0 ? 0 : expert;
  int64_t slot = t.slots ? scalar_i32(t.slots, e) : e;
  if (slot < 0) slot = 0;  // an expert that is not resident: never address outside the pool
  return {(const uint8_t*)t.gate_up + slot * t.gate_up_stride,
          (const uint8_t*)t.gate_up_scales + slot * t.gate_up_scales_stride,
          (const uint8_t*)t.down + slot * t.down_stride, (const uint8_t*)t.down_scales + slot * t.down_scales_stride,
          t.up_first, t.swiglu_limit};
}

// ---------------------------------------------------------------------------------
// Grouped GEMMs on v_mfma_scale_f32_32x32x64_f8f6f4 against the E2M3 split rows, for
// MXFP4 weights (Mx4: fp4 x fp6 at twice the FP8 rate) and FP8-E4M3 weights with fp32
// 128 x 128 block scales (Mx8: fp8 x fp6 at the FP8 rate). A workgroup computes a 128-row
// x TW-weight-row tile with 8 waves: wave w = (wm, wn) = (w & 1, w >> 1) owns 64 rows
// (2 tiles of 32) and MI weight tiles of 32 rows. Each 128-wide K step's operands go
// straight from global memory into LDS (global_load_lds: lane i of a wave writes LDS
// base + 16 i).
//
// LDS (see RingMx): a ring of weight slots and a ring of split-row slots, one deeper than
// the other so the operand with the longer way from memory is loaded further ahead:
//   split rows: 128 rows x 208 bytes (one row's step), unswizzled; one load takes 4 rows
//     (52 lanes: row 4q + lane / 13, piece lane % 13), so each row's step arrives as one run;
//   weight rows: 16-row groups [PIECES][16 rows][16 bytes], a row's step being PIECES
//     16-byte pieces (fp4: 4, fp8: 8); one load fills 4 pieces of a group: in the prefill
//     tile layout one contiguous KB, in the row layout 64 contiguous bytes of each row;
//   MXFP4 weight scales: one dword per row (its 4 E8M0 bytes of the step). FP8 block scales
//     are one float per wave and step, read through the scalar cache.
//
// Operand layouts (32 x 32 x 64; lane l, r = l % 32, g = l / 32):
//   fp4 A: row r's K [32g, 32g + 32) as nibbles, 16 bytes;
//   fp8 A: row r's K [16g, 16g + 16) in bytes 0-15 and [32 + 16g, 32 + 16g + 16) in 16-31;
//   fp6 B: row r's K [32g, 32g + 32) as contiguous 6-bit fields, 24 bytes;
//   scale lane (r, g): K block g; result register i: D[8 (i / 4) + 4 g + i % 4][r].
// WAVES: waves per workgroup (4: one per SIMD, 8: two); MI = TW / (16 WAVES) weight tiles
// of 32 rows per wave; DA, DB: depths of the weight and split-row rings.
// Activation term formats of the split rows (the B operand):
//   E2M3 pairs: XS = 208 bytes per row and step, scales inside (read from LDS unswizzled);
//   E4M3 pairs (bf16-exact): 256 term bytes per row and step plus a scale dword from its own
//   array; in LDS the row's 16-byte pieces are XOR-swizzled by (row & 15), so the 8 rows one
//   ds_read_b128 cycle serves fall on distinct banks at the 256-byte pitch, and the scale
//   dwords follow the 128 rows.
struct TermsE2M3 {
  static constexpr bool E4 = false;
  static constexpr int XS = XSTEP, FMT = FMT_FP6, SLOT = BM * XSTEP;
};
struct TermsE4M3 {
  static constexpr bool E4 = true;
  static constexpr int XS = XSTEP8, FMT = FMT_FP8, SLOT = BM * XSTEP8 + BM * 4;
};

// FP8: the A operand is E4M3 bytes (else E2M1 nibbles). A_SCALED: E8M0 A scales are staged
// per weight row and step (4 bytes) and fed to the MFMA (MXFP4, and FP8 with E8M0 32 x 32
// blocks, whose rows of one 32-row block share their bytes); BLOCK_F32: FP8 with fp32
// 128 x 128 block scales, which cannot ride on the MFMA's E8M0 scales. Terms: the
// activation terms; the E4M3 variants hold two slots per ring (the deeper rings of the E2M3
// variants do not fit 160 KB beside 256-byte split rows).
struct Mx4 {
  static constexpr bool FP8 = false, A_SCALED = true, BLOCK_F32 = false;
  static constexpr int TW = 512, PIECES = 4, A_FMT = FMT_FP4, DA = 2, DB = 3, WAVES = 8, LW = 8;
  static constexpr int MI = TW / (16 * WAVES);
  using Terms = TermsE2M3;
};
struct Mx4x : Mx4 {
  static constexpr int DA = 2, DB = 2;
  using Terms = TermsE4M3;
};
struct Mx8 {
  static constexpr bool FP8 = true, A_SCALED = false, BLOCK_F32 = true;
  static constexpr int TW = 256, PIECES = 8, A_FMT = FMT_FP8, DA = 3, DB = 2, WAVES = 8, LW = 8;
  static constexpr int MI = TW / (16 * WAVES);
  using Terms = TermsE2M3;
};
struct Mx8x : Mx8 {
  static constexpr int DA = 2, DB = 2;
  using Terms = TermsE4M3;
};
struct Mx8e {
  static constexpr bool FP8 = true, A_SCALED = true, BLOCK_F32 = false;
  static constexpr int TW = 256, PIECES = 8, A_FMT = FMT_FP8, DA = 3, DB = 2, WAVES = 8, LW = 8;
  static constexpr int MI = TW / (16 * WAVES);
  using Terms = TermsE2M3;
};
struct Mx8ex : Mx8e {
  static constexpr int DA = 2, DB = 2;
  using Terms = TermsE4M3;
};
constexpr int NI4 = 2;      // 32-row row tiles per wave

// LDS of a workgroup: a ring of DA weight slots (a step's weight rows, then MXFP4 their
// scales) and a ring of DB split-row slots (128 rows x XSTEP bytes, unswizzled: XSTEP / 16 =
// 13 is odd, so the 8 rows one ds_read_b128 cycle serves fall on distinct banks). Step g
// uses weight slot g % DA and split-row slot g % DB; the deeper ring runs its loads further
// ahead (the operand with the longer way from memory).
template <typename F, int DA, int DB>
struct RingMx {
  static constexpr int A_BYTES = F::TW * F::PIECES * 16;
  static constexpr int A_SLOT = A_BYTES + (F::A_SCALED ? F::TW * 4 : 0);
  static constexpr int B_SLOT = F::Terms::SLOT;
  static constexpr int BYTES = DA * A_SLOT + DB * B_SLOT;
  static_assert(BYTES <= 160 * 1024, "LDS");
};

// Per-lane LDS read offsets. Weight tile mi of the wave is rows wave_row0 + mrow(mi) + r
// (multiples of 32 plus the lane's row); row tile ni is rows 64 wm + 32 ni + r. Half h of
// the step is K [64h, 64h + 64); the lane's K block in it is 2h + g.
// Split-row LDS offsets of tile row `row`: piece p (16 bytes) of an E4M3 row is stored at
// piece p ^ (row & 15); its scale dword is written by the loader at position
// 16 w + 4 i + d for row 4 (w + 8 i) + d (the wave that loads the row's terms).
__device__ __forceinline__ uint32_t e4_piece(int row, int p) { return (uint32_t)(row * XSTEP8 + 16 * (p ^ (row & 15))); }
// The gate_up epilogue stages the tile's E4M3 act rows at a 512-byte pitch (two steps), so
// the 16 rows one ds_write_b128 cycle serves would all hit the same 16 bytes of banks:
// piece q (0..15) of a row's staged step goes to q ^ (row & 15) instead.
__device__ __forceinline__ int e4_stage_piece(int row, int q) { return q ^ (row & 15); }
__device__ __forceinline__ uint32_t e4_scale(int row) {
  return (uint32_t)(BM * XSTEP8 + 4 * (16 * ((row / 4) % 8) + 4 * (row / 32) + row % 4));
}

template <typename F>
struct LaneMx {
  uint32_t a;        // + 16 PIECES mrow(mi) + (fp4: 512, fp8: 1024) h; fp8 second piece + 512
  uint32_t as;       // + 4 mrow(mi)
  uint32_t b[2][4];  // [h][piece]: E2M3 the 3 pieces of the lane's 48 bytes (+ 32 XSTEP ni);
                     // E4M3 hi K [64h + 16g, +16), hi K [64h + 32 + 16g, +16), then lo (+ 32 XSTEP8 ni)
  uint32_t bs[2];    // the row's scale bytes: E2M3 192..199 of the step (+ 32 XSTEP ni); E4M3 the
                     // scale dword of row tile ni
  uint32_t shift;    // 8 g
};

template <typename F>
__device__ __forceinline__ LaneMx<F> lane_mx(int wave_row0, int wm) {
  const int lane = threadIdx.x % 64, r = lane % 32, g = lane / 32;
  LaneMx<F> o;
  o.a = (uint32_t)((wave_row0 / 16 + r / 16) * (F::PIECES * 256) + 256 * g + 16 * (r % 16));
  o.as = (uint32_t)(4 * (wave_row0 + r));
  const int row = 64 * wm + r;
  if constexpr (F::Terms::E4) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      o.b[h][0] = e4_piece(row, 4 * h + g);
      o.b[h][1] = e4_piece(row, 4 * h + 2 + g);
      o.b[h][2] = e4_piece(row, 8 + 4 * h + g);
      o.b[h][3] = e4_piece(row, 8 + 4 * h + 2 + g);
    }
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) o.bs[ni] = e4_scale(row + 32 * ni);
  } else {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int e = 0; e < 3; ++e) o.b[h][e] = (uint32_t)(row * XSTEP + 16 * (6 * h + 3 * g + e));
      o.b[h][3] = 0;
    }
#pragma unroll
    for (int ni = 0; ni < 2; ++ni) o.bs[ni] = (uint32_t)((row + 32 * ni) * XSTEP + 192);
  }
  o.shift = (uint32_t)(8 * g);
  return o;
}

// One 128-wide K step of the wave's sub-tile. Per half: the MI A fragments, then per row
// tile its hi B fragment feeds MI MFMAs and its lo fragment MI more, so no MFMA waits on
// the one before it; between(g) follows group g = 2 h + ni (the next step's loads). FP8
// accumulates the step in blk and adds it times its block scale
// bscale(mi) (the fp32 scale cannot ride on the MFMA's E8M0 scales). AHEAD issues every
// split-row fragment read of a half before its first MFMA (held there by a scheduling
// barrier), where the compiler would otherwise sink the lo term's read behind the hi MFMAs
// and wait for it: 3% faster for the MXFP4 gate_up, slower where the extra registers spill
// (the down kernels) or for FP8.
template <typename F, bool AHEAD = false, typename MRow, typename BScale, typename Between>
__device__ __forceinline__ void step_mx(const uint8_t* sta, const uint8_t* stb, const LaneMx<F>& lo,
                                        v16f (&acc)[F::MI][NI4], MRow mrow, BScale bscale, Between between) {
  constexpr int A_BYTES = F::TW * F::PIECES * 16;
  constexpr int MI = F::MI;
  uint32_t sa[MI];
  uint2 sb[NI4];
  if constexpr (F::A_SCALED) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) sa[mi] = *reinterpret_cast<const uint32_t*>(sta + A_BYTES + lo.as + 4 * mrow(mi));
  }
#pragma unroll
  for (int ni = 0; ni < NI4; ++ni) {
    if constexpr (F::Terms::E4) {
      sb[ni].x = *reinterpret_cast<const uint32_t*>(stb + lo.bs[ni]);
      sb[ni].y = sb[ni].x - 0x04040404u;  // lo scales: hi - 4 (every hi scale byte is >= 5)
    } else {
      sb[ni] = *reinterpret_cast<const uint2*>(stb + lo.bs[ni]);
    }
  }
  v16f blk[F::BLOCK_F32 ? MI : 1][NI4];
  // FP8 block scales (scalar loads) issued before the MFMAs, so their memory round trip
  // overlaps the step instead of stalling the scale-and-add at its end
  float bs[F::BLOCK_F32 ? MI : 1];
  if constexpr (F::BLOCK_F32) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) bs[mi] = bscale(mi);
  }
  if constexpr (F::BLOCK_F32) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI4; ++ni)
#pragma unroll
        for (int i = 0; i < 16; ++i) blk[mi][ni][i] = 0.0f;
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint32_t sh = lo.shift + 16u * (uint32_t)h;
    v8i a[MI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      if constexpr (F::FP8) {
        const uint8_t* p = sta + lo.a + 128 * mrow(mi) + 1024 * h;
        const uint4 v0 = *reinterpret_cast<const uint4*>(p);
        const uint4 v1 = *reinterpret_cast<const uint4*>(p + 512);
        a[mi] = v8i{(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
      } else {
        const uint4 v = *reinterpret_cast<const uint4*>(sta + lo.a + 64 * mrow(mi) + 512 * h);
        a[mi] = v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
      }
    }
    constexpr int NP = F::Terms::E4 ? 4 : 3;               // 16-byte B pieces per row tile and half
    constexpr uint32_t TSTEP = 32 * F::Terms::XS;           // LDS bytes between the two row tiles
    uint4 bq[NI4][NP];
    if constexpr (AHEAD) {
#pragma unroll
      for (int ni = 0; ni < NI4; ++ni)
#pragma unroll
        for (int e = 0; e < NP; ++e) bq[ni][e] = *reinterpret_cast<const uint4*>(stb + lo.b[h][e] + TSTEP * ni);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int ni = 0; ni < NI4; ++ni) {
      uint4 b[NP];
#pragma unroll
      for (int e = 0; e < NP; ++e) {
        if constexpr (AHEAD)
          b[e] = bq[ni][e];
        else
          b[e] = *reinterpret_cast<const uint4*>(stb + lo.b[h][e] + TSTEP * ni);
      }
      v8i bh, bl;
      if constexpr (F::Terms::E4) {
        bh = v8i{(int)b[0].x, (int)b[0].y, (int)b[0].z, (int)b[0].w, (int)b[1].x, (int)b[1].y, (int)b[1].z, (int)b[1].w};
        bl = v8i{(int)b[2].x, (int)b[2].y, (int)b[2].z, (int)b[2].w, (int)b[3].x, (int)b[3].y, (int)b[3].z, (int)b[3].w};
      } else {
        bh = v8i{(int)b[0].x, (int)b[0].y, (int)b[0].z, (int)b[0].w, (int)b[1].x, (int)b[1].y, 0, 0};
        bl = v8i{(int)b[1].z, (int)b[1].w, (int)b[2].x, (int)b[2].y, (int)b[2].z, (int)b[2].w, 0, 0};
      }
      const int sbh = (int)(sb[ni].x >> sh), sbl = (int)(sb[ni].y >> sh);
      if constexpr (F::BLOCK_F32) {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          blk[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], bh, blk[mi][ni], FMT_FP8, F::Terms::FMT,
                                                                        0, 127, 0, sbh);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          blk[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], bl, blk[mi][ni], FMT_FP8, F::Terms::FMT,
                                                                        0, 127, 0, sbl);
      } else {
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], bh, acc[mi][ni], F::A_FMT,
                                                                        F::Terms::FMT, 0, (int)(sa[mi] >> sh), 0, sbh);
#pragma unroll
        for (int mi = 0; mi < MI; ++mi)
          acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[mi], bl, acc[mi][ni], F::A_FMT,
                                                                        F::Terms::FMT, 0, (int)(sa[mi] >> sh), 0, sbl);
      }
      __builtin_amdgcn_sched_barrier(0);
      between(2 * h + ni);
    }
  }
  if constexpr (F::BLOCK_F32) {
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      const float s = bs[mi];
#pragma unroll
      for (int ni = 0; ni < NI4; ++ni)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mi][ni][i] = fmaf(s, blk[mi][ni][i], acc[mi][ni][i]);
    }
  }
}

// Per-lane sources of one K step's loads: split rows, loads q = w + 8i (i = 0..3) of 52
// lanes, rows 4q + lane / 13, piece lane % 13 (LDS: slot + 832 q + 16 lane); weights, loads
// q = w + 8i (fp4: group q; fp8: group q / 2, pieces 4 (q % 2)..); MXFP4 scales, rows
// 64 w + lane. Offsets are taken at step 0; step ks adds ks * XSTEP, ks * a_step and
// ks * s_step.
template <typename F>
struct LoaderMx {
  const uint8_t* b;
  const uint8_t* bsbase;  // E4M3 terms: the split rows' scale dwords
  const uint8_t* wbase;
  const uint8_t* sbase;
  static constexpr int NQ = 32 / F::LW;                // 1 KB loads per wave and operand
  // E4M3 terms: one scale load per wave and step (lanes 0..15, the scale dwords of the
  // wave's 16 term rows), counted like the A scales
  static constexpr int SQB = F::Terms::E4 ? 1 : 0;
  // A scales: one load per wave and step, a dword (4 E8M0 bytes) per weight row, wave w
  // taking rows RPWS w + lane for lane < RPWS. Every wave issues it (lanes past RPWS masked),
  // so every wave has the same loads in flight when the step's ring wait counts them.
  static constexpr int SQ = F::A_SCALED ? 1 : 0;
  static constexpr int RPWS = F::TW / F::LW;
  static_assert(!F::A_SCALED || RPWS <= 64, "one scale load per wave covers the tile's rows");
  uint32_t boff[NQ];
  uint32_t bsoff;
  uint32_t aoff[NQ];
  uint32_t soff[SQ > 0 ? SQ : 1];
  uint32_t a_step, s_step;

  // Half h (0, 1) of step ks's weight loads into weight slot `slot`: NQ / 2 loads, and for
  // MXFP4 with h = 1 the scale loads (NQ + SQ instructions per step).
  __device__ __forceinline__ void issue_a(uint8_t* slot, int ks, int h) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    if (F::LW < F::WAVES && w >= F::LW) return;
#pragma unroll
    for (int i = h * NQ / 2; i < (h + 1) * NQ / 2; ++i)
      dma16(wbase, aoff[i] + (uint32_t)ks * a_step, lds_addr(slot + (w + F::LW * i) * 1024));
    if (SQ && h == 1 && threadIdx.x % 64 < RPWS)
      dma4(sbase, soff[0] + (uint32_t)ks * s_step, lds_addr(slot + F::TW * F::PIECES * 16 + 4 * RPWS * w));
  }
  // Half h of step ks's split-row loads into split-row slot `slot` (NQ + SQB instructions
  // per step): E2M3 rows 4 to a load (52 lanes x 16 bytes), E4M3 rows 4 to a load (64 lanes)
  // and with h = 1 the scale dwords of the wave's rows.
  __device__ __forceinline__ void issue_b(uint8_t* slot, int ks, int h) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    if (F::LW < F::WAVES && w >= F::LW) return;
    if constexpr (F::Terms::E4) {
#pragma unroll
      for (int i = h * NQ / 2; i < (h + 1) * NQ / 2; ++i)
        dma16(b, boff[i] + (uint32_t)ks * XSTEP8, lds_addr(slot + (w + F::LW * i) * 1024));
      if (h == 1 && threadIdx.x % 64 < 16) dma4(bsbase, bsoff + (uint32_t)ks * 4, lds_addr(slot + BM * XSTEP8 + 64 * w));
    } else {
#pragma unroll
      for (int i = h * NQ / 2; i < (h + 1) * NQ / 2; ++i)
        if (threadIdx.x % 64 < 52) dma16(b, boff[i] + (uint32_t)ks * XSTEP, lds_addr(slot + (w + F::LW * i) * 832));
    }
  }
};

// The split-row part of a loader: row_index(r) is the split row (a token, or a permuted
// row) of tile row r, called with wave-uniform r only (it may use scalar loads); row_bytes
// and srow_bytes are a split row's bytes in the term and (E4M3) scale arrays. A wave loads
// tile rows 4 (w + 8 i) + d, d = 0..3: E2M3 lanes 13 d + piece, E4M3 lanes 16 d + piece with
// the piece swizzled by (row & 15), and E4M3 scale lane 4 i + d.
template <typename F, typename RowIndex>
__device__ __forceinline__ void split_row_offsets(LoaderMx<F>& ld, RowIndex row_index, uint32_t row_bytes,
                                                  uint32_t srow_bytes) {
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
  ld.bsoff = 0;
#pragma unroll
  for (int i = 0; i < LoaderMx<F>::NQ; ++i) {
    const int q0 = 4 * (w + F::LW * i);
    int idx[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) idx[d] = row_index(q0 + d);
    if constexpr (F::Terms::E4) {
      const int d = lane / 16, piece = (lane % 16) ^ ((q0 + d) & 15);
      const int mine = d == 0 ? idx[0] : d == 1 ? idx[1] : d == 2 ? idx[2] : idx[3];
      ld.boff[i] = (uint32_t)mine * row_bytes + 16u * (uint32_t)piece;
      const int sd = lane % 4;
      const int srow = sd == 0 ? idx[0] : sd == 1 ? idx[1] : sd == 2 ? idx[2] : idx[3];
      if (lane / 4 == i) ld.bsoff = (uint32_t)srow * srow_bytes;
    } else {
      const int d = lane < 52 ? lane / 13 : 3, piece = lane < 52 ? lane % 13 : 0;
      const int mine = d == 0 ? idx[0] : d == 1 ? idx[1] : d == 2 ? idx[2] : idx[3];
      ld.boff[i] = (uint32_t)mine * row_bytes + 16u * (uint32_t)piece;
    }
  }
}

// The weight part: tile rows [0, TW) are expert rows row_of(j) (multiples of 16 in runs of
// 16, so a tile group is an expert group); rows is the expert region's row count, k its K.
template <typename F, typename RowOf>
__device__ __forceinline__ void weight_offsets(LoaderMx<F>& ld, const uint8_t* w_region, const uint8_t* s_region,
                                               int rows, int k, int tiled, RowOf row_of) {
  const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
  ld.wbase = uniform_u8(w_region);
  ld.sbase = uniform_u8(s_region);
  constexpr int NQ = LoaderMx<F>::NQ, SQ = LoaderMx<F>::SQ;
  if constexpr (F::FP8) {
    if (tiled) {
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int q = w + F::LW * i;
        ld.aoff[i] = (uint32_t)(row_of(16 * (q / 2)) / 16 * 2048 + 1024 * (q % 2) + 16 * lane);
      }
      ld.a_step = (uint32_t)(rows * 128);
    } else {  // row layout: [rows][k] bytes, 128 per step
#pragma unroll
      for (int i = 0; i < NQ; ++i) {
        const int q = w + F::LW * i;
        ld.aoff[i] = (uint32_t)(row_of(16 * (q / 2) + lane % 16) * k + 16 * (4 * (q % 2) + lane / 16));
      }
      ld.a_step = 128;
    }
    if constexpr (F::A_SCALED) {  // E8M0 32 x 32 blocks, [rows / 32][k / 32] bytes in either layout
      constexpr int RPWS = LoaderMx<F>::RPWS;
      ld.soff[0] = lane < RPWS ? (uint32_t)(row_of(RPWS * w + lane) / 32 * (k / 32)) : 0u;
      ld.s_step = 4;
    } else {
      ld.soff[0] = 0;
      ld.s_step = 0;
    }
  } else if (tiled) {
#pragma unroll
    for (int i = 0; i < NQ; ++i) ld.aoff[i] = (uint32_t)(row_of(16 * (w + F::LW * i)) / 16 * 1024 + 16 * lane);
    constexpr int RPWS = LoaderMx<F>::RPWS;
    ld.soff[0] = lane < RPWS ? (uint32_t)(row_of(RPWS * w + lane) * 4) : 0u;
    ld.a_step = (uint32_t)(rows * 64);
    ld.s_step = (uint32_t)(rows * 4);
  } else {
#pragma unroll
    for (int i = 0; i < NQ; ++i)
      ld.aoff[i] = (uint32_t)(row_of(16 * (w + F::LW * i) + lane % 16) * (k / 2) + 16 * (lane / 16));
    constexpr int RPWS = LoaderMx<F>::RPWS;
    ld.soff[0] = lane < RPWS ? (uint32_t)(row_of(RPWS * w + lane) * (k / 32)) : 0u;
    ld.a_step = 64;
    ld.s_step = 4;
  }
}

template <typename F>
struct TileMx {
  LoaderMx<F> ld;
  int begin, end, nt, valid;
  float limit;
  const_f32_ptr s0, s1;  // FP8: block scale rows of the wave's weight tiles (gate / up, or down)
};

template <typename F>
__device__ __forceinline__ void zero_acc(v16f (&acc)[F::MI][NI4]) {
#pragma unroll
  for (int mi = 0; mi < F::MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI4; ++ni)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mi][ni][i] = 0.0f;
}

// Every wave's LDS reads of the stage have returned (the epilogue may overwrite it).
__device__ __forceinline__ void stage_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// This wave's LDS writes are done before its next LDS reads (and its reads before its writes).
__device__ __forceinline__ void wave_lds_fence() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// The ring wait leaving this wave's last N vector memory instructions (the deeper ring's
// loads of the previous step) in flight: loads complete in issue order, and no store may
// be outstanding.
template <int N>
__device__ __forceinline__ void ring_wait_keep();
template <>
__device__ __forceinline__ void ring_wait_keep<4>() {
  asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <>
__device__ __forceinline__ void ring_wait_keep<5>() {
  asm volatile("s_waitcnt vmcnt(5) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <>
__device__ __forceinline__ void ring_wait_keep<8>() {
  asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
template <>
__device__ __forceinline__ void ring_wait_keep<10>() {
  asm volatile("s_waitcnt vmcnt(10) lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Persistent K loop over this workgroup's tiles, as one flat sequence of 128-wide steps.
// Step g reads weight slot g % DA and split-row slot g % DB. At the top of step g every
// wave has step g's loads landed and is done with step g - 1's slots; the shallower ring
// then loads step g + 1 into its freed slot and the deeper ring (depth D) step g + D - 1
// (a tile's later step, or the next tile's first steps), each in two halves issued at the
// top of the step or between its MFMA groups, the deeper ring's last. With K steps fewer than D the
// deeper ring also loads one step ahead. The next tile is set up (index loads, load
// offsets) after the MFMAs of the step before its first loads; after an epilogue (whose
// stores may complete out of order with loads) the top waits for everything.
//   setup(j, tile) -> bool: fills tile j's state; false for a tile with no rows
//   mfma(tile, wslot, rslot, k, load_part): step k of a tile, calling load_part(p) for
//     p = 0..3 between its MFMAs
//   epilogue(tile, wslot, rslot): after a tile's last step (its two slots are free)
template <typename F, int DA, int DB, typename Tile, typename Setup, typename Mfma, typename Epilogue>
__device__ __forceinline__ void persistent_tiles(const TileRange& tr, int steps, uint8_t* lds, Setup setup, Mfma mfma,
                                                 Epilogue epilogue) {
  using R = RingMx<F, DA, DB>;
  constexpr bool A_DEEP = DA > DB;
  constexpr int D = A_DEEP ? DA : DB, DS = A_DEEP ? DB : DA;
  // deeper ring's load instructions per wave and step
  constexpr int N_DEEP = LoaderMx<F>::NQ + (A_DEEP ? LoaderMx<F>::SQ : LoaderMx<F>::SQB);
  if (tr.count == 0) return;
  const int la = steps >= D ? D - 1 : 1;  // deeper ring's lookahead
  auto wslot = [&](int i) { return lds + i * R::A_SLOT; };
  auto rslot = [&](int i) { return lds + DA * R::A_SLOT + i * R::B_SLOT; };
  // half h of tile t's step ks into slot i of the deeper (deep) or shallower ring
  auto issue = [&](Tile& t, bool deep, int i, int ks, int h) {
    if (deep == A_DEEP)
      t.ld.issue_a(wslot(i), ks, h);
    else
      t.ld.issue_b(rslot(i), ks, h);
  };
  Tile cur, nxt;
  bool cur_ok = setup(0, cur), nxt_ok = false;
  if (cur_ok) {
#pragma unroll
    for (int h = 0; h < 2; ++h) issue(cur, false, 0, 0, h);
    for (int d = 0; d < la; ++d)
#pragma unroll
      for (int h = 0; h < 2; ++h) issue(cur, true, d, d, h);
  }
  const int total = tr.count * steps;
  bool deep_last = false;  // the previous step's last loads were the deeper ring's
  for (int g = 0; g < total; ++g) {
    const int j = g / steps, k = g - j * steps;
    if (k != 0 && la >= 2 && deep_last)
      ring_wait_keep<N_DEEP>();
    else
      ring_wait_all();
    // targets: 0 none, 1 this tile, 2 the next tile
    const bool more = j + 1 < tr.count && nxt_ok;
    const int ts = k + 1 < steps ? (cur_ok ? 1 : 0) : (more ? 2 : 0);
    const int kd = k + la;
    const int td = kd < steps ? (cur_ok ? 1 : 0) : (more ? 2 : 0);
    const int ks_s = k + 1 < steps ? k + 1 : 0, ks_d = kd < steps ? kd : kd - steps;
    const int sl_s = (g + 1) % DS, sl_d = (g + la) % D;
    // half h of the deeper (deep) or shallower ring's loads of this step
    auto part = [&](bool deep, int h) {
      const int t = deep ? td : ts;
      if (t == 1)
        issue(cur, deep, deep ? sl_d : sl_s, deep ? ks_d : ks_s, h);
      else if (t == 2)
        issue(nxt, deep, deep ? sl_d : sl_s, deep ? ks_d : ks_s, h);
    };
    // Rings of equal depth (the shallower one is then the weight ring): one operand's halves
    // at the top of the step and the other's after MFMA groups 0 and 1; FP8 weights (32 KB a
    // step) go first, and with MXFP4 weights (16 KB and their scales) the split rows do.
    // Otherwise the shallower ring's halves after groups 0 and 1 and the deeper ring's after
    // groups 2 and 3, so the deeper ring's loads are the last ones the ring wait leaves in
    // flight.
    constexpr bool EQUAL = DA == DB, SPLIT_FIRST = !F::FP8;
    auto load_part = [&](int p) {
      if (EQUAL && cur_ok) {
        if (p < 2) part(!SPLIT_FIRST, p);
      } else {
        part(p >= 2, p & 1);
      }
    };
    if (EQUAL && cur_ok) {
      part(SPLIT_FIRST, 0);
      part(SPLIT_FIRST, 1);
    }
    if (cur_ok) {
      mfma(cur, wslot(g % DA), rslot(g % DB), k, load_part);
    } else {
#pragma unroll
      for (int p = 0; p < 4; ++p) load_part(p);
    }
    deep_last = td != 0;
    if (k == steps - la - 1 && j + 1 < tr.count) nxt_ok = setup(j + 1, nxt);
    if (k == steps - 1) {
      if (cur_ok) epilogue(cur, wslot(g % DA), rslot(g % DB));
      if (steps == 1 && j + 1 < tr.count) {
        nxt_ok = setup(j + 1, nxt);
        if (nxt_ok) {
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            issue(nxt, false, (g + 1) % DS, 0, h);
            issue(nxt, true, (g + 1) % D, 0, h);
          }
        }
      }
      cur = nxt;
      cur_ok = nxt_ok;
      nxt_ok = false;
    }
  }
}

// The expert regions of a tile (scalar loads only).
__device__ __forceinline__ TileWeights tile_weights_s(const wm_fp8_experts& routed, const wm_fp8_experts& shared,
                                                      int expert) {
  const wm_fp8_experts& t = expert < 0 ? shared : routed;
  const int e = expert < 0 ? 0 : expert;
  int64_t slot = t.slots ? scalar_i32(t.slots, e) : e;
  if (slot < 0) slot = 0;
  return {(const uint8_t*)t.w13 + slot * t.w13_stride, (const uint8_t*)t.w13_scales + slot * t.w13_scales_stride,
          (const uint8_t*)t.w2 + slot * t.w2_stride, (const uint8_t*)t.w2_scales + slot * t.w2_scales_stride,
          t.up_first, t.swiglu_limit};
}
__device__ __forceinline__ int table_tiled(const wm_mxfp4_experts& t) { return t.tiled; }
__device__ __forceinline__ int table_tiled(const wm_fp8_experts& t) { return t.tiled; }

// gate_up: act rows of a tile's TG = TW / 2 intermediate columns; weight tile rows [0, TG)
// are the gate rows nt * TG + j, [TG, TW) the matching up rows; wave wn owns gate rows
// 32 (MI / 2) wn + [0, 32 MI / 2) (mi < MI / 2) and the same up rows (mi >= MI / 2).
// x6 / a6: the split rows' terms (and, E4M3, x6s / a6s their scale dwords).
template <typename F, int DA, int DB, typename Table>
__global__ void __launch_bounds__(64 * F::WAVES, F::WAVES / 4) gate_up_mx_kernel(const uint8_t* __restrict__ x6,
                                                                 const uint8_t* __restrict__ x6s,
                                                                 const int32_t* __restrict__ row_token, Lists L,
                                                                 Table routed, Table shared, uint8_t* __restrict__ a6,
                                                                 uint32_t* __restrict__ a6s) {
  constexpr int TG = F::TW / 2, MI = F::MI, HM = MI / 2;
  constexpr int XS = F::Terms::XS;
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = (I + TG - 1) / TG;
  const TileRange tr = tile_range(active_row_tiles(L) * n_tiles);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave & 1, wn = wave >> 1;
  const LaneMx<F> lo = lane_mx<F>(32 * HM * wn, wm);
  const uint32_t x_row = (uint32_t)(H / 128 * XS);
  const int64_t a_row = (int64_t)(I / 128) * XS;
  using Tile = TileMx<F>;

  auto setup = [&](int j, Tile& t) {
    int mt = 0;
    order_tile(L, tr.first + tr.stride * j, n_tiles, mt, t.nt);
    int expert = 0, begin = 0, end = 0;
    if (!resolve_tile_s(L, mt, expert, begin, end)) return false;
    t.begin = begin;
    t.end = end;
    const TileWeights tw = tile_weights_s(routed, shared, expert);
    t.limit = tw.limit;
    t.valid = min(TG, I - t.nt * TG);  // a multiple of 128
    const int gate0 = (tw.up_first ? I : 0) + t.nt * TG;
    const int up0 = (tw.up_first ? 0 : I) + t.nt * TG;
    const int valid = t.valid;
    weight_offsets<F>(t.ld, tw.w13, tw.w13s, 2 * I, H, table_tiled(expert < 0 ? shared : routed),
                      [gate0, up0, valid](int r) {
                        const int rr = r % TG;
                        return (r < TG ? gate0 : up0) + (rr < valid ? rr : rr % valid);
                      });
    if constexpr (F::BLOCK_F32) {  // a wave's gate (up) rows lie in one 128-row scale block
      t.s0 = uniform_ptr(reinterpret_cast<const float*>(tw.w13s) + (int64_t)(gate0 / 128) * (H / 128));
      t.s1 = uniform_ptr(reinterpret_cast<const float*>(tw.w13s) + (int64_t)(up0 / 128) * (H / 128));
    }
    t.ld.b = uniform_u8(x6);
    if constexpr (F::Terms::E4) t.ld.bsbase = uniform_u8(x6s);
    // the tokens of the tile's split rows, through scalar loads
    split_row_offsets<F>(
        t.ld, [&](int r) { return scalar_i32(row_token, begin + r < end ? begin + r : begin); }, x_row,
        (uint32_t)(H / 128 * 4));
    return true;
  };

  v16f acc[MI][NI4];
  zero_acc<F>(acc);
  auto mrow = [](int mi) { return (mi < HM ? 0 : TG) + 32 * (mi % HM); };
  auto mfma = [&](const Tile& t, const uint8_t* wa, const uint8_t* rb, int k, auto load_part) {
    step_mx<F, !F::FP8 && !F::Terms::E4>(wa, rb, lo, acc, mrow, [&](int mi) { return mi < HM ? t.s0[k] : t.s1[k]; }, load_part);
  };

  // Epilogue: lane (r, half) holds act rows 8 j + 4 half + q (j, q = 0..3; register 4 j + q)
  // of a 32-column block for row 64 wm + 32 ni + r. One swap between the lane halves gives
  // each lane a whole block: for MXFP4 (two gate tiles per wave) blocks 2 wn + half of row
  // tile ni, for FP8 (one gate tile) block wn of row tile half. The lane forms the block's
  // two terms and writes them with the scales into the consumed stage as the tile's act
  // rows (TG / 128 steps of 208 bytes), which all threads then copy out row by row.
  auto epilogue = [&](const Tile& t, uint8_t* wa, uint8_t* rb) {
    constexpr int STG = TG / 128 * XS;  // staged bytes per row: rows 0..63 in the split-row slot
    stage_barrier();                    // (64 STG = its size for MXFP4), 64..127 in the weight slot
    auto srow = [&](int lr) { return lr < 64 ? rb + lr * STG : wa + (lr - 64) * STG; };
    // E4M3: the row's scale dwords (TG / 128 of them) after the 64 rows' terms of its slot
    auto sscale = [&](int lr) { return (lr < 64 ? rb : wa) + 64 * STG + (lr % 64) * (TG / 128) * 4; };
    if (32 * HM * wn < t.valid) {
      const int r = lane % 32, half = lane / 32;
      auto act = [&](int b, int ni, int i) {
        float gv = acc[b][ni][i], uv = acc[b + HM][ni][i];
        if (t.limit > 0.0f) {
          gv = fminf(gv, t.limit);
          uv = fminf(fmaxf(uv, -t.limit), t.limit);
        }
        return silu(gv) * uv;
      };
      // HM >= 2: the swap pairs gate tiles (2p, 2p + 1) of row tile ni, lane half h taking
      // tile 2p + h; HM = 1: it pairs row tiles 0 and 1 of the one gate tile
      constexpr int PAIRS = HM >= 2 ? NI4 * HM / 2 : 1;
#pragma unroll
      for (int pi = 0; pi < PAIRS; ++pi) {
        const int ni = HM >= 2 ? pi / (HM / 2) : 0, p = HM >= 2 ? pi % (HM / 2) : 0;
        float full[32];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float x0 = HM >= 2 ? act(2 * p, ni, i) : act(0, 0, i);
          const float x1 = HM >= 2 ? act((2 * p + 1) % HM, ni, i) : act(0, 1, i);
          const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(x0), __float_as_uint(x1), false, false);
          full[8 * (i / 4) + i % 4] = __uint_as_float(pr[0]);
          full[8 * (i / 4) + 4 + i % 4] = __uint_as_float(pr[1]);
        }
        const int lr = HM >= 2 ? 64 * wm + 32 * ni + r : 64 * wm + 32 * half + r;
        const int kb = HM >= 2 ? HM * wn + 2 * p + half : wn;  // block of the tile: step kb / 4, block kb % 4
        uint8_t* step = srow(lr) + (kb / 4) * XS;
        if constexpr (F::Terms::E4) {
          uint32_t hi[8], lo8[8];
          int s_hi;
          fp8_terms32(full, hi, lo8, s_hi);
          // 16-byte piece q of a staged step at q ^ (lr & 15) (see e4_stage_piece)
          const int q0 = 2 * (kb % 4);
          auto piece = [&](int q) { return reinterpret_cast<uint4*>(step + 16 * e4_stage_piece(lr, q)); };
          *piece(q0) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
          *piece(q0 + 1) = make_uint4(hi[4], hi[5], hi[6], hi[7]);
          *piece(8 + q0) = make_uint4(lo8[0], lo8[1], lo8[2], lo8[3]);
          *piece(8 + q0 + 1) = make_uint4(lo8[4], lo8[5], lo8[6], lo8[7]);
          sscale(lr)[kb] = (uint8_t)s_hi;  // byte kb % 4 of the row's dword kb / 4
        } else {
          v6u_t hi, lo6;
          int s_hi, s_lo;
          fp6_terms32(full, hi, lo6, s_hi, s_lo);
          uint4* dst = reinterpret_cast<uint4*>(step + (kb % 4) * 48);
          dst[0] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
          dst[1] = make_uint4(hi[4], hi[5], lo6[0], lo6[1]);
          dst[2] = make_uint4(lo6[2], lo6[3], lo6[4], lo6[5]);
          step[192 + kb % 4] = (uint8_t)s_hi;
          step[196 + kb % 4] = (uint8_t)s_lo;
        }
      }
    }
    stage_barrier();
    const int chunks = t.valid / 128 * (XS / 16);  // 16-byte pieces of a row's act steps
    const int n = (t.end - t.begin) * chunks;
    for (int idx = threadIdx.x; idx < n; idx += 64 * F::WAVES) {
      const int lr = idx / chunks, c = idx - lr * chunks;
      const int cs = F::Terms::E4 ? (c & ~15) | e4_stage_piece(lr, c & 15) : c;
      const uint4 v4 = *reinterpret_cast<const uint4*>(srow(lr) + 16 * cs);
      *reinterpret_cast<uint4*>(a6 + (int64_t)(t.begin + lr) * a_row + (int64_t)(t.nt * TG / 128) * XS + 16 * c) = v4;
    }
    if constexpr (F::Terms::E4) {
      const int steps = t.valid / 128;
      const int ns = (t.end - t.begin) * steps;
      for (int idx = threadIdx.x; idx < ns; idx += 64 * F::WAVES) {
        const int lr = idx / steps, j = idx - lr * steps;
        a6s[(int64_t)(t.begin + lr) * (I / 128) + t.nt * TG / 128 + j] =
            *reinterpret_cast<const uint32_t*>(sscale(lr) + 4 * j);
      }
    }
    zero_acc<F>(acc);
  };

  __shared__ __attribute__((aligned(16))) uint8_t lds[RingMx<F, DA, DB>::BYTES];
  persistent_tiles<F, DA, DB, Tile>(tr, H / 128, lds, setup, mfma, epilogue);
}

// down: out[row, n] = act[row] . W2[n], bf16, permuted rows (the combine applies the routing
// weights); tile = 128 rows x TW output columns, wave wn owns columns 32 MI wn + [0, 32 MI).
template <typename F, int DA, int DB, typename Table>
__global__ void __launch_bounds__(64 * F::WAVES, F::WAVES / 4) down_mx_kernel(const uint8_t* __restrict__ a6,
                                                              const uint8_t* __restrict__ a6s, Lists L, Table routed,
                                                              Table shared, uint16_t* __restrict__ out) {
  constexpr int MI = F::MI;
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = (H + F::TW - 1) / F::TW;
  const TileRange tr = tile_range(active_row_tiles(L) * n_tiles);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave & 1, wn = wave >> 1;
  const LaneMx<F> lo = lane_mx<F>(32 * MI * wn, wm);
  const uint32_t a_row = (uint32_t)(I / 128 * F::Terms::XS);
  using Tile = TileMx<F>;

  auto setup = [&](int j, Tile& t) {
    int mt = 0;
    order_tile(L, tr.first + tr.stride * j, n_tiles, mt, t.nt);
    int expert = 0, begin = 0, end = 0;
    if (!resolve_tile_s(L, mt, expert, begin, end)) return false;
    t.begin = begin;
    t.end = end;
    const TileWeights tw = tile_weights_s(routed, shared, expert);
    t.valid = min(F::TW, H - t.nt * F::TW);  // a multiple of 128
    const int nt = t.nt, valid = t.valid;
    auto col_row = [nt, valid](int r) { return nt * F::TW + (r < valid ? r : r % valid); };  // never past H
    weight_offsets<F>(t.ld, tw.w2, tw.w2s, H, I, table_tiled(expert < 0 ? shared : routed), col_row);
    if constexpr (F::BLOCK_F32)  // the wave's columns lie in one 128-row scale block
      t.s0 = t.s1 = uniform_ptr(reinterpret_cast<const float*>(tw.w2s) +
                                (int64_t)(col_row(32 * MI * wn) / 128) * (I / 128));
    t.ld.b = uniform_u8(a6);
    if constexpr (F::Terms::E4) t.ld.bsbase = uniform_u8(a6s);
    split_row_offsets<F>(t.ld, [&](int r) { return begin + r < end ? begin + r : begin; }, a_row,
                         (uint32_t)(I / 128 * 4));
    return true;
  };

  v16f acc[MI][NI4];
  zero_acc<F>(acc);
  auto mfma = [&](const Tile& t, const uint8_t* wa, const uint8_t* rb, int k, auto load_part) {
    step_mx<F>(wa, rb, lo, acc, [](int mi) { return 32 * mi; }, [&](int) { return t.s0[k]; }, load_part);
  };

  // Epilogue: lane (r, half) holds output columns nt * TW + 32 MI wn + 32 mi + 8 j + 4 half + q
  // (register 4 j + q) of row 64 wm + 32 ni + r. Each wave turns 32 rows x 64 columns at a
  // time around in its own slice of the consumed stage (rows of 144 bytes) and stores each
  // row's 128 bytes as 8 lanes x 16.
  auto epilogue = [&](const Tile& t, uint8_t* wa, uint8_t* rb) {
    stage_barrier();
    if (32 * MI * wn < t.valid) {
      // waves 0..5 in the weight slot, 6 and 7 in the split-row slot
      uint8_t* slice = wave < 6 ? wa + wave * 4608 : rb + (wave - 6) * 4608;
      const int r = lane % 32, half = lane / 32;
#pragma unroll
      for (int ni = 0; ni < NI4; ++ni)
#pragma unroll
        for (int mp = 0; mp < MI / 2; ++mp) {
#pragma unroll
          for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              const v16f& a = acc[2 * mp + m][ni];
              uint2 o;
              o.x = pack_bf16x2(a[4 * j], a[4 * j + 1]);
              o.y = pack_bf16x2(a[4 * j + 2], a[4 * j + 3]);
              *reinterpret_cast<uint2*>(slice + r * 144 + 64 * m + 16 * j + 8 * half) = o;
            }
          wave_lds_fence();
#pragma unroll
          for (int it = 0; it < 4; ++it) {
            const int rr = lane / 8 + 8 * it, c = lane % 8;
            const uint4 v4 = *reinterpret_cast<const uint4*>(slice + rr * 144 + 16 * c);
            const int row = t.begin + 64 * wm + 32 * ni + rr;
            if (row < t.end)
              *reinterpret_cast<uint4*>(out + (int64_t)row * H + t.nt * F::TW + 32 * MI * wn + 64 * mp + 8 * c) = v4;
          }
          wave_lds_fence();
        }
    }
    zero_acc<F>(acc);
  };

  __shared__ __attribute__((aligned(16))) uint8_t lds[RingMx<F, DA, DB>::BYTES];
  persistent_tiles<F, DA, DB, Tile>(tr, I / 128, lds, setup, mfma, epilogue);
}

// Token of every permuted row: order[p] / K for routed rows, p - P for the shared rows.
__global__ void __launch_bounds__(256) row_tokens_kernel(const int32_t* __restrict__ order, int pairs, int k,
                                                         int rows, int32_t* __restrict__ row_token) {
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p < rows) row_token[p] = p < pairs ? order[p] / k : p - pairs;
}

// ---------------------------------------------------------------------------------
// gate[t] = sigmoid(x[t] . g) (1 when g is null); one wave per token.
__global__ void __launch_bounds__(64) shared_gate_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                         int tokens, int hidden, float* __restrict__ gate) {
  const int t = blockIdx.x, lane = threadIdx.x;
  if (t >= tokens) return;
  float v = 1.0f;
  if (g) {
    const uint32_t* xr = reinterpret_cast<const uint32_t*>(x) + (int64_t)t * (hidden / 2);
    const uint32_t* gr = reinterpret_cast<const uint32_t*>(g);
    float a = 0.0f;
    for (int q = lane; q < hidden / 2; q += 64) a = dot2_bf16(bits_to_bf16x2(xr[q]), bits_to_bf16x2(gr[q]), a);
    a = segment_sum<64>(a);
    v = 1.0f / (1.0f + __expf(-a));
  }
  if (lane == 0) gate[t] = v;
}

// Whether pair p's expert is resident: its slot map entry (when the table has one) is
// not negative. The GEMMs read slot 0 for a non-resident expert; its rows are dropped here.
__device__ __forceinline__ bool pair_resident(const int32_t* __restrict__ indices, const int32_t* __restrict__ slots,
                                              int p) {
  return !slots || slots[indices[p]] >= 0;
}

// combine: y[t, c] = sum_k w[t, k] rows[inverse[t*K + k], c] (+ gate[t] rows[P + t, c]), fp32
// sum in k order, bf16 out (the expert rows are unweighted). Pairs with an unknown or
// non-resident expert contribute nothing; so does a non-resident shared expert.
// per-pair (combine = 0): out[p, c] = rows[inverse[p], c], a zero row for an unknown or
// non-resident expert, and no write at all for a masked pair (negative index).
// 8 columns per thread.
__global__ void __launch_bounds__(256) combine_rows_kernel(const uint16_t* __restrict__ rows,
                                                           const int32_t* __restrict__ inverse,
                                                           const float* __restrict__ weights,
                                                           const float* __restrict__ gate, int tokens, int k,
                                                           int hidden, int has_shared, int combine,
                                                           const int32_t* __restrict__ indices,
                                                           const int32_t* __restrict__ slots,
                                                           const int32_t* __restrict__ shared_slots,
                                                           uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int c8 = blockIdx.y * blockDim.x + threadIdx.x;
  if (c8 * 8 >= hidden) return;
  const int pairs = tokens * k;
  if (!combine) {
    if (indices[t] < 0) return;
    const int row = inverse[t];
    const bool live = row >= 0 && pair_resident(indices, slots, t);
    const uint4 v = live ? reinterpret_cast<const uint4*>(rows + (int64_t)row * hidden)[c8] : make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(out + (int64_t)t * hidden)[c8] = v;
    return;
  }
  const bool shared_live = has_shared && (!shared_slots || shared_slots[0] >= 0);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](const uint4 v, float s) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] = fmaf(s, bf16_bits_to_f32(w[q] & 0xffffu), acc[2 * q]);
      acc[2 * q + 1] = fmaf(s, bf16_bits_to_f32(w[q] >> 16), acc[2 * q + 1]);
    }
  };
  // the rows of the token's pairs and its shared row are loaded before any is summed (sums
  // stay in k order, the shared row last); row indices are block-uniform (scalar addressing).
  // Each row is read once, so the loads carry the non-temporal hint (a buffer load over the
  // row, nt): 2.5% of the C3 layer against plain loads.
  const int n = k + (has_shared ? 1 : 0);
  auto load_row = [&](int r) {
    const __amdgpu_buffer_rsrc_t rr =
        __builtin_amdgcn_make_buffer_rsrc((void*)(rows + (int64_t)r * hidden), 0, hidden * 2, 0x00020000);
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rr, c8 * 16, 0, 2));
  };
  auto row_of = [&](int j) {
    int r = j < k ? inverse[t * k + j] : (j < n && shared_live ? pairs + t : -1);
    if (j < k && r >= 0 && !pair_resident(indices, slots, t * k + j)) r = -1;
    return __builtin_amdgcn_readfirstlane(r);
  };
  constexpr int ONE_PASS = 17;  // up to 16 pairs + the shared row in one unrolled pass
  if (n <= ONE_PASS) {
    int row[ONE_PASS];
    uint4 v[ONE_PASS];
#pragma unroll
    for (int j = 0; j < ONE_PASS; ++j) row[j] = j < n ? row_of(j) : -1;
#pragma unroll
    for (int j = 0; j < ONE_PASS; ++j)
      if (row[j] >= 0) v[j] = load_row(row[j]);
#pragma unroll
    for (int j = 0; j < ONE_PASS; ++j)
      if (row[j] >= 0) add(v[j], j < k ? weights[t * k + j] : gate[t]);
  }
  constexpr int BATCH = 16;
  for (int j0 = 0; n > ONE_PASS && j0 < n; j0 += BATCH) {
    int row[BATCH];
    uint4 v[BATCH];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) row[q] = j0 + q < n ? row_of(j0 + q) : -1;
#pragma unroll
    for (int q = 0; q < BATCH; ++q)
      if (row[q] >= 0) v[q] = load_row(row[q]);
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      const int j = j0 + q;
      if (row[q] >= 0) add(v[q], j < k ? weights[t * k + j] : gate[t]);
    }
  }
  uint4 o;
  o.x = pack_bf16x2(acc[0], acc[1]);
  o.y = pack_bf16x2(acc[2], acc[3]);
  o.z = pack_bf16x2(acc[4], acc[5]);
  o.w = pack_bf16x2(acc[6], acc[7]);
  reinterpret_cast<uint4*>(out + (int64_t)t * hidden)[c8] = o;
}

// ---------------------------------------------------------------------------------
// Host side.

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Optional event timing of the two grouped GEMMs (off unless wm_set_kernel_timing(1)):
// events recorded on the call's stream around gate_up and down; one set per device.
static std::atomic<int> g_timing{0};
struct TimingEvents {
  hipEvent_t ev[3] = {nullptr, nullptr, nullptr};
};
static TimingEvents* timing_events() {
  static TimingEvents per_device[64];
  static std::mutex lock;
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) fail("prefill timing: device index out of range");
  std::lock_guard<std::mutex> g(lock);
  TimingEvents& t = per_device[dev];
  for (auto& e : t.ev)
    if (!e) check_hip(hipEventCreate(&e), "hipEventCreate");
  return &t;
}

// Compute units of the current device (queried once per device).
static int compute_units() {
  static int cached[64] = {0};
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) fail("prefill: device index out of range");
  if (!cached[dev]) {
    int n = 0;
    check_hip(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute");
    cached[dev] = n > 0 ? n : 1;
  }
  return cached[dev];
}

struct Layout {
  size_t permute_ws, order, inverse, offsets, tiles, tile_count, gate, row_token, x6, x6s, a6, a6s, rows, total;
};

// Split rows take the larger of the two term formats' bytes per 128-wide K step (E4M3: 256
// term bytes plus a scale dword; E2M3: 208 bytes, scales inside), so one workspace size
// serves either.
static Layout layout(int tokens, int k, int experts, int hidden, int inter, bool has_shared) {
  const int64_t pairs = (int64_t)tokens * k;
  const int64_t rows = pairs + (has_shared ? tokens : 0);
  const int64_t max_tiles = (pairs + BM - 1) / BM + experts;
  Layout p{};
  size_t at = 0;
  p.permute_ws = at; at += align256(wm_permute_workspace_size(pairs, experts));
  p.order = at;      at += align256(sizeof(int32_t) * (size_t)(pairs > 0 ? pairs : 1));
  p.inverse = at;    at += align256(sizeof(int32_t) * (size_t)(pairs > 0 ? pairs : 1));
  p.offsets = at;    at += align256(sizeof(int32_t) * (size_t)(experts + 1));
  p.tiles = at;      at += align256(sizeof(int32_t) * 2 * (size_t)max_tiles);
  p.tile_count = at; at += align256(sizeof(int32_t));
  p.gate = at;       at += align256(sizeof(float) * (size_t)(tokens > 0 ? tokens : 1));
  p.row_token = at;  at += align256(sizeof(int32_t) * (size_t)(rows > 0 ? rows : 1));
  p.x6 = at;         at += align256((size_t)tokens * (hidden / 128) * XSTEP8);
  p.x6s = at;        at += align256((size_t)tokens * (hidden / 128) * 4);
  p.a6 = at;         at += align256((size_t)rows * (inter / 128) * XSTEP8);
  p.a6s = at;        at += align256((size_t)rows * (inter / 128) * 4);
  p.rows = at;       at += align256(sizeof(uint16_t) * (size_t)rows * hidden);
  p.total = at;
  return p;
}

template <typename F, typename Table>
static void run(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                const Table& routed, const Table* shared, const uint16_t* shared_gate, uint16_t* y, bool combine,
                void* ws, size_t ws_bytes, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  if (H % 128 || I % 128) fail("prefill: hidden and intermediate must be multiples of 128");
  const bool has_shared = combine && shared != nullptr;
  const Layout p = layout(tokens, k, routed.experts, H, I, has_shared);
  if (ws_bytes < p.total) fail("prefill: workspace too small");
  const int64_t pairs = (int64_t)tokens * k;
  const int64_t rows = pairs + (has_shared ? tokens : 0);
  if constexpr (!F::FP8) {  // the K loop reads 4 scale bytes of a row as one dword
    auto dword_rows = [](const void* p, int64_t stride) { return (uintptr_t)p % 4 == 0 && stride % 4 == 0; };
    for (const Table* t : {&routed, shared})
      if (t && (!dword_rows(t->gate_up_scales, t->gate_up_scales_stride) ||
                !dword_rows(t->down_scales, t->down_scales_stride)))
        fail("prefill: MXFP4 scale regions and strides must be 4-byte aligned");
  } else {  // 16-byte loads of weight rows; the fp32 block scales go through scalar loads
    auto rows16 = [](const void* p, int64_t stride) { return (uintptr_t)p % 16 == 0 && stride % 16 == 0; };
    auto f32 = [](const void* p, int64_t stride) { return (uintptr_t)p % 4 == 0 && stride % 4 == 0; };
    for (const Table* t : {&routed, shared})
      if (t && (!rows16(t->w13, t->w13_stride) || !rows16(t->w2, t->w2_stride) ||
                !f32(t->w13_scales, t->w13_scales_stride) || !f32(t->w2_scales, t->w2_scales_stride)))
        fail("prefill: FP8 weight regions and strides must be 16-byte aligned, scales 4-byte");
  }
  constexpr int XS = F::Terms::XS;
  if ((int64_t)rows * (I / 128) * XS >= ((int64_t)1 << 32) || (int64_t)tokens * (H / 128) * XS >= ((int64_t)1 << 32))
    fail("prefill: split operands of 4 GiB or more (split the call into smaller token batches)");
  uint8_t* base = (uint8_t*)ws;
  Lists L;
  L.order = (int32_t*)(base + p.order);
  L.offsets = (int32_t*)(base + p.offsets);
  L.tiles = (int32_t*)(base + p.tiles);
  L.tile_count = (int32_t*)(base + p.tile_count);
  L.shared_gate = (float*)(base + p.gate);
  L.pairs = (int)pairs;
  L.tokens = tokens;
  L.k = k;
  L.has_shared = has_shared ? 1 : 0;
  int32_t* inverse = (int32_t*)(base + p.inverse);
  if (wm_permute(indices, pairs, routed.experts, BM, (int32_t*)L.order, inverse, (int32_t*)L.offsets,
                 (int32_t*)L.tiles, (int32_t*)L.tile_count, base + p.permute_ws,
                 wm_permute_workspace_size(pairs, routed.experts), s) != 0)
    fail(std::string("prefill permute: ") + wm_last_error());
  // the split kernel computes the shared gate when a row's blocks fit one wave in a
  // power-of-two group; otherwise a kernel of its own does
  const bool fused_gate = has_shared && shared_gate && (H / 32) <= 64 && ((H / 32) & (H / 32 - 1)) == 0;
  if (has_shared && !fused_gate) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3(tokens), dim3(64), 0, s, x, shared_gate, tokens, H,
                       (float*)L.shared_gate);
    check_launch("shared_gate");
  }
  uint8_t* x6 = base + p.x6;
  int32_t* row_token = (int32_t*)(base + p.row_token);
  if (rows > 0) {
    hipLaunchKernelGGL(row_tokens_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, s, L.order, (int)pairs,
                       k, (int)rows, row_token);
    check_launch("row_tokens");
  }
  uint8_t* x6s = base + p.x6s;
  const int64_t split_jobs = (int64_t)tokens * (H / 32);
  if constexpr (F::Terms::E4)
    hipLaunchKernelGGL(split8_rows_kernel, dim3((unsigned)((split_jobs + 255) / 256)), dim3(256), 0, s, x, tokens, H,
                       x6, (uint32_t*)x6s, fused_gate ? shared_gate : nullptr, (float*)L.shared_gate);
  else
    hipLaunchKernelGGL(split6_rows_kernel, dim3((unsigned)((split_jobs + 255) / 256)), dim3(256), 0, s, x, tokens, H,
                       x6, fused_gate ? shared_gate : nullptr, (float*)L.shared_gate);
  check_launch("split_rows");
  const Table sh = shared ? *shared : routed;
  const int64_t max_row_tiles = (pairs + BM - 1) / BM + routed.experts + (has_shared ? (tokens + BM - 1) / BM : 0);
  // Persistent launches: one workgroup per CU (the LDS stages allow one), a multiple of the
  // 8 XCDs, and no more than the work tiles can use.
  const int cus = compute_units();
  auto grid_for = [&](int n_tiles) {
    const int64_t work = max_row_tiles * n_tiles;
    const int64_t per_xcd = std::min<int64_t>((work + XCDS - 1) / XCDS, std::max(cus / XCDS, 1));
    return dim3((unsigned)(per_xcd * XCDS));
  };
  uint8_t* a6 = base + p.a6;
  uint32_t* a6s = (uint32_t*)(base + p.a6s);
  uint16_t* out_rows = (uint16_t*)(base + p.rows);
  TimingEvents* te = g_timing.load() ? timing_events() : nullptr;
  if (te) check_hip(hipEventRecord(te->ev[0], s), "hipEventRecord");
  hipLaunchKernelGGL((gate_up_mx_kernel<F, F::DA, F::DB, Table>), grid_for((I + F::TW / 2 - 1) / (F::TW / 2)),
                     dim3(64 * F::WAVES), 0, s, x6, x6s, row_token, L, routed, sh, a6, a6s);
  check_launch("gate_up");
  if (te) check_hip(hipEventRecord(te->ev[1], s), "hipEventRecord");
  // unweighted rows: the combine applies the routing weights and the shared gate
  hipLaunchKernelGGL((down_mx_kernel<F, F::DA, F::DB, Table>), grid_for((H + F::TW - 1) / F::TW), dim3(64 * F::WAVES), 0,
                     s, a6, (const uint8_t*)a6s, L, routed, sh, out_rows);
  check_launch("down");
  if (te) check_hip(hipEventRecord(te->ev[2], s), "hipEventRecord");
  const int32_t* shared_slots = has_shared ? shared->slots : nullptr;
  if (combine)
    hipLaunchKernelGGL(combine_rows_kernel, dim3(tokens, (H / 8 + 255) / 256), dim3(256), 0, s, out_rows, inverse,
                       weights, L.shared_gate, tokens, k, H, has_shared ? 1 : 0, 1, indices, routed.slots,
                       shared_slots, y);
  else
    hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)pairs, (H / 8 + 255) / 256), dim3(256), 0, s, out_rows,
                       inverse, weights, L.shared_gate, tokens, k, H, 0, 0, indices, routed.slots, nullptr, y);
  check_launch("combine_rows");
}

}  // namespace mf

size_t prefill_workspace_size(int tokens, int k, const wm_mxfp4_experts& e, bool has_shared) {
  return mf::layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

// act_terms 0: the bf16-exact E4M3 activation terms; 1: the faster E2M3 terms.
void prefill_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                   const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                   uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  if (routed.act_terms == 1)
    mf::run<mf::Mx4>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
  else
    mf::run<mf::Mx4x>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
}

size_t prefill_fp8_workspace_size(int tokens, int k, const wm_fp8_experts& e, bool has_shared) {
  return mf::layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

void prefill_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                 const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                 uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  const bool e2m3 = routed.act_terms == 1;
  if (routed.scale_format == 1) {
    if (e2m3)
      mf::run<mf::Mx8e>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
    else
      mf::run<mf::Mx8ex>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
  } else {
    if (e2m3)
      mf::run<mf::Mx8>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
    else
      mf::run<mf::Mx8x>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
  }
}

}  // namespace wm

extern "C" {

WM_EXPORT int wm_repack_prefill_mxfp4(const wm_mxfp4_experts* src, void* gate_up, void* gate_up_scales, void* down,
                                      void* down_scales, void* stream) {
  return wm::guarded([&] {
    wm::validate_experts(src, "wm_repack_prefill_mxfp4 source", false);
    if (src->tiled) wm::fail("wm_repack_prefill_mxfp4: the source is already in the prefill tile layout");
    if (src->hidden % 128 || src->inter % 128)
      wm::fail("wm_repack_prefill_mxfp4: hidden and intermediate must be multiples of 128");
    if (!gate_up || !gate_up_scales || !down || !down_scales) wm::fail("wm_repack_prefill_mxfp4: null destination");
    auto aligned = [](const void* p, uintptr_t a) { return (uintptr_t)p % a == 0; };
    if (!aligned(gate_up, 16) || !aligned(down, 16) || !aligned(gate_up_scales, 4) || !aligned(down_scales, 4))
      wm::fail("wm_repack_prefill_mxfp4: destination weights must be 16-byte and scales 4-byte aligned");
    if (!aligned(src->gate_up_scales, 4) || !aligned(src->down_scales, 4) || src->gate_up_scales_stride % 4 ||
        src->down_scales_stride % 4)
      wm::fail("wm_repack_prefill_mxfp4: source scale regions and strides must be 4-byte aligned");
    const int E = src->experts, H = src->hidden, I = src->inter;
    hipStream_t s = wm::as_stream(stream);
    auto launch = [&](const void* w, const void* ws, int64_t stride, int64_t stride_s, int rows, int k, void* dst,
                      void* dst_s) {
      const int64_t words = (int64_t)rows * (k / 128);
      const int64_t n = (int64_t)E * ((int64_t)rows * (k / 32) + words);
      hipLaunchKernelGGL(wm::mf::repack_prefill_kernel<4>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                         (const uint8_t*)w, (const uint8_t*)ws, stride, stride_s, src->slots, E, rows, k, words,
                         (uint8_t*)dst, (uint8_t*)dst_s);
      wm::check_launch("repack_prefill");
    };
    launch(src->gate_up, src->gate_up_scales, src->gate_up_stride, src->gate_up_scales_stride, 2 * I, H, gate_up,
           gate_up_scales);
    launch(src->down, src->down_scales, src->down_stride, src->down_scales_stride, H, I, down, down_scales);
  });
}

WM_EXPORT int wm_repack_prefill_fp8(const wm_fp8_experts* src, void* w13, void* w13_scales, void* w2,
                                    void* w2_scales, void* stream) {
  return wm::guarded([&] {
    if (!src) wm::fail("wm_repack_prefill_fp8: source table is null");
    if (!src->w13 || !src->w2 || !src->w13_scales || !src->w2_scales)
      wm::fail("wm_repack_prefill_fp8: source region pointer is null");
    if (src->tiled) wm::fail("wm_repack_prefill_fp8: the source is already in the prefill tile layout");
    if (src->experts < 1 || src->experts > 1024) wm::fail("wm_repack_prefill_fp8: expert count must be in 1..1024");
    if (src->hidden < 128 || src->hidden % 128 || src->inter < 128 || src->inter % 128)
      wm::fail("wm_repack_prefill_fp8: hidden and intermediate must be positive multiples of 128");
    if (src->scale_format != 0 && src->scale_format != 1) wm::fail("wm_repack_prefill_fp8: unknown scale format");
    if (!w13 || !w2 || !w13_scales || !w2_scales) wm::fail("wm_repack_prefill_fp8: null destination");
    auto aligned = [](const void* p, uintptr_t a) { return (uintptr_t)p % a == 0; };
    if (!aligned(w13, 16) || !aligned(w2, 16) || !aligned(src->w13, 16) || !aligned(src->w2, 16) ||
        src->w13_stride % 16 || src->w2_stride % 16 || src->w13_stride < 0 || src->w2_stride < 0)
      wm::fail("wm_repack_prefill_fp8: weight regions and strides must be 16-byte aligned");
    if (!aligned(w13_scales, 4) || !aligned(w2_scales, 4) || !aligned(src->w13_scales, 4) ||
        !aligned(src->w2_scales, 4) || src->w13_scales_stride % 4 || src->w2_scales_stride % 4 ||
        src->w13_scales_stride < 0 || src->w2_scales_stride < 0)
      wm::fail("wm_repack_prefill_fp8: scale regions and strides must be 4-byte aligned");
    const int E = src->experts, H = src->hidden, I = src->inter;
    hipStream_t s = wm::as_stream(stream);
    auto launch = [&](const void* w, const void* ws, int64_t stride, int64_t stride_s, int rows, int k, void* dst,
                      void* dst_s) {
      // scale words per expert: fp32 [rows/128][k/128], or E8M0 bytes [rows/32][k/32] as dwords
      const int64_t words = src->scale_format == 1 ? (int64_t)(rows / 32) * (k / 128) : (int64_t)(rows / 128) * (k / 128);
      const int64_t n = (int64_t)E * ((int64_t)rows * (k / 16) + words);
      hipLaunchKernelGGL(wm::mf::repack_prefill_kernel<8>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                         (const uint8_t*)w, (const uint8_t*)ws, stride, stride_s, src->slots, E, rows, k, words,
                         (uint8_t*)dst, (uint8_t*)dst_s);
      wm::check_launch("repack_prefill_fp8");
    };
    launch(src->w13, src->w13_scales, src->w13_stride, src->w13_scales_stride, 2 * I, H, w13, w13_scales);
    launch(src->w2, src->w2_scales, src->w2_stride, src->w2_scales_stride, H, I, w2, w2_scales);
  });
}

WM_EXPORT int wm_split_rows_e2m3(const void* x, int32_t rows, int32_t hidden, void* out, void* stream) {
  return wm::guarded([&] {
    if (rows < 0 || hidden < 128 || hidden % 128) wm::fail("wm_split_rows_e2m3: hidden must be a positive multiple of 128");
    if (rows == 0) return;
    if (!x || !out) wm::fail("wm_split_rows_e2m3: null pointer");
    if ((uintptr_t)x % 16 || (uintptr_t)out % 16) wm::fail("wm_split_rows_e2m3: x and out must be 16-byte aligned");
    const int64_t jobs = (int64_t)rows * (hidden / 32);
    hipLaunchKernelGGL(wm::mf::split6_rows_kernel, dim3((unsigned)((jobs + 255) / 256)), dim3(256), 0,
                       wm::as_stream(stream), (const uint16_t*)x, (int)rows, (int)hidden, (uint8_t*)out, nullptr,
                       nullptr);
    wm::check_launch("split_rows_e2m3");
  });
}

WM_EXPORT int wm_split_rows_e4m3(const void* x, int32_t rows, int32_t hidden, void* terms, void* scales, void* stream) {
  return wm::guarded([&] {
    if (rows < 0 || hidden < 128 || hidden % 128) wm::fail("wm_split_rows_e4m3: hidden must be a positive multiple of 128");
    if (rows == 0) return;
    if (!x || !terms || !scales) wm::fail("wm_split_rows_e4m3: null pointer");
    if ((uintptr_t)x % 16 || (uintptr_t)terms % 16 || (uintptr_t)scales % 4)
      wm::fail("wm_split_rows_e4m3: x and terms must be 16-byte aligned, scales 4-byte");
    const int64_t jobs = (int64_t)rows * (hidden / 32);
    hipLaunchKernelGGL(wm::mf::split8_rows_kernel, dim3((unsigned)((jobs + 255) / 256)), dim3(256), 0,
                       wm::as_stream(stream), (const uint16_t*)x, (int)rows, (int)hidden, (uint8_t*)terms,
                       (uint32_t*)scales, nullptr, nullptr);
    wm::check_launch("split_rows_e4m3");
  });
}

WM_EXPORT int wm_set_kernel_timing(int enable) {
  wm::mf::g_timing.store(enable ? 1 : 0);
  return 0;
}

WM_EXPORT int wm_kernel_timing_ms(float* out2) {
  return wm::guarded([&] {
    if (!out2) wm::fail("wm_kernel_timing_ms: null output");
    wm::mf::TimingEvents* te = wm::mf::timing_events();
    wm::check_hip(hipEventSynchronize(te->ev[2]), "hipEventSynchronize");
    wm::check_hip(hipEventElapsedTime(&out2[0], te->ev[0], te->ev[1]), "hipEventElapsedTime");
    wm::check_hip(hipEventElapsedTime(&out2[1], te->ev[1], te->ev[2]), "hipEventElapsedTime");
  });
}

}  // extern "C"
