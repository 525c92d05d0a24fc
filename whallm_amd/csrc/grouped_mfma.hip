// Prefill-time expert FFN on gfx950 scaled MFMA (v_mfma_scale_f32_16x16x128_f8f6f4):
// grouped GEMMs over the row tiles of the permute kernel, for MXFP4 weights (E2M1 codes
// with an E8M0 scale per 32, fed to the MFMA as stored) and for FP8-E4M3 weights with
// fp32 128 x 128 block scales.
//
// Replaces gather_rows16 + expert_gemm_sg (gate_up) + expert_act + expert_gemm_sg (down) +
// moe_combine_rows (Native/QwenNative/kernels.metal:691-765, engine.mm:2104-2162) and
// mx.gather_qmm (qwen4_exp.py:857-897, model.py:435-501):
//
//   split   : every token row of x (bf16) becomes two E4M3 terms, hi and lo, each with
//             an E8M0 scale per 32 values: x = hi * 2^(s-127) + lo * 2^(s-131), which keeps
//             the 8 significant bits of a bf16 for values within 2^8 of their block's
//             maximum. The bytes are stored in MFMA B-operand order (below), so the GEMMs
//             copy them to LDS unchanged.
//   gate_up : tile = 128 permuted rows x (64 gate + the 64 matching up weight rows); per
//             128-wide K step each wave runs 4 x 4 (weight tile x row tile) MFMA pairs
//             (hi term, lo term). SwiGLU is the epilogue, which writes act straight back
//             as E4M3 hi/lo terms with per-32 scales (the down GEMM's B operand).
//   down    : tile = 128 permuted rows x 128 output columns over K = intermediate; the
//             row's routing weight (or the shared expert's sigmoid gate) is applied in the
//             epilogue; bf16 rows in permuted order.
//   combine : y[t] = sum of the token's K rows in k order, plus the shared row.
//
// MFMA operand layout (16 x 16 x 128; lane l, c = l % 16, g = l / 16):
//   fp4 operand: lane holds row c's K values [32g, 32g+32) as nibbles (low first), 16 bytes;
//   fp8 operand: lane holds row c's K values [16g, 16g+16) in bytes 0-15 and
//                [64+16g, 64+16g+16) in bytes 16-31;
//   scale     : lane (c, g) gives the E8M0 scale of row c, K block [32g, 32g+32);
//   result    : lane holds D[4g + r][c], r = 0..3 (A rows = weight rows, B columns = rows).
// "B-operand order" of a 128-value chunk is therefore position 32g + 16h + e for K value
// 64h + 16g + e, so lane group g reads its 32 bytes contiguously.
//
// Precision: per element the two terms carry 8 significant bits (bf16 has 8); the MFMA's
// own summation keeps about 2^-13 of the sum of |products|.
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
constexpr int CHUNK = 256;  // bytes per (row, 128-wide K step) of a split operand: hi | lo
constexpr int XSTR = 272;   // LDS bytes per row of the split operand: 256 + 16 pad
constexpr int FMT_FP8 = 0;
constexpr int FMT_FP4 = 4;

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

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

// Row range and expert of logical row tile m; expert -1 is the shared expert.
__device__ __forceinline__ bool resolve_tile(const Lists& L, int m, int& expert, int& begin, int& end) {
  const int routed_tiles = L.tile_count[0];
  if (m < routed_tiles) {
    expert = L.tiles[2 * m];
    begin = L.tiles[2 * m + 1];
    end = min(begin + BM, L.offsets[expert + 1]);
    return true;
  }
  const int j = m - routed_tiles;
  if (!L.has_shared || j * BM >= L.tokens) return false;
  expert = -1;
  begin = L.pairs + j * BM;
  end = min(begin + BM, L.pairs + L.tokens);
  return true;
}

__device__ __forceinline__ int active_row_tiles(const Lists& L) {
  return L.tile_count[0] + (L.has_shared ? (L.tokens + BM - 1) / BM : 0);
}

// XCD-major work mapping (block b runs on XCD b % 8): each XCD takes a contiguous range
// of the (row tile, column tile) list. False for workgroups past the active work.
__device__ __forceinline__ bool map_work(int active, int& logical) {
  const int l = blockIdx.x;
  const int xcd = l % XCDS, local = l / XCDS;
  const int share = (active + XCDS - 1) / XCDS;
  if (local >= share) return false;
  logical = xcd * share + local;
  return logical < active;
}

// ---------------------------------------------------------------------------------
// split: one wave per 128-wide chunk of a row; lane l holds values 2l, 2l+1.

__device__ __forceinline__ int term_exponent(float amax) {
  const int be = (int)((__float_as_uint(amax) >> 23) & 0xff);
  return be - 7 > 1 ? be - 7 : 1;  // maps the block maximum into [2^7, 2^8): E4M3 max is 448
}
__device__ __forceinline__ float pow2_biased(int e) { return __uint_as_float((uint32_t)e << 23); }
__device__ __forceinline__ float e4m3_byte0(uint32_t w) { return __builtin_amdgcn_cvt_f32_fp8((int)w, 0); }
__device__ __forceinline__ float e4m3_byte1(uint32_t w) { return __builtin_amdgcn_cvt_f32_fp8((int)w, 1); }

// Maximum over the 16 lanes of each row of the wave (DPP within rows of 16).
__device__ __forceinline__ float max16(float v) {
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false)));
  v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false)));
  return v;
}

// x [rows, H] bf16 -> x8 [rows][H/128][hi 128 | lo 128] (B-operand order), xs [rows][H/128][hi 4 | lo 4].
__global__ void __launch_bounds__(256) split_rows_kernel(const uint16_t* __restrict__ x, int rows, int hidden,
                                                         uint8_t* __restrict__ x8, uint8_t* __restrict__ xs) {
  const int chunks = hidden / 128;
  const int64_t job = (int64_t)blockIdx.x * 4 + threadIdx.x / 64;  // (row, chunk)
  if (job >= (int64_t)rows * chunks) return;
  const int lane = threadIdx.x % 64;
  const int64_t row = job / chunks;
  const int c = (int)(job % chunks);
  const uint32_t pair = reinterpret_cast<const uint32_t*>(x + row * hidden + c * 128)[lane];
  const float v0 = bf16_bits_to_f32(pair & 0xffffu), v1 = bf16_bits_to_f32(pair >> 16);
  const float amax = max16(fmaxf(fabsf(v0), fabsf(v1)));  // lanes 16b..16b+15 hold block b
  const int s = term_exponent(amax);
  const float f = pow2_biased(254 - s);
  const float h0 = v0 * f, h1 = v1 * f;
  const uint32_t hw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(h0, h1, 0, false);
  const float l0 = (h0 - e4m3_byte0(hw)) * 16.0f, l1 = (h1 - e4m3_byte1(hw)) * 16.0f;
  const uint32_t lw = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(l0, l1, 0, false);
  const int kk = 2 * lane;  // K value within the chunk
  const int pos = 32 * ((kk >> 4) & 3) + 16 * (kk >> 6) + (kk & 15);
  uint8_t* dst = x8 + (row * chunks + c) * CHUNK;
  *reinterpret_cast<uint16_t*>(dst + pos) = (uint16_t)hw;
  *reinterpret_cast<uint16_t*>(dst + 128 + pos) = (uint16_t)lw;
  if ((lane & 15) == 0) {
    uint8_t* sd = xs + (row * chunks + c) * 8;
    sd[lane >> 4] = (uint8_t)s;
    sd[4 + (lane >> 4)] = (uint8_t)(s > 4 ? s - 4 : 0);
  }
}

// ---------------------------------------------------------------------------------
// Tiles and formats.
//
// A workgroup computes a 128-row x TW-weight-row tile with WAVES waves: wave (wm, wn) =
// (w & 1, w >> 1) owns rows 64 wm + [0, 64) and weight rows wrow(wn, mi) + [0, 16) for
// mi = 0..7, i.e. 8 x 4 MFMA tiles per term (each B fragment of the split rows, 64 bytes
// per lane, feeds 8 weight tiles). MXFP4: 8 waves (two per SIMD, which overlap one wave's
// LDS reads with the other's MFMAs), TW = 512. FP8: 4 waves, TW = 256 (its weight rows
// are twice as large). Each K step's operands go straight from global memory into LDS
// (global_load_lds: lane i of a wave writes LDS base + size * i) in a ring of 2 stages;
// the loads of step k + 1 are issued when step k starts.
//
// LDS placement (16-byte pieces, swizzled so the 16 rows served by one ds_read_b128 cycle
// fall on distinct banks): split row r piece p at r * 256 + 16 (p ^ (r & 15)); weight row j
// piece p at j * STEP_BYTES + 16 (p ^ swz(j)).

constexpr int MI = 8;        // weight tiles per wave
constexpr int NI = 4;        // row tiles per wave

struct Fp4Weights {
  static constexpr int FMT = FMT_FP4;
  static constexpr int STEP_BYTES = 64;   // bytes of one weight row per 128-wide K step
  static constexpr int PIECES = 4;
  static constexpr int WAVES = 8;
  static constexpr int TW = 512;          // weight rows per tile
  static constexpr int SCALE_BYTES = TW * 4;  // E8M0 scales of the step: 4 per weight row
  __device__ static int swz(int row) { return (row >> 2) & 3; }
};
struct Fp8Weights {
  static constexpr int FMT = FMT_FP8;
  static constexpr int STEP_BYTES = 128;
  static constexpr int PIECES = 8;
  static constexpr int WAVES = 4;
  static constexpr int TW = 256;
  static constexpr int SCALE_BYTES = 16;      // unused: block scales are read from global memory
  __device__ static int swz(int row) { return (row >> 1) & 7; }
};

template <typename W>
struct Stage {
  __attribute__((aligned(16))) uint8_t b[BM * CHUNK];              // split rows: hi 128 | lo 128
  __attribute__((aligned(16))) uint8_t bs[BM * 8];                 // their scales: hi 4 | lo 4
  __attribute__((aligned(16))) uint8_t a[W::TW * W::STEP_BYTES];   // weight rows
  __attribute__((aligned(16))) uint8_t as[W::SCALE_BYTES];         // MXFP4: 4 E8M0 bytes per row
};

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
__device__ __forceinline__ int uniform_i(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float uniform_f(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ const uint8_t* uniform_u8(const uint8_t* p) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<const uint8_t*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// Per-lane LDS read offsets of a wave's operands within a stage. Weight tile mi of wave
// (wm, wn) is rows wave_row0 + mrow(mi) + c, where mrow is a compile-time constant; its
// swizzle depends on the lane only (rows are 16-aligned). Row tile ni is rows
// 64 wm + 16 ni + c, whose swizzle r & 15 = c & 15 is also per lane. So every read is a
// per-lane base plus an immediate offset.
struct LaneOffsets {
  uint32_t a, a2;        // weight piece g (and, FP8, piece g + 4) of row wave_row0 + c
  uint32_t as;           // its MXFP4 scale byte: (wave_row0 + c) * 4 + g
  uint32_t b[4];         // split-row pieces 2g, 2g+1, 8+2g, 9+2g of row 64 wm + c
  uint32_t bs;           // its scale byte: (64 wm + c) * 8 + g
};

template <typename W>
__device__ __forceinline__ LaneOffsets lane_offsets(int wave_row0, int wm) {
  const int lane = threadIdx.x % 64, c = lane % 16, g = lane / 16;
  LaneOffsets o;
  const int arow = wave_row0 + c, z = W::swz(arow);
  o.a = arow * W::STEP_BYTES + 16 * (g ^ z);
  o.a2 = arow * W::STEP_BYTES + 16 * ((g + 4) ^ z);
  o.as = arow * 4 + g;
  const int brow = 64 * wm + c, zb = brow & 15;
  o.b[0] = brow * CHUNK + 16 * ((2 * g) ^ zb);
  o.b[1] = brow * CHUNK + 16 * ((2 * g + 1) ^ zb);
  o.b[2] = brow * CHUNK + 16 * ((8 + 2 * g) ^ zb);
  o.b[3] = brow * CHUNK + 16 * ((9 + 2 * g) ^ zb);
  o.bs = brow * 8 + g;
  return o;
}

// One 128-wide K step of the wave's 64 x 128 sub-tile from LDS (rows 64 wm + 16 ni + c,
// weight rows wave_row0 + MROW(mi) + c). The 8 A fragments are read first; then each row
// tile's B fragment feeds the 8 weight tiles (16 MFMAs). For FP8 weights each (mi, ni)
// accumulates the step on its own and adds it times the block scale bscale(mi).
template <typename W, typename MRow, typename BScale>
__device__ __forceinline__ void step_mfma(const Stage<W>& st, const LaneOffsets& lo, v4f (&acc)[MI][NI], MRow mrow,
                                          BScale bscale) {
  v8i a[MI];
  int sa[MI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi) {
    const int dr = mrow(mi);  // compile-time after unrolling
    if constexpr (W::FMT == FMT_FP4) {
      const uint4 v = *reinterpret_cast<const uint4*>(st.a + lo.a + dr * W::STEP_BYTES);
      a[mi] = v8i{(int)v.x, (int)v.y, (int)v.z, (int)v.w, 0, 0, 0, 0};
      sa[mi] = st.as[lo.as + dr * 4];
    } else {
      const uint4 v0 = *reinterpret_cast<const uint4*>(st.a + lo.a + dr * W::STEP_BYTES);
      const uint4 v1 = *reinterpret_cast<const uint4*>(st.a + lo.a2 + dr * W::STEP_BYTES);
      a[mi] = v8i{(int)v0.x, (int)v0.y, (int)v0.z, (int)v0.w, (int)v1.x, (int)v1.y, (int)v1.z, (int)v1.w};
      sa[mi] = 127;
    }
  }
#pragma unroll
  for (int ni = 0; ni < NI; ++ni) {
    const int db = 16 * ni * CHUNK;
    const uint4 h0 = *reinterpret_cast<const uint4*>(st.b + lo.b[0] + db);
    const uint4 h1 = *reinterpret_cast<const uint4*>(st.b + lo.b[1] + db);
    const uint4 l0 = *reinterpret_cast<const uint4*>(st.b + lo.b[2] + db);
    const uint4 l1 = *reinterpret_cast<const uint4*>(st.b + lo.b[3] + db);
    const v8i bh = {(int)h0.x, (int)h0.y, (int)h0.z, (int)h0.w, (int)h1.x, (int)h1.y, (int)h1.z, (int)h1.w};
    const v8i bl = {(int)l0.x, (int)l0.y, (int)l0.z, (int)l0.w, (int)l1.x, (int)l1.y, (int)l1.z, (int)l1.w};
    const int sbh = st.bs[lo.bs + 16 * ni * 8], sbl = st.bs[lo.bs + 16 * ni * 8 + 4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi) {
      if constexpr (W::FMT == FMT_FP4) {
        acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], bh, acc[mi][ni], FMT_FP4, FMT_FP8, 0,
                                                                       sa[mi], 0, sbh);
        acc[mi][ni] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], bl, acc[mi][ni], FMT_FP4, FMT_FP8, 0,
                                                                       sa[mi], 0, sbl);
      } else {
        v4f blk = {0.0f, 0.0f, 0.0f, 0.0f};
        blk = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], bh, blk, FMT_FP8, FMT_FP8, 0, 127, 0, sbh);
        blk = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a[mi], bl, blk, FMT_FP8, FMT_FP8, 0, 127, 0, sbl);
        const float s = bscale(mi);
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[mi][ni][r] = fmaf(s, blk[r], acc[mi][ni][r]);
      }
    }
    // one row tile's fragment live at a time (the scheduler would otherwise hoist all four
    // reads and run out of registers)
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Per-lane sources of the direct-to-LDS loads of one K step. Split rows: 32 x 1 KB
// (4 rows each; slot q of wave w is slot w + WAVES q: rows 4 slot + lane / 16, piece
// (lane % 16) ^ (row & 15)); their scales: 4 x 256 B (slot s = rows 32 s + lane / 2, hi or
// lo word lane % 2), issued by waves 0-3. Weight rows: TW * STEP_BYTES / 1024 x 1 KB
// (slot q of wave w is slot w + WAVES q: rows slot * (1024 / STEP_BYTES) + lane / PIECES).
// MXFP4 scales: TW / 64 x 256 B (slot w + WAVES q: weight rows 64 slot + lane). Only 4-
// and 16-byte loads (their lane layout is the documented base + size * lane). Offsets
// are taken at K step 0; step ks adds ks * CHUNK, ks * 8, ks * STEP_BYTES and ks * 4.
template <typename W>
struct Loader {
  static constexpr int BQ = 32 / W::WAVES;                                   // split-row loads per wave
  static constexpr int AQ = W::TW * W::STEP_BYTES / 1024 / W::WAVES;         // weight loads per wave
  static constexpr int SQ = W::FMT == FMT_FP4 ? W::TW / 64 / W::WAVES : 0;   // MXFP4 scale loads per wave
  const uint8_t* b;              // split operand [rows][chunks][CHUNK]
  const uint8_t* bsc;            // its scales [rows][chunks][8]
  const uint8_t* wbase;          // the tile's weight region (wave-uniform)
  const uint8_t* sbase;          // its MXFP4 scale region (wave-uniform)
  uint32_t boff[BQ];
  uint32_t bsoff;
  uint32_t aoff[AQ];             // byte offsets from wbase
  uint32_t soff[SQ > 0 ? SQ : 1];

  // row_b(r): split-operand row of tile row r; row_w(j): byte offset from wbase of tile
  // weight row j; row_s(j): byte offset from sbase of its MXFP4 scale row.
  template <typename RowB, typename RowW, typename RowS>
  __device__ __forceinline__ void init(const uint8_t* b_, const uint8_t* bsc_, int chunks, const uint8_t* wbase_,
                                       const uint8_t* sbase_, RowB row_b, RowW row_w, RowS row_s) {
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64;
    b = uniform_u8(b_);
    bsc = uniform_u8(bsc_);
    wbase = uniform_u8(wbase_);
    sbase = uniform_u8(sbase_);
#pragma unroll
    for (int q = 0; q < BQ; ++q) {
      const int r = 4 * (w + W::WAVES * q) + lane / 16;
      boff[q] = (uint32_t)row_b(r) * (uint32_t)(chunks * CHUNK) + 16u * (uint32_t)((lane % 16) ^ (r & 15));
    }
    bsoff = (uint32_t)row_b((32 * w + lane / 2) & (BM - 1)) * (uint32_t)(chunks * 8) + 4u * (uint32_t)(lane % 2);
    constexpr int RPI = 1024 / W::STEP_BYTES;  // weight rows per 1 KB load
#pragma unroll
    for (int q = 0; q < AQ; ++q) {
      const int j = (w + W::WAVES * q) * RPI + lane / W::PIECES;
      aoff[q] = row_w(j) + 16u * (uint32_t)((lane % W::PIECES) ^ W::swz(j));
    }
#pragma unroll
    for (int q = 0; q < SQ; ++q) soff[q] = row_s(64 * (w + W::WAVES * q) + lane);
  }

  __device__ __forceinline__ void issue(Stage<W>& st, int ks) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
#pragma unroll
    for (int q = 0; q < BQ; ++q) dma16(b, boff[q] + (uint32_t)ks * CHUNK, lds_addr(st.b + (w + W::WAVES * q) * 1024));
#pragma unroll
    for (int q = 0; q < AQ; ++q)
      dma16(wbase, aoff[q] + (uint32_t)(ks * W::STEP_BYTES), lds_addr(st.a + (w + W::WAVES * q) * 1024));
    if (w < 4) dma4(bsc, bsoff + (uint32_t)ks * 8, lds_addr(st.bs + 256 * w));
#pragma unroll
    for (int q = 0; q < SQ; ++q) dma4(sbase, soff[q] + (uint32_t)ks * 4, lds_addr(st.as + 256 * (w + W::WAVES * q)));
  }
};

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

// Persistent K loop over this workgroup's tiles, as one flat sequence of 128-wide steps
// through two LDS stages (global step g uses stage g % 2; the loop is unrolled over the
// two stages so their addresses are static). At the top of each step every wave has the
// step's loads landed and is done with the other stage, which then takes the next step's
// loads: the tile's next K step, or at a tile's last step the next tile's first step. The
// next tile is set up (index loads, load offsets) after the MFMAs of the tile's
// second-to-last step, and its first loads fly during this tile's epilogue.
//   setup(j, tile) -> bool: fills tile j's state; false for a tile with no rows
//   mfma(tile, stage, k): step k of a tile
//   epilogue(tile): after a tile's last step
template <typename W, typename Tile, typename Setup, typename Mfma, typename Epilogue>
__device__ __forceinline__ void persistent_tiles(const TileRange& tr, int steps, Stage<W>& s0, Stage<W>& s1,
                                                 Setup setup, Mfma mfma, Epilogue epilogue) {
  if (tr.count == 0) return;
  Tile cur, nxt;
  bool cur_ok = setup(0, cur), nxt_ok = false;
  if (cur_ok) cur.ld.issue(s0, 0);
  const int total = tr.count * steps;
  auto body = [&](int g, Stage<W>& stage, Stage<W>& other) {
    if (g >= total) return;
    const int j = g / steps, k = g - j * steps;
    ring_wait_all();
    if (k + 1 < steps) {
      if (cur_ok) cur.ld.issue(other, k + 1);
    } else if (j + 1 < tr.count && steps > 1 && nxt_ok) {
      nxt.ld.issue(other, 0);
    }
    if (cur_ok) mfma(cur, stage, k);
    if (k == steps - 2 && j + 1 < tr.count) nxt_ok = setup(j + 1, nxt);
    if (k == steps - 1) {
      if (cur_ok) epilogue(cur);
      if (steps == 1 && j + 1 < tr.count) {
        nxt_ok = setup(j + 1, nxt);
        if (nxt_ok) nxt.ld.issue(other, 0);
      }
      cur = nxt;
      cur_ok = nxt_ok;
      nxt_ok = false;
    }
  };
  for (int g = 0; g < total; g += 2) {
    body(g, s0, s1);
    body(g + 1, s1, s0);
  }
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

__device__ __forceinline__ TileWeights tile_weights(const wm_mxfp4_experts& routed, const wm_mxfp4_experts& shared,
                                                    int expert) {
  const wm_mxfp4_experts& t = expert < 0 ? shared : routed;
  const ExpertRegions r = expert_regions(t, expert < 0 ? 0 : expert);
  return {r.gate_up, r.gate_up_scales, r.down, r.down_scales, t.up_first, t.swiglu_limit};
}
__device__ __forceinline__ TileWeights tile_weights(const wm_fp8_experts& routed, const wm_fp8_experts& shared,
                                                    int expert) {
  const wm_fp8_experts& t = expert < 0 ? shared : routed;
  const Fp8Regions r = fp8_regions(t, expert < 0 ? 0 : expert);
  return {r.w13, reinterpret_cast<const uint8_t*>(r.w13_scales), r.w2, reinterpret_cast<const uint8_t*>(r.w2_scales),
          t.up_first, t.swiglu_limit};
}

// E4M3 hi/lo terms of 4 act values (already times 2^(127 - s)) into bytes 0..3 of hi, lo.
__device__ __forceinline__ void act_terms(float v0, float v1, float v2, float v3, uint32_t& hi, uint32_t& lo) {
  const uint32_t w01 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  const uint32_t w23 = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, 0, false);
  const float l0 = (v0 - e4m3_byte0(w01)) * 16.0f, l1 = (v1 - e4m3_byte1(w01)) * 16.0f;
  const float l2 = (v2 - e4m3_byte0(w23)) * 16.0f, l3 = (v3 - e4m3_byte1(w23)) * 16.0f;
  hi = (w01 & 0xffffu) | (w23 << 16);
  lo = ((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(l0, l1, 0, false) & 0xffffu) |
       ((uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(l2, l3, 0, false) << 16);
}

// ---------------------------------------------------------------------------------
// gate_up: act rows of a tile's TW / 2 intermediate columns. Weight tile rows [0, TW/2)
// are the gate rows nt * TW/2 + j, [TW/2, TW) the matching up rows; wave wn owns gate rows
// 64 wn + [0, 64) (mi 0..3) and the same up rows (mi 4..7). When I is not a multiple of
// TW / 2, the last tile's columns past I are computed on repeated rows and not written.

template <typename W>
struct GateUpTile {
  Loader<W> ld;
  int begin, end, nt, valid;
  float limit;
  const_f32_ptr sg, su;   // FP8 block scales of the wave's gate and up rows (per K step)
};

template <typename W, typename Table>
__global__ void __launch_bounds__(64 * W::WAVES) gate_up_kernel(const uint8_t* __restrict__ x8,
                                                                const uint8_t* __restrict__ xs, Lists L,
                                                                Table routed, Table shared, uint8_t* __restrict__ a8,
                                                                uint8_t* __restrict__ as8) {
  constexpr int TG = W::TW / 2;  // gate (and up) rows per tile
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = (I + TG - 1) / TG;
  const TileRange tr = tile_range(active_row_tiles(L) * n_tiles);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave & 1, wn = wave >> 1;
  const LaneOffsets lo = lane_offsets<W>(64 * wn, wm);
  const int64_t wrow_bytes = (int64_t)H * W::STEP_BYTES / 128;
  using Tile = GateUpTile<W>;

  auto setup = [&](int j, Tile& t) {
    const int logical = tr.first + tr.stride * j;
    const int mt = logical / n_tiles;
    t.nt = logical - mt * n_tiles;
    int expert, begin_, end_;
    if (!resolve_tile(L, mt, expert, begin_, end_)) return false;
    t.begin = uniform_i(begin_);
    t.end = uniform_i(end_);
    const TileWeights tw = tile_weights(routed, shared, uniform_i(expert));
    t.limit = uniform_f(tw.limit);
    t.valid = min(TG, I - t.nt * TG);  // a multiple of 128
    const int gate0 = (tw.up_first ? I : 0) + t.nt * TG;
    const int up0 = (tw.up_first ? 0 : I) + t.nt * TG;
    const int valid = t.valid;
    auto weight_row = [gate0, up0, valid](int r) {
      const int rr = r % TG;
      return (r < TG ? gate0 : up0) + (rr < valid ? rr : rr % valid);
    };
    const int begin = t.begin, end = t.end;
    auto token_of = [&](int pr) { return pr < L.pairs ? L.order[pr] / L.k : pr - L.pairs; };
    t.ld.init(
        x8, xs, H / 128, tw.w13, tw.w13s,
        // pad rows repeat the tile's first row; their results are never written
        [&](int r) { return token_of(begin + r < end ? begin + r : begin); },
        [&](int r) { return (uint32_t)(weight_row(r) * wrow_bytes); },
        [&](int r) { return (uint32_t)(weight_row(r) * (H / 32)); });
    // FP8: the wave's 64 gate (up) rows lie in one 128-row scale block
    t.sg = uniform_ptr(reinterpret_cast<const float*>(tw.w13s) + (int64_t)(weight_row(64 * wn) / 128) * (H / 128));
    t.su = uniform_ptr(reinterpret_cast<const float*>(tw.w13s) + (int64_t)(weight_row(TG + 64 * wn) / 128) * (H / 128));
    return true;
  };

  v4f acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  auto mfma = [&](const Tile& t, const Stage<W>& st, int k) {
    step_mfma<W>(st, lo, acc, [](int mi) { return (mi < 4 ? 0 : TG) + 16 * (mi & 3); },
                 [&](int mi) { return W::FMT == FMT_FP8 ? (mi < 4 ? t.sg[k] : t.su[k]) : 1.0f; });
  };

  // Epilogue: lane holds act columns col0 + 16 mi + 4 g + r (mi 0..3) of row
  // 64 wm + 16 ni + c, col0 = nt * TG + 64 wn: 128-wide act chunk col0 / 128, K offset
  // kin0 = col0 % 128 (0 or 64). E8M0 block (kin0 + 32 half) / 32 holds mi 2 half, 2 half + 1.
  auto epilogue = [&](const Tile& t) {
    if (64 * wn < t.valid) {
      const int c = lane % 16, g = lane / 16;
      const int chunks = I / 128;
      const int col0 = t.nt * TG + 64 * wn;
      const int chunk = col0 / 128, kin0 = col0 % 128;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int row = t.begin + 64 * wm + 16 * ni + c;
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          float h[2][4];
          float amax = 0.0f;
#pragma unroll
          for (int m = 0; m < 2; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int mi = 2 * half + m;
              float gv = acc[mi][ni][r], uv = acc[mi + 4][ni][r];
              if (t.limit > 0.0f) {
                gv = fminf(gv, t.limit);
                uv = fminf(fmaxf(uv, -t.limit), t.limit);
              }
              h[m][r] = silu(gv) * uv;
              amax = fmaxf(amax, fabsf(h[m][r]));
            }
          amax = fmaxf(amax, __shfl_xor(amax, 16, 64));
          amax = fmaxf(amax, __shfl_xor(amax, 32, 64));
          if (row >= t.end) continue;
          const int s = term_exponent(amax);
          const float f = pow2_biased(254 - s);
          uint8_t* dst = a8 + ((int64_t)row * chunks + chunk) * CHUNK;
#pragma unroll
          for (int m = 0; m < 2; ++m) {
            uint32_t hi, lo_;
            act_terms(h[m][0] * f, h[m][1] * f, h[m][2] * f, h[m][3] * f, hi, lo_);
            // K = kin0 + 32 half + 16 m + 4 g + r -> B-operand position 32 (K/16 % 4) + 16 (K/64) + K % 16
            const int K = kin0 + 32 * half + 16 * m + 4 * g;
            const int pos = 32 * ((K >> 4) & 3) + 16 * (K >> 6) + (K & 15);
            *reinterpret_cast<uint32_t*>(dst + pos) = hi;
            *reinterpret_cast<uint32_t*>(dst + 128 + pos) = lo_;
          }
          if (g == 0) {
            const int blk = (kin0 >> 5) + half;
            uint8_t* sd = as8 + ((int64_t)row * chunks + chunk) * 8;
            sd[blk] = (uint8_t)s;
            sd[4 + blk] = (uint8_t)(s > 4 ? s - 4 : 0);
          }
        }
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  };

  __shared__ Stage<W> s0, s1;
  persistent_tiles<W, Tile>(tr, H / 128, s0, s1, setup, mfma, epilogue);
}

// ---------------------------------------------------------------------------------
// down: out[row, n] = w(row) * act[row] . W2[n], bf16, permuted rows; tile = 128 rows x
// TW output columns, wave wn owns columns 128 wn + [0, 128). When H is not a multiple of
// TW, the last tile's columns past H are computed on repeated rows and not written.

template <typename W>
struct DownTile {
  Loader<W> ld;
  int begin, end, nt, valid;
  int slot;               // LDS slot of the tile's row weights (tiles alternate)
  const_f32_ptr sd;       // FP8 block scales of the wave's 128 columns (per K step)
};

template <typename W, typename Table>
__global__ void __launch_bounds__(64 * W::WAVES) down_kernel(const uint8_t* __restrict__ a8,
                                                             const uint8_t* __restrict__ as8, Lists L,
                                                             const float* __restrict__ weights, int weighted,
                                                             Table routed, Table shared, uint16_t* __restrict__ out) {
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = (H + W::TW - 1) / W::TW;
  const TileRange tr = tile_range(active_row_tiles(L) * n_tiles);
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int wm = wave & 1, wn = wave >> 1;
  const LaneOffsets lo = lane_offsets<W>(128 * wn, wm);
  const int64_t wrow_bytes = (int64_t)I * W::STEP_BYTES / 128;
  using Tile = DownTile<W>;
  __shared__ float row_weight[2][BM];

  auto setup = [&](int j, Tile& t) {
    const int logical = tr.first + tr.stride * j;
    const int mt = logical / n_tiles;
    t.nt = logical - mt * n_tiles;
    int expert, begin_, end_;
    if (!resolve_tile(L, mt, expert, begin_, end_)) return false;
    t.begin = uniform_i(begin_);
    t.end = uniform_i(end_);
    const TileWeights tw = tile_weights(routed, shared, uniform_i(expert));
    t.valid = min(W::TW, H - t.nt * W::TW);  // a multiple of 128
    const int nt = t.nt, valid = t.valid, begin = t.begin, end = t.end;
    auto col_row = [nt, valid](int r) { return nt * W::TW + (r < valid ? r : r % valid); };  // never past H
    t.ld.init(
        a8, as8, I / 128, tw.w2, tw.w2s, [&](int r) { return begin + r < end ? begin + r : begin; },
        [&](int r) { return (uint32_t)(col_row(r) * wrow_bytes); },
        [&](int r) { return (uint32_t)(col_row(r) * (I / 32)); });
    // routing weight (or shared gate) of the tile's rows, kept in LDS until the epilogue (at
    // least one barrier later; the two slots alternate between consecutive tiles)
    t.slot = j & 1;
    if (threadIdx.x < BM) {
      const int row = begin + (int)threadIdx.x;
      float w = 1.0f;
      if (weighted && row < end) w = row < L.pairs ? weights[L.order[row]] : L.shared_gate[row - L.pairs];
      row_weight[t.slot][threadIdx.x] = w;
    }
    // FP8: the wave's 128 columns are one 128-row scale block
    t.sd = uniform_ptr(reinterpret_cast<const float*>(tw.w2s) + (int64_t)(col_row(128 * wn) / 128) * (I / 128));
    return true;
  };

  v4f acc[MI][NI];
#pragma unroll
  for (int mi = 0; mi < MI; ++mi)
#pragma unroll
    for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  auto mfma = [&](const Tile& t, const Stage<W>& st, int k) {
    step_mfma<W>(st, lo, acc, [](int mi) { return 16 * mi; },
                 [&](int) { return W::FMT == FMT_FP8 ? t.sd[k] : 1.0f; });
  };

  // lane holds output columns nt*TW + 128 wn + 16 mi + 4 g + r of row 64 wm + 16 ni + c
  auto epilogue = [&](const Tile& t) {
    if (128 * wn < t.valid) {
      const int c = lane % 16, g = lane / 16;
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) {
        const int row = t.begin + 64 * wm + 16 * ni + c;
        if (row >= t.end) continue;
        const float w = row_weight[t.slot][64 * wm + 16 * ni + c];
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) {
          const int col = t.nt * W::TW + 128 * wn + 16 * mi + 4 * g;
          uint2 o;
          o.x = f32_to_bf16_bits(w * acc[mi][ni][0]) | ((uint32_t)f32_to_bf16_bits(w * acc[mi][ni][1]) << 16);
          o.y = f32_to_bf16_bits(w * acc[mi][ni][2]) | ((uint32_t)f32_to_bf16_bits(w * acc[mi][ni][3]) << 16);
          *reinterpret_cast<uint2*>(out + (int64_t)row * H + col) = o;
        }
      }
    }
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
      for (int ni = 0; ni < NI; ++ni) acc[mi][ni] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  };

  __shared__ Stage<W> s0, s1;
  persistent_tiles<W, Tile>(tr, I / 128, s0, s1, setup, mfma, epilogue);
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

// combine: y[t, c] = sum_k rows[inverse[t*K + k], c] (+ rows[P + t, c]), fp32 sum, bf16 out.
// per-pair (combine = 0): out[p, c] = rows[inverse[p], c]. 8 columns per thread.
__global__ void __launch_bounds__(256) combine_rows_kernel(const uint16_t* __restrict__ rows,
                                                           const int32_t* __restrict__ inverse, int tokens, int k,
                                                           int hidden, int has_shared, int combine,
                                                           uint16_t* __restrict__ out) {
  const int t = blockIdx.x;
  const int c8 = blockIdx.y * blockDim.x + threadIdx.x;
  if (c8 * 8 >= hidden) return;
  const int pairs = tokens * k;
  if (!combine) {
    const int row = inverse[t];
    const uint4 v = row >= 0 ? reinterpret_cast<const uint4*>(rows + (int64_t)row * hidden)[c8] : make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(out + (int64_t)t * hidden)[c8] = v;
    return;
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](int row) {
    const uint4 v = reinterpret_cast<const uint4*>(rows + (int64_t)row * hidden)[c8];
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += bf16_bits_to_f32(w[q] & 0xffffu);
      acc[2 * q + 1] += bf16_bits_to_f32(w[q] >> 16);
    }
  };
  for (int j = 0; j < k; ++j) {
    const int row = inverse[t * k + j];
    if (row >= 0) add(row);
  }
  if (has_shared) add(pairs + t);
  uint4 o;
  o.x = f32_to_bf16_bits(acc[0]) | ((uint32_t)f32_to_bf16_bits(acc[1]) << 16);
  o.y = f32_to_bf16_bits(acc[2]) | ((uint32_t)f32_to_bf16_bits(acc[3]) << 16);
  o.z = f32_to_bf16_bits(acc[4]) | ((uint32_t)f32_to_bf16_bits(acc[5]) << 16);
  o.w = f32_to_bf16_bits(acc[6]) | ((uint32_t)f32_to_bf16_bits(acc[7]) << 16);
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
  size_t permute_ws, order, inverse, offsets, tiles, tile_count, gate, x8, xs, a8, as8, rows, total;
};

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
  p.x8 = at;         at += align256((size_t)tokens * (hidden / 128) * CHUNK);
  p.xs = at;         at += align256((size_t)tokens * (hidden / 128) * 8);
  p.a8 = at;         at += align256((size_t)rows * (inter / 128) * CHUNK);
  p.as8 = at;        at += align256((size_t)rows * (inter / 128) * 8);
  p.rows = at;       at += align256(sizeof(uint16_t) * (size_t)rows * hidden);
  p.total = at;
  return p;
}

template <typename W, typename Table>
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
  if constexpr (W::FMT == FMT_FP4) {  // the K loop reads 4 scale bytes of a row as one dword
    auto dword_rows = [](const void* p, int64_t stride) { return (uintptr_t)p % 4 == 0 && stride % 4 == 0; };
    for (const Table* t : {&routed, shared})
      if (t && (!dword_rows(t->gate_up_scales, t->gate_up_scales_stride) ||
                !dword_rows(t->down_scales, t->down_scales_stride)))
        fail("prefill: MXFP4 scale regions and strides must be 4-byte aligned");
  }
  if ((int64_t)rows * (I / 128) * CHUNK >= ((int64_t)1 << 32) || (int64_t)tokens * (H / 128) * CHUNK >= ((int64_t)1 << 32))
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
  if (has_shared) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3(tokens), dim3(64), 0, s, x, shared_gate, tokens, H,
                       (float*)L.shared_gate);
    check_launch("shared_gate");
  }
  uint8_t* x8 = base + p.x8;
  uint8_t* xs = base + p.xs;
  const int64_t split_jobs = (int64_t)tokens * (H / 128);
  hipLaunchKernelGGL(split_rows_kernel, dim3((unsigned)((split_jobs + 3) / 4)), dim3(256), 0, s, x, tokens, H, x8, xs);
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
  uint8_t* a8 = base + p.a8;
  uint8_t* as8 = base + p.as8;
  uint16_t* out_rows = (uint16_t*)(base + p.rows);
  TimingEvents* te = g_timing.load() ? timing_events() : nullptr;
  if (te) check_hip(hipEventRecord(te->ev[0], s), "hipEventRecord");
  hipLaunchKernelGGL((gate_up_kernel<W, Table>), grid_for((I + W::TW / 2 - 1) / (W::TW / 2)), dim3(64 * W::WAVES), 0,
                     s, x8, xs, L, routed, sh, a8, as8);
  check_launch("gate_up");
  if (te) check_hip(hipEventRecord(te->ev[1], s), "hipEventRecord");
  hipLaunchKernelGGL((down_kernel<W, Table>), grid_for((H + W::TW - 1) / W::TW), dim3(64 * W::WAVES), 0, s, a8, as8, L,
                     weights,
                     combine ? 1 : 0, routed, sh, out_rows);
  check_launch("down");
  if (te) check_hip(hipEventRecord(te->ev[2], s), "hipEventRecord");
  if (combine)
    hipLaunchKernelGGL(combine_rows_kernel, dim3(tokens, (H / 8 + 255) / 256), dim3(256), 0, s, out_rows, inverse,
                       tokens, k, H, has_shared ? 1 : 0, 1, y);
  else
    hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)pairs, (H / 8 + 255) / 256), dim3(256), 0, s, out_rows,
                       inverse, tokens, k, H, 0, 0, y);
  check_launch("combine_rows");
}

}  // namespace mf

size_t prefill_workspace_size(int tokens, int k, const wm_mxfp4_experts& e, bool has_shared) {
  return mf::layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

void prefill_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                   const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                   uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  mf::run<mf::Fp4Weights>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
}

size_t prefill_fp8_workspace_size(int tokens, int k, const wm_fp8_experts& e, bool has_shared) {
  return mf::layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

void prefill_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                 const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                 uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  mf::run<mf::Fp8Weights>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, ws, ws_bytes, s);
}

}  // namespace wm

extern "C" {

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
