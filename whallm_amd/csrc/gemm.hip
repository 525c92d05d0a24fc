// Prefill-time MXFP4 expert FFN: grouped GEMMs on gfx950 bf16 MFMA with the
// FP4 weights dequantized in registers (exact: every E2M1 value times a power of
// two is a bf16), over the row tiles the permute kernel lists.
//
// Replaces gather_rows16 + expert_gemm_sg (gate_up) + expert_act + expert_gemm_sg
// (down) + moe_combine_rows (Native/QwenNative/kernels.metal:691-765, driven from
// engine.mm:2104-2162) and mx.gather_qmm (qwen4_exp.py:857-897):
//
//   gate_up : tile = 128 permuted rows x 64 intermediate columns. The B tile holds
//             the 64 gate rows and the 64 matching up rows of the expert, so each
//             lane owns gate and up of the same (row, column) and SwiGLU is the
//             epilogue. A rows are gathered straight from x through the permute's
//             row -> pair list: no packed copy of the input is made.
//   down    : tile = 128 permuted rows x 128 output columns, act (bf16) in, the
//             row's routing weight (or the shared expert's sigmoid gate) applied in
//             the epilogue; out rows stay in permuted order.
//   combine : y[t] = sum of the token's K + 1 rows, in k order, shared last.
//
// The shared expert is one more row group after the routed ones (rows P .. P+T-1).
// Work tiles are mapped XCD-major: the 8 XCDs each take a contiguous range of
// (row tile, column tile) pairs, so the column tiles of one row tile and the row
// tiles of one expert meet in the same L2.
#include <cmath>

#include "wm_common.h"
#include "moe_internal.h"

namespace wm {

constexpr int BM = 128;          // rows per tile
constexpr int BN = 128;          // B rows per tile
constexpr int BK = 64;           // K per LDS stage (two MFMA k-steps of 32)
constexpr int A_STRIDE = 72;     // bf16 per LDS row of A: 64 + 8 pad (16-byte shift per row)
constexpr int B_STRIDE = 48;     // bytes per LDS row of packed B: 32 + 16 pad
constexpr int XCDS = 8;

struct PrefillLists {
  const int32_t* order;       // [P] pair of each permuted row
  const int32_t* inverse;     // [P] permuted row of each pair
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
__device__ __forceinline__ bool resolve_tile(const PrefillLists& L, int m, int& expert, int& begin, int& end) {
  int routed_tiles = L.tile_count[0];
  if (m < routed_tiles) {
    expert = L.tiles[2 * m];
    begin = L.tiles[2 * m + 1];
    end = min(begin + BM, L.offsets[expert + 1]);
    return true;
  }
  int j = m - routed_tiles;
  if (!L.has_shared || j * BM >= L.tokens) return false;
  expert = -1;
  begin = L.pairs + j * BM;
  end = min(begin + BM, L.pairs + L.tokens);
  return true;
}

__device__ __forceinline__ int active_row_tiles(const PrefillLists& L) {
  return L.tile_count[0] + (L.has_shared ? (L.tokens + BM - 1) / BM : 0);
}

// XCD-major work mapping: returns false for workgroups past the active work.
__device__ __forceinline__ bool map_work(int active, int& logical) {
  int l = blockIdx.x;
  int xcd = l % XCDS, local = l / XCDS;
  int share = (active + XCDS - 1) / XCDS;
  if (local >= share) return false;
  logical = xcd * share + local;
  return logical < active;
}

// B fragment of a 16x16x32 MFMA from packed FP4 in LDS: 8 k-values of B row j.
__device__ __forceinline__ wm_bf16x8 b_fragment(const uint8_t* b_lds, const uint8_t* s_lds, int j, int ks, int quad) {
  uint32_t word = *reinterpret_cast<const uint32_t*>(b_lds + j * B_STRIDE + ks * 16 + quad * 4);
  float scale = e8m0_scale_operand(s_lds[j * 2 + ks]);
  wm_bf16x2 v[4];
  fp4x8_to_bf16(word, scale, v);
  wm_bf16x8 out;
  out[0] = v[0][0]; out[1] = v[0][1]; out[2] = v[1][0]; out[3] = v[1][1];
  out[4] = v[2][0]; out[5] = v[2][1]; out[6] = v[3][0]; out[7] = v[3][1];
  return out;
}

__device__ __forceinline__ wm_bf16x8 a_fragment(const uint16_t* a_lds, int row, int ks, int quad) {
  uint4 v = *reinterpret_cast<const uint4*>(a_lds + row * A_STRIDE + ks * 32 + quad * 8);
  return __builtin_bit_cast(wm_bf16x8, v);
}

// The shared K loop of both GEMMs. `a_src[q]` are this thread's 4 A source rows
// (nullptr = zero row), `b_src` its B row (16-byte half `b_half` of each 32-byte
// stage row), `s_src` its scale row (threads < 128). acc[mi][ni] for the wave's
// 4 x 4 16x16 sub-tiles; B-tile row of sub-tile ni is b_row(ni).
struct KLoopArgs {
  const uint16_t* a_src[4];
  int a_col8[4];
  int a_row[4];
  const uint8_t* b_src;
  int b_row;
  int b_half;
  const uint8_t* s_src;
  int k_tiles;
};

template <typename BRow>
__device__ __forceinline__ void k_loop(const KLoopArgs& g, uint16_t* a_lds, uint8_t* b_lds, uint8_t* s_lds,
                                       wm_f32x4 (&acc)[4][4], int wm_, BRow b_row) {
  const int tid = threadIdx.x, lane = tid % 64;
  const int quad = lane / 16, r16 = lane % 16;
  uint4 a_reg[4];
  uint4 b_reg;
  uint16_t s_reg = 0;
  auto load = [&](int kt) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      a_reg[q] = g.a_src[q] ? *reinterpret_cast<const uint4*>(g.a_src[q] + kt * BK + g.a_col8[q] * 8)
                            : make_uint4(0, 0, 0, 0);
    b_reg = *reinterpret_cast<const uint4*>(g.b_src + kt * 32 + g.b_half * 16);
    if (g.s_src) s_reg = *reinterpret_cast<const uint16_t*>(g.s_src + kt * 2);
  };
  auto store = [&](int buf) {
    uint16_t* a = a_lds + buf * BM * A_STRIDE;
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(a + g.a_row[q] * A_STRIDE + g.a_col8[q] * 8) = a_reg[q];
    *reinterpret_cast<uint4*>(b_lds + buf * BN * B_STRIDE + g.b_row * B_STRIDE + g.b_half * 16) = b_reg;
    if (g.s_src) *reinterpret_cast<uint16_t*>(s_lds + buf * BN * 2 + tid * 2) = s_reg;
  };
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < g.k_tiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < g.k_tiles) load(kt + 1);
    const uint16_t* a = a_lds + cur * BM * A_STRIDE;
    const uint8_t* b = b_lds + cur * BN * B_STRIDE;
    const uint8_t* s = s_lds + cur * BN * 2;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      wm_bf16x8 af[4], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) af[mi] = a_fragment(a, wm_ * 64 + mi * 16 + r16, ks, quad);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) bfr[ni] = b_fragment(b, s, b_row(ni) + r16, ks, quad);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
    }
    if (kt + 1 < g.k_tiles) store(cur ^ 1);
    __syncthreads();
  }
}

// act[row, c] = swiglu(x[token(row)] . Wg[c], x[token(row)] . Wu[c]) for the tile's rows.
__global__ void __launch_bounds__(256) grouped_gate_up_kernel(const uint16_t* __restrict__ x, PrefillLists L,
                                                              wm_mxfp4_experts routed, wm_mxfp4_experts shared,
                                                              uint16_t* __restrict__ act) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2 * BM * A_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[2 * BN * B_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t s_lds[2 * BN * 2];
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = I / 64;
  int logical;
  if (!map_work(active_row_tiles(L) * n_tiles, logical)) return;
  const int mt = logical / n_tiles, nt = logical % n_tiles;
  int expert, begin, end;
  if (!resolve_tile(L, mt, expert, begin, end)) return;
  const wm_mxfp4_experts& table = expert < 0 ? shared : routed;
  ExpertRegions r = expert_regions(table, expert < 0 ? 0 : expert);
  const int up_first = table.up_first;
  const float limit = table.swiglu_limit;

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  KLoopArgs g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int c = tid + 256 * q;          // 1024 chunks of 8 bf16: 128 rows x 8 chunks
    int row = c / 8;
    g.a_row[q] = row;
    g.a_col8[q] = c % 8;
    int pr = begin + row;
    if (pr < end) {
      int token = pr < L.pairs ? L.order[pr] / L.k : pr - L.pairs;
      g.a_src[q] = x + (int64_t)token * H;
    } else {
      g.a_src[q] = nullptr;
    }
  }
  // B tile rows 0..63: gate rows nt*64 + j; 64..127: the matching up rows.
  {
    int j = tid / 2;
    int c = nt * 64 + (j & 63);
    bool gate = j < 64;
    int wrow = (gate ^ (up_first != 0)) ? c : I + c;
    g.b_row = j;
    g.b_half = tid % 2;
    g.b_src = r.gate_up + (int64_t)wrow * (H / 2);
    if (tid < 128) {
      int cj = nt * 64 + (tid & 63);
      bool gate_s = tid < 64;
      int srow = (gate_s ^ (up_first != 0)) ? cj : I + cj;
      g.s_src = r.gate_up_scales + (int64_t)srow * (H / 32);
    } else {
      g.s_src = nullptr;
    }
  }
  g.k_tiles = H / BK;
  wm_f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int wm_ = wave / 2, wn = wave % 2;
  // Sub-tiles 0, 1: gate columns 32 wn + 16 ni; 2, 3: the same up columns.
  k_loop(g, a_lds, b_lds, s_lds, acc, wm_, [&](int ni) { return (ni < 2 ? 0 : 64) + 32 * wn + 16 * (ni & 1); });

  const int quad = lane / 16, r16 = lane % 16;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int row = begin + wm_ * 64 + mi * 16 + quad * 4 + e;
        if (row >= end) continue;
        float gv = acc[mi][ni][e], uv = acc[mi][ni + 2][e];
        if (limit > 0.0f) {
          gv = fminf(gv, limit);
          uv = fminf(fmaxf(uv, -limit), limit);
        }
        int col = nt * 64 + 32 * wn + 16 * ni + r16;
        act[(int64_t)row * I + col] = f32_to_bf16_bits(silu(gv) * uv);
      }
}

// out[row, n] = w(row) * act[row] . Wd[n].
__global__ void __launch_bounds__(256) grouped_down_kernel(const uint16_t* __restrict__ act, PrefillLists L,
                                                           const float* __restrict__ weights, int weighted,
                                                           wm_mxfp4_experts routed, wm_mxfp4_experts shared,
                                                           uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2 * BM * A_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[2 * BN * B_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t s_lds[2 * BN * 2];
  const int H = routed.hidden, I = routed.inter;
  const int n_tiles = H / BN;
  int logical;
  if (!map_work(active_row_tiles(L) * n_tiles, logical)) return;
  const int mt = logical / n_tiles, nt = logical % n_tiles;
  int expert, begin, end;
  if (!resolve_tile(L, mt, expert, begin, end)) return;
  const wm_mxfp4_experts& table = expert < 0 ? shared : routed;
  ExpertRegions r = expert_regions(table, expert < 0 ? 0 : expert);

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  KLoopArgs g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int c = tid + 256 * q;
    int row = c / 8;
    g.a_row[q] = row;
    g.a_col8[q] = c % 8;
    g.a_src[q] = begin + row < end ? act + (int64_t)(begin + row) * I : nullptr;
  }
  {
    int j = tid / 2;
    g.b_row = j;
    g.b_half = tid % 2;
    g.b_src = r.down + (int64_t)(nt * BN + j) * (I / 2);
    g.s_src = tid < 128 ? r.down_scales + (int64_t)(nt * BN + tid) * (I / 32) : nullptr;
  }
  g.k_tiles = I / BK;
  wm_f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int wm_ = wave / 2, wn = wave % 2;
  k_loop(g, a_lds, b_lds, s_lds, acc, wm_, [&](int ni) { return 64 * wn + 16 * ni; });

  const int quad = lane / 16, r16 = lane % 16;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = begin + wm_ * 64 + mi * 16 + quad * 4 + e;
      if (row >= end) continue;
      float w = 1.0f;
      if (weighted) w = row < L.pairs ? weights[L.order[row]] : L.shared_gate[row - L.pairs];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        int col = nt * BN + 64 * wn + 16 * ni + r16;
        out[(int64_t)row * H + col] = f32_to_bf16_bits(w * acc[mi][ni][e]);
      }
    }
}

// gate[t] = sigmoid(x[t] . g) (1 when g is null); one wave per token.
__global__ void __launch_bounds__(64) shared_gate_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ g,
                                                         int tokens, int hidden, float* __restrict__ gate) {
  int t = blockIdx.x, lane = threadIdx.x;
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
  int t = blockIdx.x;
  int c8 = blockIdx.y * blockDim.x + threadIdx.x;
  if (c8 * 8 >= hidden) return;
  int pairs = tokens * k;
  if (!combine) {
    int row = inverse[t];
    uint4 v = row >= 0 ? reinterpret_cast<const uint4*>(rows + (int64_t)row * hidden)[c8] : make_uint4(0, 0, 0, 0);
    reinterpret_cast<uint4*>(out + (int64_t)t * hidden)[c8] = v;
    return;
  }
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  auto add = [&](int row) {
    uint4 v = reinterpret_cast<const uint4*>(rows + (int64_t)row * hidden)[c8];
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += bf16_bits_to_f32(w[q] & 0xffffu);
      acc[2 * q + 1] += bf16_bits_to_f32(w[q] >> 16);
    }
  };
  for (int j = 0; j < k; ++j) {
    int row = inverse[t * k + j];
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
// FP8-E4M3 weights with fp32 128 x 128 block scales (DeepSeek-V3 expert format). The
// bytes convert to bf16 exactly inside the B fragment; each 128-wide K block is
// accumulated on its own and added to the running sums times its block scale, so the
// scale is applied in fp32 as in the dequant-then-matmul reference.
constexpr int B8_STRIDE = 80;    // bytes per LDS row of E4M3 B: 64 + 16 pad

__device__ __forceinline__ wm_bf16x8 b_fragment_fp8(const uint8_t* b_lds, int j, int ks, int quad) {
  const uint2 w = *reinterpret_cast<const uint2*>(b_lds + j * B8_STRIDE + ks * 32 + quad * 8);
  const wm_bf16x2 v0 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, false);
  const wm_bf16x2 v1 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.x, 1.0f, true);
  const wm_bf16x2 v2 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, false);
  const wm_bf16x2 v3 = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w.y, 1.0f, true);
  wm_bf16x8 out;
  out[0] = v0[0]; out[1] = v0[1]; out[2] = v1[0]; out[3] = v1[1];
  out[4] = v2[0]; out[5] = v2[1]; out[6] = v3[0]; out[7] = v3[1];
  return out;
}

// The K loop of the FP8 GEMMs: like k_loop, with 64-byte B rows (two 16-byte halves per
// thread) and the per-block scale step every two K tiles. scale(kb, ni) is the fp32
// block scale of sub-tile column group ni for K block kb.
template <typename BRow, typename Scale>
__device__ __forceinline__ void k_loop_fp8(const KLoopArgs& g, uint16_t* a_lds, uint8_t* b_lds,
                                           wm_f32x4 (&acc)[4][4], int wm_, BRow b_row, Scale scale) {
  const int tid = threadIdx.x, lane = tid % 64;
  const int quad = lane / 16, r16 = lane % 16;
  uint4 a_reg[4];
  uint4 b_reg[2];
  wm_f32x4 blk[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) blk[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  auto load = [&](int kt) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      a_reg[q] = g.a_src[q] ? *reinterpret_cast<const uint4*>(g.a_src[q] + kt * BK + g.a_col8[q] * 8)
                            : make_uint4(0, 0, 0, 0);
    const uint8_t* b = g.b_src + kt * 64 + g.b_half * 32;
    b_reg[0] = *reinterpret_cast<const uint4*>(b);
    b_reg[1] = *reinterpret_cast<const uint4*>(b + 16);
  };
  auto store = [&](int buf) {
    uint16_t* a = a_lds + buf * BM * A_STRIDE;
#pragma unroll
    for (int q = 0; q < 4; ++q) *reinterpret_cast<uint4*>(a + g.a_row[q] * A_STRIDE + g.a_col8[q] * 8) = a_reg[q];
    uint8_t* b = b_lds + buf * BN * B8_STRIDE + g.b_row * B8_STRIDE + g.b_half * 32;
    *reinterpret_cast<uint4*>(b) = b_reg[0];
    *reinterpret_cast<uint4*>(b + 16) = b_reg[1];
  };
  load(0);
  store(0);
  __syncthreads();
  for (int kt = 0; kt < g.k_tiles; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < g.k_tiles) load(kt + 1);
    const uint16_t* a = a_lds + cur * BM * A_STRIDE;
    const uint8_t* b = b_lds + cur * BN * B8_STRIDE;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      wm_bf16x8 af[4], bfr[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) af[mi] = a_fragment(a, wm_ * 64 + mi * 16 + r16, ks, quad);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) bfr[ni] = b_fragment_fp8(b, b_row(ni) + r16, ks, quad);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          blk[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], blk[mi][ni], 0, 0, 0);
    }
    if (kt & 1) {  // end of a 128-wide K block (k_tiles is even)
      const int kb = kt / 2;
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        const float sc = scale(kb, ni);
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
          for (int e = 0; e < 4; ++e) acc[mi][ni][e] = fmaf(sc, blk[mi][ni][e], acc[mi][ni][e]);
          blk[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
      }
    }
    if (kt + 1 < g.k_tiles) store(cur ^ 1);
    __syncthreads();
  }
}

__device__ __forceinline__ Fp8Regions fp8_tile_regions(const wm_fp8_experts& routed, const wm_fp8_experts& shared,
                                                       int expert) {
  return expert < 0 ? fp8_regions(shared, 0) : fp8_regions(routed, expert);
}

// act[row, c] = swiglu(x[token(row)] . W1[c], x[token(row)] . W3[c]) with FP8 weights.
__global__ void __launch_bounds__(256) fp8_grouped_gate_up_kernel(const uint16_t* __restrict__ x, PrefillLists L,
                                                                  wm_fp8_experts routed, wm_fp8_experts shared,
                                                                  uint16_t* __restrict__ act) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2 * BM * A_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[2 * BN * B8_STRIDE];
  const int H = routed.hidden, I = routed.inter, HB = H / 128;
  const int n_tiles = I / 64;
  int logical;
  if (!map_work(active_row_tiles(L) * n_tiles, logical)) return;
  const int mt = logical / n_tiles, nt = logical % n_tiles;
  int expert, begin, end;
  if (!resolve_tile(L, mt, expert, begin, end)) return;
  const wm_fp8_experts& table = expert < 0 ? shared : routed;
  const Fp8Regions r = fp8_tile_regions(routed, shared, expert);
  const int up_first = table.up_first;
  const float limit = table.swiglu_limit;

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  KLoopArgs g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int c = tid + 256 * q;
    int row = c / 8;
    g.a_row[q] = row;
    g.a_col8[q] = c % 8;
    int pr = begin + row;
    if (pr < end) {
      int token = pr < L.pairs ? L.order[pr] / L.k : pr - L.pairs;
      g.a_src[q] = x + (int64_t)token * H;
    } else {
      g.a_src[q] = nullptr;
    }
  }
  // B tile rows 0..63: gate rows nt*64 + j; 64..127: the matching up rows.
  const int gate_row0 = up_first ? I + nt * 64 : nt * 64;
  const int up_row0 = up_first ? nt * 64 : I + nt * 64;
  {
    int j = tid / 2;
    int wrow = (j < 64 ? gate_row0 : up_row0) + (j & 63);
    g.b_row = j;
    g.b_half = tid % 2;
    g.b_src = r.w13 + (int64_t)wrow * H;
    g.s_src = nullptr;
  }
  g.k_tiles = H / BK;
  wm_f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int wm_ = wave / 2, wn = wave % 2;
  const float* sg = r.w13_scales + (int64_t)(gate_row0 / 128) * HB;
  const float* su = r.w13_scales + (int64_t)(up_row0 / 128) * HB;
  k_loop_fp8(g, a_lds, b_lds, acc, wm_, [&](int ni) { return (ni < 2 ? 0 : 64) + 32 * wn + 16 * (ni & 1); },
             [&](int kb, int ni) { return ni < 2 ? sg[kb] : su[kb]; });

  const int quad = lane / 16, r16 = lane % 16;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 2; ++ni)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        int row = begin + wm_ * 64 + mi * 16 + quad * 4 + e;
        if (row >= end) continue;
        float gv = acc[mi][ni][e], uv = acc[mi][ni + 2][e];
        if (limit > 0.0f) {
          gv = fminf(gv, limit);
          uv = fminf(fmaxf(uv, -limit), limit);
        }
        int col = nt * 64 + 32 * wn + 16 * ni + r16;
        act[(int64_t)row * I + col] = f32_to_bf16_bits(silu(gv) * uv);
      }
}

// out[row, n] = w(row) * act[row] . W2[n] with FP8 weights.
__global__ void __launch_bounds__(256) fp8_grouped_down_kernel(const uint16_t* __restrict__ act, PrefillLists L,
                                                               const float* __restrict__ weights, int weighted,
                                                               wm_fp8_experts routed, wm_fp8_experts shared,
                                                               uint16_t* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) uint16_t a_lds[2 * BM * A_STRIDE];
  __shared__ __attribute__((aligned(16))) uint8_t b_lds[2 * BN * B8_STRIDE];
  const int H = routed.hidden, I = routed.inter, IB = I / 128;
  const int n_tiles = H / BN;
  int logical;
  if (!map_work(active_row_tiles(L) * n_tiles, logical)) return;
  const int mt = logical / n_tiles, nt = logical % n_tiles;
  int expert, begin, end;
  if (!resolve_tile(L, mt, expert, begin, end)) return;
  const Fp8Regions r = fp8_tile_regions(routed, shared, expert);

  const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
  KLoopArgs g;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int c = tid + 256 * q;
    int row = c / 8;
    g.a_row[q] = row;
    g.a_col8[q] = c % 8;
    g.a_src[q] = begin + row < end ? act + (int64_t)(begin + row) * I : nullptr;
  }
  {
    int j = tid / 2;
    g.b_row = j;
    g.b_half = tid % 2;
    g.b_src = r.w2 + (int64_t)(nt * BN + j) * I;
    g.s_src = nullptr;
  }
  g.k_tiles = I / BK;
  wm_f32x4 acc[4][4];
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = wm_f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  const int wm_ = wave / 2, wn = wave % 2;
  const float* sd = r.w2_scales + (int64_t)nt * IB;  // BN = 128: one row block per tile
  k_loop_fp8(g, a_lds, b_lds, acc, wm_, [&](int ni) { return 64 * wn + 16 * ni; },
             [&](int kb, int) { return sd[kb]; });

  const int quad = lane / 16, r16 = lane % 16;
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      int row = begin + wm_ * 64 + mi * 16 + quad * 4 + e;
      if (row >= end) continue;
      float w = 1.0f;
      if (weighted) w = row < L.pairs ? weights[L.order[row]] : L.shared_gate[row - L.pairs];
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) {
        int col = nt * BN + 64 * wn + 16 * ni + r16;
        out[(int64_t)row * H + col] = f32_to_bf16_bits(w * acc[mi][ni][e]);
      }
    }
}

// ---------------------------------------------------------------------------------
static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct PrefillLayout {
  size_t permute_ws, order, inverse, offsets, tiles, tile_count, gate, act, rows, total;
};

static PrefillLayout prefill_layout(int tokens, int k, int experts, int hidden, int inter, bool has_shared) {
  int64_t pairs = (int64_t)tokens * k;
  int64_t rows = pairs + (has_shared ? tokens : 0);
  int64_t max_tiles = (pairs + BM - 1) / BM + experts;
  PrefillLayout p{};
  size_t at = 0;
  p.permute_ws = at; at += align256(wm_permute_workspace_size(pairs, experts));
  p.order = at;      at += align256(sizeof(int32_t) * (size_t)(pairs > 0 ? pairs : 1));
  p.inverse = at;    at += align256(sizeof(int32_t) * (size_t)(pairs > 0 ? pairs : 1));
  p.offsets = at;    at += align256(sizeof(int32_t) * (size_t)(experts + 1));
  p.tiles = at;      at += align256(sizeof(int32_t) * 2 * (size_t)max_tiles);
  p.tile_count = at; at += align256(sizeof(int32_t));
  p.gate = at;       at += align256(sizeof(float) * (size_t)(tokens > 0 ? tokens : 1));
  p.act = at;        at += align256(sizeof(uint16_t) * (size_t)rows * inter);
  p.rows = at;       at += align256(sizeof(uint16_t) * (size_t)rows * hidden);
  p.total = at;
  return p;
}

size_t prefill_workspace_size(int tokens, int k, const wm_mxfp4_experts& e, bool has_shared) {
  return prefill_layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

void prefill_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                   const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                   uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  if (H % BN || I % BK) fail("prefill: hidden must be a multiple of 128 and intermediate of 64");
  const bool has_shared = combine && shared != nullptr;
  PrefillLayout p = prefill_layout(tokens, k, routed.experts, H, I, has_shared);
  if (ws_bytes < p.total) fail("prefill: workspace too small");
  uint8_t* base = (uint8_t*)ws;
  int64_t pairs = (int64_t)tokens * k;
  PrefillLists L;
  L.order = (int32_t*)(base + p.order);
  L.inverse = (int32_t*)(base + p.inverse);
  L.offsets = (int32_t*)(base + p.offsets);
  L.tiles = (int32_t*)(base + p.tiles);
  L.tile_count = (int32_t*)(base + p.tile_count);
  L.shared_gate = (float*)(base + p.gate);
  L.pairs = (int)pairs;
  L.tokens = tokens;
  L.k = k;
  L.has_shared = has_shared ? 1 : 0;
  if (wm_permute(indices, pairs, routed.experts, BM, (int32_t*)L.order, (int32_t*)L.inverse, (int32_t*)L.offsets,
                 (int32_t*)L.tiles, (int32_t*)L.tile_count, base + p.permute_ws,
                 wm_permute_workspace_size(pairs, routed.experts), s) != 0)
    fail(std::string("prefill permute: ") + wm_last_error());
  if (has_shared) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3(tokens), dim3(64), 0, s, x, shared_gate, tokens, H,
                       (float*)L.shared_gate);
    check_launch("shared_gate");
  }
  wm_mxfp4_experts sh = shared ? *shared : routed;
  int64_t max_row_tiles = (pairs + BM - 1) / BM + routed.experts + (has_shared ? (tokens + BM - 1) / BM : 0);
  // Upper bound of the work tiles, rounded up so every XCD's share fits the grid.
  auto grid_for = [&](int n_tiles) {
    int64_t work = max_row_tiles * n_tiles;
    int64_t per_xcd = (work + XCDS - 1) / XCDS;
    return dim3((unsigned)(per_xcd * XCDS));
  };
  uint16_t* act = (uint16_t*)(base + p.act);
  uint16_t* rows = (uint16_t*)(base + p.rows);
  hipLaunchKernelGGL(grouped_gate_up_kernel, grid_for(I / 64), dim3(256), 0, s, x, L, routed, sh, act);
  check_launch("grouped_gate_up");
  hipLaunchKernelGGL(grouped_down_kernel, grid_for(H / BN), dim3(256), 0, s, act, L, weights, combine ? 1 : 0, routed,
                     sh, rows);
  check_launch("grouped_down");
  if (combine)
    hipLaunchKernelGGL(combine_rows_kernel, dim3(tokens, (H / 8 + 255) / 256), dim3(256), 0, s, rows, L.inverse,
                       tokens, k, H, has_shared ? 1 : 0, 1, y);
  else
    hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)pairs, (H / 8 + 255) / 256), dim3(256), 0, s, rows,
                       L.inverse, tokens, k, H, 0, 0, y);
  check_launch("combine_rows");
}

size_t prefill_fp8_workspace_size(int tokens, int k, const wm_fp8_experts& e, bool has_shared) {
  return prefill_layout(tokens, k, e.experts, e.hidden, e.inter, has_shared).total;
}

void prefill_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                 const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                 uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  if (H % 128 || I % 128) fail("FP8 prefill: hidden and intermediate must be multiples of 128");
  const bool has_shared = combine && shared != nullptr;
  PrefillLayout p = prefill_layout(tokens, k, routed.experts, H, I, has_shared);
  if (ws_bytes < p.total) fail("prefill: workspace too small");
  uint8_t* base = (uint8_t*)ws;
  int64_t pairs = (int64_t)tokens * k;
  PrefillLists L;
  L.order = (int32_t*)(base + p.order);
  L.inverse = (int32_t*)(base + p.inverse);
  L.offsets = (int32_t*)(base + p.offsets);
  L.tiles = (int32_t*)(base + p.tiles);
  L.tile_count = (int32_t*)(base + p.tile_count);
  L.shared_gate = (float*)(base + p.gate);
  L.pairs = (int)pairs;
  L.tokens = tokens;
  L.k = k;
  L.has_shared = has_shared ? 1 : 0;
  if (wm_permute(indices, pairs, routed.experts, BM, (int32_t*)L.order, (int32_t*)L.inverse, (int32_t*)L.offsets,
                 (int32_t*)L.tiles, (int32_t*)L.tile_count, base + p.permute_ws,
                 wm_permute_workspace_size(pairs, routed.experts), s) != 0)
    fail(std::string("prefill permute: ") + wm_last_error());
  if (has_shared) {
    hipLaunchKernelGGL(shared_gate_kernel, dim3(tokens), dim3(64), 0, s, x, shared_gate, tokens, H,
                       (float*)L.shared_gate);
    check_launch("shared_gate");
  }
  const wm_fp8_experts sh = shared ? *shared : routed;
  int64_t max_row_tiles = (pairs + BM - 1) / BM + routed.experts + (has_shared ? (tokens + BM - 1) / BM : 0);
  auto grid_for = [&](int n_tiles) {
    int64_t work = max_row_tiles * n_tiles;
    int64_t per_xcd = (work + XCDS - 1) / XCDS;
    return dim3((unsigned)(per_xcd * XCDS));
  };
  uint16_t* act = (uint16_t*)(base + p.act);
  uint16_t* rows = (uint16_t*)(base + p.rows);
  hipLaunchKernelGGL(fp8_grouped_gate_up_kernel, grid_for(I / 64), dim3(256), 0, s, x, L, routed, sh, act);
  check_launch("fp8_grouped_gate_up");
  hipLaunchKernelGGL(fp8_grouped_down_kernel, grid_for(H / BN), dim3(256), 0, s, act, L, weights, combine ? 1 : 0,
                     routed, sh, rows);
  check_launch("fp8_grouped_down");
  if (combine)
    hipLaunchKernelGGL(combine_rows_kernel, dim3(tokens, (H / 8 + 255) / 256), dim3(256), 0, s, rows, L.inverse,
                       tokens, k, H, has_shared ? 1 : 0, 1, y);
  else
    hipLaunchKernelGGL(combine_rows_kernel, dim3((unsigned)pairs, (H / 8 + 255) / 256), dim3(256), 0, s, rows,
                       L.inverse, tokens, k, H, 0, 0, y);
  check_launch("combine_rows");
}

}  // namespace wm
