// Decode-time FP8-E4M3 expert FFN with fp32 128x128 block scales (the DeepSeek-V3
// expert format, mimo/weights.py:17-43) or E8M0 32x32 block scales (the V4.1 release,
// deepseek_v41/dequant.py:45-50): fused dequant + GEMV, HBM-bound. Widths are multiples of
// 128 up to 8192: a lane reads 16 bytes of each 1024-byte chunk of a row, and the lanes past
// a row's end (the last chunk of a width that is not a multiple of 1024) load nothing.
//
// Replaces the reference's FP8 expert linears (Native/DeepSeekNative/kernels.metal:82-124,
// linear_fp8 of the shared expert; the routed experts decode FP8 only at install time,
// Sources/DeepSeekRepack/Repacker.swift:622-627) with two kernels:
//
//   fp8_gate_up_act : one workgroup = (pair, 8 intermediate rows); a wave streams the
//                     gate and up rows of 2 rows i: each lane reads 16 bytes of a row per
//                     1024-byte chunk (fully coalesced), converts them to bf16 exactly
//                     (v_cvt_scalef32_pk_bf16_fp8 with scale 1), dots them with the bf16
//                     input (v_dot2_f32_bf16) and multiplies the 16-column partial by the
//                     scale of its block (fp32, or 2^(b-127) of its E8M0 byte, both exact
//                     powers or floats applied once per partial); silu(gate) * up (clamped when the
//                     table sets a SwiGLU limit) in fp32 -> act, stored as bf16. The reference
//                     rounds the gate and up projections to bf16 before the SwiGLU and feeds the
//                     shared expert's act to w2 as bf16 (deepseek_v41/moe.py:86-93), so rounding
//                     act once is an error of the size it already carries; the bf16 rows halve the
//                     down kernel's act reads and take the bf16 dot.
//   fp8_down        : one workgroup = (token, 8 output rows); the four waves split the
//                     token's experts (routed + shared) and keep routing-weighted partial
//                     sums per row, reduced once: y[t, o] = sum_k w_k act_k . Wd_k[o]
//                     (+ gate(t) act_s . Wd_s[o]), each 16-column partial a v_dot2_f32_bf16
//                     chain of the exactly converted weights with the bf16 act. The per-pair
//                     mode writes each pair's row unweighted (router order, the
//                     StreamingExperts contract).
//
// Weight rows are streamed once per call, so their loads carry the non-temporal hint (4%
// faster C4 decode steps than plain loads).
#include <cmath>

#include "wm_common.h"
#include "moe_internal.h"

namespace wm {

// 16 E4M3 bytes dotted with 16 bf16 values (8 words); products exact, fp32 sum.
__device__ __forceinline__ float e4m3x16_dot_bf16(uint4 w, const uint32_t* xw, float acc) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const wm_bf16x2 lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(words[j], 1.0f, false);
    const wm_bf16x2 hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(words[j], 1.0f, true);
    acc = dot2_bf16(lo, bits_to_bf16x2(xw[2 * j]), acc);
    acc = dot2_bf16(hi, bits_to_bf16x2(xw[2 * j + 1]), acc);
  }
  return acc;
}

// The pair's token and expert (or the shared expert); false for an unknown expert id or
// an expert that is not resident (slot map entry < 0).
__device__ __forceinline__ bool fp8_pair(int p, int tokens, int k, const int32_t* __restrict__ indices,
                                         const wm_fp8_experts& routed, bool has_shared, const wm_fp8_experts& shared,
                                         int& t, Fp8Regions& r, bool& is_shared) {
  bool resident;
  is_shared = p >= tokens * k;
  if (!is_shared) {
    t = p / k;
    const int e = indices[p];
    if (e < 0 || e >= routed.experts) return false;
    r = fp8_regions(routed, e, resident);
    return resident;
  }
  t = p - tokens * k;
  if (!has_shared) return false;
  r = fp8_regions(shared, 0, resident);
  return resident;
}

// The block's (row block x, pair or token p). One token: a 2-D grid (X, P), the row blocks
// of a pair in launch order. Several tokens: a 1-D grid of X * P blocks in which the P blocks
// of one row block lie 8 apart (block b runs on XCD b % 8), so they run on one XCD at about
// the same time and its L2 serves the rows they share: the shared expert's, read once per
// token, and any routed expert two tokens picked (C5 verify 1.24-1.26 ms against 1.31 ms;
// one token keeps the row-block order, whose reads each XCD spreads over fewer experts).
// X is a multiple of 8 (widths are multiples of 128).
__device__ __forceinline__ void block_order(int X, int P, bool interleave, int& x, int& p) {
  if (!interleave) {
    x = blockIdx.x;
    p = blockIdx.y;
    return;
  }
  const int b = blockIdx.x, lo = b % 8, q = b / 8;
  p = q % P;
  x = 8 * (q / P) + lo;
}

constexpr int FP8_RPW = 2;  // intermediate rows per wave (4 weight rows: gate and up of each)

// The block scale of the 16 columns [c, c + 16) of row `row` in a matrix of `cols` columns:
// SF 0, fp32 128 x 128 blocks; SF 1, E8M0 32 x 32 blocks (2^(b - 127)).
template <int SF>
__device__ __forceinline__ uint32_t fp8_block_scale_raw(const uint8_t* scales, int row, int cols, int c) {
  if constexpr (SF == 0)
    return gload<uint32_t>(reinterpret_cast<const uint32_t*>(scales) + (int64_t)(row / 128) * (cols / 128) + c / 128);
  else
    return gload<uint8_t>(scales + (int64_t)(row / 32) * (cols / 32) + c / 32);
}
// The scale value of a raw load, converted where it is used (a conversion next to the load
// would make the lane wait for it before issuing the loads after it).
template <int SF>
__device__ __forceinline__ float fp8_scale_value(uint32_t raw) {
  if constexpr (SF == 0)
    return __uint_as_float(raw);
  else
    return e8m0_value(raw);
}

// grid: (I / (4 * FP8_RPW), pairs), one 1-D grid of as many blocks with several tokens
// (block_order). CPL = ceil(H / 1024) chunks of 16 bytes per lane per row;
// SF the scale format.
template <int CPL, int SF>
__global__ void __launch_bounds__(256) fp8_gate_up_act_kernel(const uint16_t* __restrict__ x, int tokens, int k,
                                                              const int32_t* __restrict__ indices,
                                                              wm_fp8_experts routed, wm_fp8_experts shared,
                                                              int has_shared, uint16_t* __restrict__ act) {
  constexpr int ROWS = 2 * FP8_RPW;
  __shared__ float sums[4][ROWS];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int H = routed.hidden, I = routed.inter;
  int bx, p;
  block_order(I / (4 * FP8_RPW), tokens * k + (has_shared ? tokens : 0), tokens > 1, bx, p);
  int t;
  Fp8Regions r;
  bool is_shared;
  if (!fp8_pair(p, tokens, k, indices, routed, has_shared != 0, shared, t, r, is_shared)) {
    // unknown or non-resident expert: its act rows are zero and the down kernels skip the pair
    for (int i = bx * 4 * FP8_RPW + threadIdx.x; i < (bx + 1) * 4 * FP8_RPW; i += 256)
      act[(int64_t)p * I + i] = 0;
    return;
  }
  const wm_fp8_experts& tab = is_shared ? shared : routed;
  const int up_first = tab.up_first;
  const float limit = tab.swiglu_limit;
  const int i_base = bx * 4 * FP8_RPW + wave * FP8_RPW;

  // Every load is issued unconditionally (lanes past a row's end read its first chunk) and
  // masked where it is used, through the chunk's scale: a load under a condition makes the
  // compiler wait for it where the branches join, before the loads after it are issued.
  uint32_t xw[CPL][8];  // x[1024 m + 16 lane .. +15] as bf16 pairs
  float inm[CPL];       // 1 for chunks inside the row, 0 past its end
  const uint16_t* xr = x + (int64_t)t * H;
#pragma unroll
  for (int m = 0; m < CPL; ++m) {
    const int off = 1024 * m + 16 * lane;
    inm[m] = off < H ? 1.0f : 0.0f;
    const uint4* src = reinterpret_cast<const uint4*>(xr + (off < H ? off : 0));
    const uint4 a = src[0], b = src[1];
    xw[m][0] = a.x; xw[m][1] = a.y; xw[m][2] = a.z; xw[m][3] = a.w;
    xw[m][4] = b.x; xw[m][5] = b.y; xw[m][6] = b.z; xw[m][7] = b.w;
  }
  // a wave's FP8_RPW gate rows lie in one scale block (128 or 32 rows), and so do its up rows
  static_assert(32 % (4 * FP8_RPW) == 0, "a workgroup's rows lie in one scale block");
  uint4 wq[ROWS][CPL];
  uint32_t sc[2][CPL];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = (h ^ up_first) ? I + i_base : i_base;  // h 0: gate, 1: up
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int off = 1024 * m + 16 * lane;
      sc[h][m] = fp8_block_scale_raw<SF>(r.w13_scales, row, H, off < H ? off : 0);
    }
  }
#pragma unroll
  for (int q = 0; q < ROWS; ++q) {
    const int i = i_base + q / 2;  // I is a multiple of 8: always in range
    const int row = ((q & 1) ^ up_first) ? I + i : i;  // q even: gate, odd: up
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int off = 1024 * m + 16 * lane;
      wq[q][m] = gload16_nt(r.w13 + (int64_t)row * H + (off < H ? off : 0));
    }
  }
  float scv[2][CPL];  // the scales' values, masked (every load above is issued by now)
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int m = 0; m < CPL; ++m) scv[h][m] = fp8_scale_value<SF>(sc[h][m]) * inm[m];
#pragma unroll
  for (int q = 0; q < ROWS; ++q) {
    float acc = 0.0f;
#pragma unroll
    for (int m = 0; m < CPL; ++m) acc = fmaf(scv[q & 1][m], e4m3x16_dot_bf16(wq[q][m], xw[m], 0.0f), acc);
    acc = segment_sum<64>(acc);
    if (lane == 0) sums[wave][q] = acc;
  }
  // sums[wave] is written and read by this wave only (LDS operations of a wave are ordered)
  if (lane < FP8_RPW) {
    float g = sums[wave][2 * lane], u = sums[wave][2 * lane + 1];
    if (limit > 0.0f) {
      g = fminf(g, limit);
      u = fminf(fmaxf(u, -limit), limit);
    }
    act[(int64_t)p * I + i_base + lane] = f32_to_bf16_bits(silu(g) * u);
  }
}

constexpr int FP8_OPW = 8;  // output rows per wave step

// grid: combine (H / FP8_OPW, tokens), one 1-D grid of as many blocks with several tokens
// (block_order); per pair (H / (4 * FP8_OPW), pairs). CPL = ceil(I / 1024).
template <int CPL, int SF, bool COMBINE>
__global__ void __launch_bounds__(256) fp8_down_kernel(const uint16_t* __restrict__ act, int tokens, int k,
                                                       const int32_t* __restrict__ indices,
                                                       const float* __restrict__ weights, wm_fp8_experts routed,
                                                       wm_fp8_experts shared, int has_shared,
                                                       const uint16_t* __restrict__ x,
                                                       const uint16_t* __restrict__ shared_gate,
                                                       uint16_t* __restrict__ y) {
  __shared__ float partial[4][FP8_OPW];
  __shared__ float gate_value;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int H = routed.hidden, I = routed.inter;
  int t, o_base, first, step, n_entries;
  if (COMBINE) {
    int bx;
    block_order(H / FP8_OPW, tokens, tokens > 1, bx, t);
    o_base = bx * FP8_OPW;
    n_entries = k + (has_shared ? 1 : 0);
    first = wave;
    step = 4;
  } else {
    t = blockIdx.y;  // the pair
    o_base = (blockIdx.x * 4 + wave) * FP8_OPW;
    n_entries = 1;
    first = 0;
    step = 1;
  }
  if (COMBINE && has_shared) {
    if (threadIdx.x < 64) {
      float gv = 1.0f;
      if (shared_gate) {
        const uint32_t* xr = reinterpret_cast<const uint32_t*>(x) + (int64_t)t * (H / 2);
        const uint32_t* gr = reinterpret_cast<const uint32_t*>(shared_gate);
        float a = 0.0f;
        for (int q = lane; q < H / 2; q += 64) a = dot2_bf16(bits_to_bf16x2(xr[q]), bits_to_bf16x2(gr[q]), a);
        a = segment_sum<64>(a);
        gv = 1.0f / (1.0f + __expf(-a));
      }
      if (lane == 0) gate_value = gv;
    }
    __syncthreads();
  }
  float acc[FP8_OPW];
#pragma unroll
  for (int q = 0; q < FP8_OPW; ++q) acc[q] = 0.0f;
  for (int entry = first; entry < n_entries; entry += step) {
    int p;
    float w;
    Fp8Regions r;
    bool resident;
    if (COMBINE) {
      if (entry < k) {
        p = t * k + entry;
        const int e = indices[p];
        if (e < 0 || e >= routed.experts) continue;
        r = fp8_regions(routed, e, resident);
        w = weights[p];
      } else {
        p = tokens * k + t;
        r = fp8_regions(shared, 0, resident);
        w = gate_value;
      }
      if (!resident) continue;  // a non-resident expert contributes nothing
    } else {
      p = t;
      const int e = indices[p];
      if (e < 0) return;  // a masked pair: its output row is left as it is (uniform per block)
      if (e >= routed.experts) break;  // zero row
      r = fp8_regions(routed, e, resident);
      if (!resident) break;  // zero row
      w = 1.0f;
    }
    // loads unconditional (lanes past the row read its first chunk), masked through the scale
    uint32_t av[CPL][8];
    float inm[CPL];
    const uint16_t* arow = act + (int64_t)p * I;
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int off = 1024 * m + 16 * lane;
      inm[m] = off < I ? 1.0f : 0.0f;
      const uint4* a4 = reinterpret_cast<const uint4*>(arow + (off < I ? off : 0));
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const uint4 v = a4[q];
        av[m][4 * q] = v.x; av[m][4 * q + 1] = v.y; av[m][4 * q + 2] = v.z; av[m][4 * q + 3] = v.w;
      }
    }
    // the step's FP8_OPW rows start at a multiple of FP8_OPW, so they share one scale block
    // (128 or 32 rows): one scale load per 1024-wide chunk
    static_assert(32 % FP8_OPW == 0, "a step's rows lie in one scale block");
    uint4 wq[FP8_OPW][CPL];
    uint32_t sc[CPL];
#pragma unroll
    for (int m = 0; m < CPL; ++m) {
      const int off = 1024 * m + 16 * lane;
      sc[m] = fp8_block_scale_raw<SF>(r.w2_scales, o_base, I, off < I ? off : 0);
    }
#pragma unroll
    for (int q = 0; q < FP8_OPW; ++q) {
      const int o = o_base + q;  // H is a multiple of 32: always in range
#pragma unroll
      for (int m = 0; m < CPL; ++m) {
        const int off = 1024 * m + 16 * lane;
        wq[q][m] = gload16_nt(r.w2 + (int64_t)o * I + (off < I ? off : 0));
      }
    }
    float scv[CPL];  // the scales' values, masked (every load above is issued by now)
#pragma unroll
    for (int m = 0; m < CPL; ++m) scv[m] = fp8_scale_value<SF>(sc[m]) * inm[m];
#pragma unroll
    for (int q = 0; q < FP8_OPW; ++q) {
      float s = 0.0f;
#pragma unroll
      for (int m = 0; m < CPL; ++m) s = fmaf(scv[m], e4m3x16_dot_bf16(wq[q][m], av[m], 0.0f), s);
      acc[q] = fmaf(w, s, acc[q]);
    }
  }
#pragma unroll
  for (int q = 0; q < FP8_OPW; ++q) {
    const float v = segment_sum<64>(acc[q]);
    if (lane == 0) partial[wave][q] = v;
  }
  __syncthreads();
  if (COMBINE) {
    if (threadIdx.x < FP8_OPW) {
      const int q = threadIdx.x;
      const float v = (partial[0][q] + partial[1][q]) + (partial[2][q] + partial[3][q]);
      y[(int64_t)t * H + o_base + q] = f32_to_bf16_bits(v);
    }
  } else {
    if (lane < FP8_OPW) y[(int64_t)t * H + o_base + lane] = f32_to_bf16_bits(partial[wave][lane]);
  }
}

template <int SF>
static void launch_decode_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                              const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                              uint16_t* y, bool combine, uint16_t* act, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  const int pairs = tokens * k + (shared ? tokens : 0);
  const wm_fp8_experts sh = shared ? *shared : routed;
  const dim3 g1 = tokens > 1 ? dim3(I / (4 * FP8_RPW) * pairs) : dim3(I / (4 * FP8_RPW), pairs);
  switch ((H + 1023) / 1024) {
#define WM_F8GU(C) case C: hipLaunchKernelGGL((fp8_gate_up_act_kernel<C, SF>), g1, dim3(256), 0, s, x, tokens, k, \
                                              indices, routed, sh, shared ? 1 : 0, act); break;
    WM_F8GU(1) WM_F8GU(2) WM_F8GU(3) WM_F8GU(4) WM_F8GU(5) WM_F8GU(6) WM_F8GU(7) WM_F8GU(8)
#undef WM_F8GU
  }
  check_launch("fp8_gate_up_act");
  if (combine) {
    const dim3 g2 = tokens > 1 ? dim3(H / FP8_OPW * tokens) : dim3(H / FP8_OPW, tokens);
    switch ((I + 1023) / 1024) {
#define WM_F8DN(C) case C: hipLaunchKernelGGL((fp8_down_kernel<C, SF, true>), g2, dim3(256), 0, s, act, tokens, k, \
                                              indices, weights, routed, sh, shared ? 1 : 0, x, shared_gate, y); break;
      WM_F8DN(1) WM_F8DN(2) WM_F8DN(3) WM_F8DN(4) WM_F8DN(5) WM_F8DN(6) WM_F8DN(7) WM_F8DN(8)
#undef WM_F8DN
    }
  } else {
    const dim3 g2(H / (4 * FP8_OPW), tokens * k);
    switch ((I + 1023) / 1024) {
#define WM_F8DP(C) case C: hipLaunchKernelGGL((fp8_down_kernel<C, SF, false>), g2, dim3(256), 0, s, act, tokens, k, \
                                              indices, weights, routed, sh, 0, x, nullptr, y); break;
      WM_F8DP(1) WM_F8DP(2) WM_F8DP(3) WM_F8DP(4) WM_F8DP(5) WM_F8DP(6) WM_F8DP(7) WM_F8DP(8)
#undef WM_F8DP
    }
  }
  check_launch("fp8_down");
}

void decode_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                uint16_t* y, bool combine, uint16_t* act, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  if (H % 128 || I % 128 || H > 8192 || I > 8192)
    fail("FP8 decode: hidden and intermediate must be multiples of 128 up to 8192");
  if (routed.scale_format == 1)
    launch_decode_fp8<1>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, act, s);
  else
    launch_decode_fp8<0>(x, tokens, indices, weights, k, routed, shared, shared_gate, y, combine, act, s);
}

}  // namespace wm
