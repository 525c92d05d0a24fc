// Wave-level top-k used by the router kernels and by the persistent decode kernel.
//
// One wave64 holds a row of up to 64 * PER_LANE scores: expert e in lane e % 64,
// register e / 64. Every per-lane array is indexed only with unrolled, compile-time
// indices, so the row stays in registers. Top-k is k rounds of a wave-wide
// arg-max, value descending and ties to the lower index (the rule fixed for this
// build; Native/DeepSeekNative/engine.mm:1881 breaks ties the same way).
#pragma once

#include <cmath>

#include "wm_common.h"

namespace wm {

__device__ __forceinline__ bool topk_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

// Wave-wide arg-max of (v, i); every lane gets the winner.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#pragma unroll
  for (int offset = 32; offset > 0; offset >>= 1) {
    float ov = __shfl_xor(v, offset, 64);
    int oi = __shfl_xor(i, offset, 64);
    if (topk_better(ov, oi, v, i)) { v = ov; i = oi; }
  }
}

// k rounds of arg-max over vals (entries with e >= experts are ignored). Lane j < k
// receives the j-th selection in (sel, sel_val).
template <int PER_LANE>
__device__ __forceinline__ void wave_topk(const float (&vals)[PER_LANE], int experts, int k, int lane, int& sel,
                                          float& sel_val) {
  uint32_t taken = 0;
  sel = -1;
  sel_val = -INFINITY;
  for (int j = 0; j < k; ++j) {
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      bool free_ = e < experts && !((taken >> r) & 1u);
      if (free_ && topk_better(vals[r], e, bv, bi)) { bv = vals[r]; bi = e; }
    }
    wave_argmax(bv, bi);
    if (lane == j) { sel = bi; sel_val = bv; }
    if (bi < experts && (bi & 63) == lane) taken |= 1u << (bi >> 6);
  }
}

// Softmax routing of one row (logits, `experts` long) by one wave: lane j < k gets the
// j-th expert and its weight exp(l_j - l_max) / sum (kept logits when `norm`, else all).
template <int PER_LANE>
__device__ __forceinline__ void wave_route_softmax(const float* __restrict__ row, int experts, int k, bool norm,
                                                   int lane, int& sel, float& weight, float* full_denominator) {
  float vals[PER_LANE];
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {
    int e = r * 64 + lane;
    vals[r] = e < experts ? row[e] : -INFINITY;
  }
  float sel_val;
  wave_topk<PER_LANE>(vals, experts, k, lane, sel, sel_val);
  float top = __shfl(sel_val, 0, 64);  // the first selection is the row maximum
  float mine = lane < k ? __expf(sel_val - top) : 0.0f;
  float denom;
  float full = 0.0f;
  if (!norm || full_denominator) {
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts) full += __expf(vals[r] - top);
    }
    full = segment_sum<64>(full);
    if (full_denominator) *full_denominator = full;
  }
  denom = norm ? segment_sum<64>(mine) : full;
  weight = mine / denom;
}

}  // namespace wm
