// Wave-level top-k used by the router kernels and by the persistent decode kernel.
//
// One wave64 holds a row of up to 64 * PER_LANE scores: expert e in lane e % 64,
// register e / 64. Every per-lane array is indexed only with unrolled, compile-time
// indices, so the row stays in registers. Top-k is a radix select on order-preserving
// keys (k rounds of a wave arg-max when a lane holds one value), value descending and ties
// to the lower index (the rule fixed for this build; Native/DeepSeekNative/engine.mm:1881
// breaks ties the same way).
#pragma once

#include <cmath>

#include "wm_common.h"

namespace wm {

// ---- the router's score arithmetic, stated in fp32 operations --------------------------
// Each operation is rounded to nearest even and none is fused (contraction off), so the
// test oracle restates it op for op in numpy float32 (oracle/moe.py exp_f32, log1p_f32,
// score_f32) and both select the same experts:
//   exp:   n = rint(x log2e); r = (x - n ln2_hi) - n ln2_lo; p = degree-7 Taylor polynomial
//          of e^r by Horner; e^x = p 2^n, 0 when n < -125, +inf when n > 128;
//   log1p: u in [0, 1]: m = 1 + u, halved when above sqrt 2 (k = 1); s = (m - 1)/(m + 1);
//          ln m = k ln2 + 2 s (1 + z/3 + ... + z^5/11), z = s^2; plus (u - (m - 1)) / m.
// Division and square root are the correctly rounded IEEE operations.
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2Hi = 0.693145751953125f;  // 0x3F317200: n * kLn2Hi is exact for |n| <= 256
constexpr float kLn2Lo = (float)(0.6931471805599453 - 0.693145751953125);
constexpr float kSqrt2 = 1.4142135623730951f;

__device__ __forceinline__ float exp_defined(float x) {
#pragma clang fp contract(off)
  if (x != x) return x;
  const float n = __builtin_rintf(x * kLog2e);
  const float r = (x - n * kLn2Hi) - n * kLn2Lo;
  float p = (float)(1.0 / 5040.0);
  p = p * r + (float)(1.0 / 720.0);
  p = p * r + (float)(1.0 / 120.0);
  p = p * r + (float)(1.0 / 24.0);
  p = p * r + (float)(1.0 / 6.0);
  p = p * r + 0.5f;
  p = p * r + 1.0f;
  p = p * r + 1.0f;
  if (n > 128.0f) return __builtin_inff();
  if (n < -125.0f) return 0.0f;
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float log1p_defined(float u) {
#pragma clang fp contract(off)
  const float m = 1.0f + u;
  const bool k = m > kSqrt2;
  const float m2 = k ? m * 0.5f : m;
  const float s = (m2 - 1.0f) / (m2 + 1.0f);
  const float z = s * s;
  float p = (float)(1.0 / 11.0);
  p = p * z + (float)(1.0 / 9.0);
  p = p * z + (float)(1.0 / 7.0);
  p = p * z + (float)(1.0 / 5.0);
  p = p * z + (float)(1.0 / 3.0);
  p = p * z + 1.0f;
  const float lg = (s + s) * p;
  const float corr = (u - (m - 1.0f)) / m;
  const float kf = k ? 1.0f : 0.0f;
  return kf * kLn2Hi + (kf * kLn2Lo + (lg + corr));
}

__device__ __forceinline__ float sigmoid_defined(float l) {
#pragma clang fp contract(off)
  return 1.0f / (1.0f + exp_defined(-l));
}

// sqrt(softplus(l)); below l = -64, where softplus(l) = e^l to fp32 precision, e^(l/2).
__device__ __forceinline__ float sqrt_softplus_defined(float l) {
#pragma clang fp contract(off)
  if (l < -64.0f) return exp_defined(0.5f * l);
  return __builtin_sqrtf(fmaxf(l, 0.0f) + log1p_defined(exp_defined(-fabsf(l))));
}

__device__ __forceinline__ bool topk_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && i < bi);
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, false);
}

// Wave-wide arg-max of (v, i); every lane gets the winner. Inside each 16-lane row the
// candidates meet through DPP moves (pairs, quads, row halves mirrored, rows mirrored: after
// each step every lane holds the best of its group), then the four rows' winners are read
// into scalar registers and compared in row order. (value, index) is a strict total order
// for non-NaN values, so the winner does not depend on the order of the comparisons.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
  auto take = [&](float ov, int oi) {
    const bool t = (ov > v) | ((ov == v) & (oi < i));
    v = t ? ov : v;
    i = t ? oi : i;
  };
  take(dpp_f<0xB1>(v), dpp_i<0xB1>(i));    // quad_perm [1,0,3,2]
  take(dpp_f<0x4E>(v), dpp_i<0x4E>(i));    // quad_perm [2,3,0,1]
  take(dpp_f<0x141>(v), dpp_i<0x141>(i));  // row_half_mirror
  take(dpp_f<0x140>(v), dpp_i<0x140>(i));  // row_mirror
  float bv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  int bi = __builtin_amdgcn_readlane(i, 0);
#pragma unroll
  for (int row = 1; row < 4; ++row) {
    const float rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16 * row));
    const int ri = __builtin_amdgcn_readlane(i, 16 * row);
    if (topk_better(rv, ri, bv, bi)) { bv = rv; bi = ri; }
  }
  v = bv;
  i = bi;
}

// Order-preserving 32-bit key of a score: a larger value has a larger key, +0 and -0 share
// one (they compare equal), and NaN gets 0, below every number, so it is never selected.
__device__ __forceinline__ uint32_t topk_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (u == 0x80000000u) u = 0u;  // -0 -> +0 on the bits (no reliance on float semantics)
  const uint32_t key = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (u & 0x7fffffffu) > 0x7f800000u ? 0u : key;  // NaN -> 0
}
__device__ __forceinline__ float topk_value(uint32_t key) {
  return __uint_as_float((key & 0x80000000u) ? (key & 0x7fffffffu) : ~key);
}

// LDS a wave's top-k uses to put its selections in order (2 KB). One per wave that routes
// at a time.
//   cand[0, 64):    the candidates in expert order, each as a 64-bit composite (low word
//                   63 - position, high word the key): a larger composite is a better
//                   candidate (a larger key, or an equal key with a lower expert id);
//   cand[64, 128):  one spare slot per lane, which takes the stores of lanes with nothing to
//                   store (so no store needs a branch around it);
//   expert[]:       the candidates' expert ids, with the same spare slots;
//   sorted[]:       the selections in selection order, (key, expert); before that, the 64
//                   words of the threshold's rank pass.
struct TopkScratch {
  uint2 cand[128];
  uint32_t expert[128];
  uint2 sorted[64];
};

// Orders this wave's LDS accesses around it (lgkmcnt 0; no hardware barrier: one wave).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Wave-wide max / min; every lane gets the result (rows through DPP, then the four rows'
// results through scalar registers).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = max(v, (uint32_t)dpp_i<0xB1>((int)v));
  v = max(v, (uint32_t)dpp_i<0x4E>((int)v));
  v = max(v, (uint32_t)dpp_i<0x141>((int)v));
  v = max(v, (uint32_t)dpp_i<0x140>((int)v));
  const uint32_t a = max((uint32_t)__builtin_amdgcn_readlane((int)v, 0), (uint32_t)__builtin_amdgcn_readlane((int)v, 16));
  const uint32_t b = max((uint32_t)__builtin_amdgcn_readlane((int)v, 32), (uint32_t)__builtin_amdgcn_readlane((int)v, 48));
  return max(a, b);
}
__device__ __forceinline__ int wave_min_i32(int v) {
  v = min(v, dpp_i<0xB1>(v));
  v = min(v, dpp_i<0x4E>(v));
  v = min(v, dpp_i<0x141>(v));
  v = min(v, dpp_i<0x140>(v));
  return min(min(__builtin_amdgcn_readlane(v, 0), __builtin_amdgcn_readlane(v, 16)),
             min(__builtin_amdgcn_readlane(v, 32), __builtin_amdgcn_readlane(v, 48)));
}

// Top-k by k rounds of arg-max over vals (entries with e >= experts are ignored), for short
// selections (one value a lane: the group stage of the scored router). Lane j < k receives
// the j-th selection in (sel, sel_val); a round with nothing left to select gives
// (0x7fffffff, -inf). Each lane keeps its best remaining entry (the lowest register
// among equal keys, so the lowest expert id); a round takes the wave max of those keys, and
// only when several lanes hold it the lowest expert id among them. The winner's lane drops
// the entry and finds its next best. Values are compared as keys, so -0 and +0 tie and a
// selected zero is reported as +0.
template <int PER_LANE>
__device__ __forceinline__ void wave_topk_rounds(const float (&vals)[PER_LANE], int experts, int k, int lane,
                                                 int& sel, float& sel_val) {
  uint32_t key[PER_LANE];
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) key[r] = r * 64 + lane < experts ? topk_key(vals[r]) : 0u;
  uint32_t hk;
  int hr;
  auto best = [&]() {
    hk = key[0];
    hr = 0;
#pragma unroll
    for (int r = 1; r < PER_LANE; ++r) {  // strict: the lowest register wins a tie
      const bool t = key[r] > hk;
      hk = t ? key[r] : hk;
      hr = t ? r : hr;
    }
  };
  best();
  sel = -1;
  sel_val = -INFINITY;
  for (int j = 0; j < k; ++j) {
    const uint32_t m = wave_max_u32(hk);
    int ew = 0x7fffffff;
    float vw = -INFINITY;
    if (m != 0u) {
      const uint64_t tied = __builtin_amdgcn_ballot_w64(hk == m);
      if (__builtin_popcountll(tied) == 1) {
        const int wl = (int)__builtin_ctzll(tied);
        ew = __builtin_amdgcn_readlane(hr, wl) * 64 + wl;
      } else {
        ew = wave_min_i32(hk == m ? hr * 64 + lane : 0x7fffffff);
      }
      vw = topk_value(m);
      const bool win = lane == (ew & 63);
      const int rw = ew >> 6;
#pragma unroll
      for (int r = 0; r < PER_LANE; ++r) key[r] = (win & (r == rw)) ? 0u : key[r];
      best();
    }
    if (lane == j) {
      sel = ew;
      sel_val = vw;
    }
  }
}

// The largest t with #{key >= t} >= k over a wave's keys (the k-th largest key, or 0 when
// fewer than k keys are above 0): a radix walk from the most significant bit, one bit a
// round from ballot counts (a v_cmp and a scalar popcount per register, no cross-lane
// reduction). It stops early once #{key >= t} == k (`exact`: that set is the top k).
template <int N>
__device__ __forceinline__ uint32_t radix_kth_key(const uint32_t (&key)[N], int k, bool& exact) {
  uint32_t prefix = 0;
  exact = false;
  // kept rolled: the round is short, and an unrolled walk is ~30 cache lines of code
#pragma nounroll
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = prefix | (1u << bit);
    int c = 0;
#pragma unroll
    for (int r = 0; r < N; ++r) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[r] >= cand));
    if (c >= k) {
      prefix = cand;
      if (c == k) {
        exact = true;
        break;
      }
    }
  }
  return prefix;
}

// A lower bound T of the k-th largest of the wave's 64 keys (one a lane, 1 <= k <= 64)
// with at least k keys >= T: each lane ranks u = ((key >> 1) & ~63) | lane (31 bits, unique)
// against the 64 values read back from LDS in one pass of independent counts (o > u exactly
// when bit 31 of u - o is set, as both are below 2^31), and the lane of rank k - 1 gives
// T = its key with the low 7 bits cleared. 0 when fewer than k keys are nonzero (a nonzero
// key is at least 0x007fffff, the key of -inf). `lds` holds 64 words; the caller orders it
// against its other uses.
__device__ __forceinline__ uint32_t wave_kth_key_floor(uint32_t key, int k, int lane, uint32_t* lds) {
  const uint32_t u = ((key >> 1) & ~63u) | (uint32_t)lane;
  lds[lane] = u;
  wave_lds_sync();
  uint32_t a0 = 0, a1 = 0, a2 = 0, a3 = 0;  // values above u
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint4 o = reinterpret_cast<const uint4*>(lds)[j];
    a0 += (u - o.x) >> 31;
    a1 += (u - o.y) >> 31;
    a2 += (u - o.z) >> 31;
    a3 += (u - o.w) >> 31;
  }
  const uint64_t at = __builtin_amdgcn_ballot_w64((int)(a0 + a1 + a2 + a3) == k - 1);  // exactly one lane
  return ((uint32_t)__builtin_amdgcn_readlane((int)u, (int)__builtin_ctzll(at)) & ~63u) << 1;
}

// Top-k of vals (entries with e >= experts ignored; k <= 64), value descending and ties to
// the lower expert id. Lane j < k receives the j-th selection in (sel, sel_val); when fewer
// than k entries are selectable (NaN never is), the lanes past them get (0x7fffffff, -inf);
// lanes >= k get (-1, -inf). Values are compared as keys, so -0 and +0 tie and a selected
// zero is reported as +0.
//
// A prefilter first: a lower bound T of the k-th largest of the 64 per-lane maximum keys
// (wave_kth_key_floor) has at least k keys at or above it, so the top k are among the keys
// >= T, and the rank of such a key among them (the keys better than it: larger, or equal with
// a lower id) is its rank in the row. When there are at most 64 of them (T > 0), they are
// compacted into LDS in expert order, each ranks itself against the others in one pass of
// 64-bit composite compares, and the first k ranks are the selection. Otherwise (heavy ties,
// or fewer than k selectable keys) a radix walk over every key finds the k-th largest key K,
// and the selection is every key above K plus the lowest-id entries equal to K, ranked the
// same way. No store sits under a branch (lanes with nothing to store write a spare slot).
template <int PER_LANE>
__device__ __forceinline__ void wave_topk(const float (&vals)[PER_LANE], int experts, int k, int lane,
                                          TopkScratch& sc, int& sel, float& sel_val) {
  if constexpr (PER_LANE == 1) {  // a few values a wave: k rounds are the shorter chain
    wave_topk_rounds<1>(vals, experts, k, lane, sel, sel_val);
    return;
  }
  uint32_t key[PER_LANE];
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {
    uint32_t kk = topk_key(vals[r]);
    asm volatile("" : "+v"(kk));  // computed on every lane, not under a branch
    key[r] = r * 64 + lane < experts ? kk : 0u;
  }
  auto count_ge = [&](uint32_t t) {
    int c = 0;
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) c += __builtin_popcountll(__builtin_amdgcn_ballot_w64(key[r] >= t));
    return c;
  };
  bool take[PER_LANE];  // this lane's entry of register r is a candidate
  uint32_t lane_max = key[0];
#pragma unroll
  for (int r = 1; r < PER_LANE; ++r) lane_max = max(lane_max, key[r]);
  wave_lds_sync();  // a previous call's reads of sc are done
  const uint32_t t = wave_kth_key_floor(lane_max, k, lane, reinterpret_cast<uint32_t*>(sc.sorted));
  if (t != 0u && count_ge(t) <= 64) {
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) take[r] = key[r] >= t;
  } else {
    bool exact;
    const uint32_t kth = radix_kth_key<PER_LANE>(key, k, exact);
    if (exact || kth == 0u) {  // kth 0: fewer than k selectable keys, take them all
      const uint32_t lo = exact ? kth : 1u;
#pragma unroll
      for (int r = 0; r < PER_LANE; ++r) take[r] = key[r] >= lo;
    } else {
      int need = k - count_ge(kth + 1u);  // ties at K to take, lowest expert id first
#pragma unroll
      for (int r = 0; r < PER_LANE; ++r) {
        uint64_t eq = __builtin_amdgcn_ballot_w64(key[r] == kth);
        uint64_t low_ids = 0;
        for (; need > 0 && eq != 0; --need) {
          const uint64_t low = eq & (~eq + 1);
          low_ids |= low;
          eq ^= low;
        }
        take[r] = (key[r] > kth) | (((low_ids >> lane) & 1ull) != 0);
      }
    }
  }
  wave_lds_sync();
  int n = 0;  // candidates (at most 64)
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {
    const uint64_t m = __builtin_amdgcn_ballot_w64(take[r]);
    const int pos = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    const int slot = take[r] ? pos : 64 + lane;
    sc.cand[slot] = make_uint2(63u - (uint32_t)pos, key[r]);
    sc.expert[slot] = (uint32_t)(r * 64 + lane);
    n += __builtin_popcountll(m);
  }
  // zero composites after the last candidate, to the end of its batch of 16 (a zero is never
  // better than a candidate: a candidate's key is nonzero)
  sc.cand[lane < 16 && n + lane < 64 ? n + lane : 64 + lane] = make_uint2(0u, 0u);
  wave_lds_sync();
  const uint2 mine = sc.cand[lane];
  const uint64_t me = lane < n ? ((uint64_t)mine.y << 32 | mine.x) : ~0ull;
  const uint32_t me_expert = sc.expert[lane];
  int r0 = 0, r1 = 0;  // better candidates
  for (int i0 = 0; i0 < n; i0 += 16) {  // sixteen candidates a batch, all reads issued together
    uint4 o[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) o[q] = reinterpret_cast<const uint4*>(sc.cand)[i0 / 2 + q];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      r0 += (int)(((uint64_t)o[q].y << 32 | o[q].x) > me);
      r1 += (int)(((uint64_t)o[q].w << 32 | o[q].z) > me);
    }
  }
  const int rank = r0 + r1;
  wave_lds_sync();
  *(lane < n && rank < k ? &sc.sorted[rank] : &sc.cand[64 + lane]) = make_uint2((uint32_t)(me >> 32), me_expert);
  wave_lds_sync();
  const uint2 s2 = sc.sorted[lane];
  sel = lane < k ? (lane < n ? (int)s2.y : 0x7fffffff) : -1;
  sel_val = lane < k && lane < n ? topk_value(s2.x) : -INFINITY;
}

// Softmax routing of one row held in registers (vals, expert e in lane e % 64, register
// e / 64; entries past `experts` ignored) by one wave: lane j < k gets the j-th expert and its
// weight exp(l_j - l_max) / sum (kept logits when `norm`, else all); with `want_full`, `full`
// receives the sum over all logits.
template <int PER_LANE>
__device__ __forceinline__ void wave_route_softmax_vals(const float (&vals)[PER_LANE], int experts, int k, bool norm,
                                                        int lane, TopkScratch& sc, int& sel, float& weight,
                                                        bool want_full, float& full) {
  float sel_val;
  wave_topk<PER_LANE>(vals, experts, k, lane, sc, sel, sel_val);
  // the first selection (lane 0) is the row maximum
  float top = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sel_val), 0));
  float mine = lane < k ? __expf(sel_val - top) : 0.0f;
  float denom;
  full = 0.0f;
  if (!norm || want_full) {
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts) full += __expf(vals[r] - top);
    }
    full = segment_sum<64>(full);
  }
  denom = norm ? segment_sum<64>(mine) : full;
  weight = mine / denom;
}

// The same for a row in memory (`experts` long).
template <int PER_LANE>
__device__ __forceinline__ void wave_route_softmax(const float* __restrict__ row, int experts, int k, bool norm,
                                                   int lane, TopkScratch& sc, int& sel, float& weight,
                                                   bool want_full, float& full) {
  float vals[PER_LANE];
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {  // every load in bounds, so all are issued together
    const int e = r * 64 + lane;
    const float v = row[e < experts ? e : experts - 1];
    vals[r] = e < experts ? v : -INFINITY;
  }
  wave_route_softmax_vals<PER_LANE>(vals, experts, k, norm, lane, sc, sel, weight, want_full, full);
}

}  // namespace wm
