// Decode-time MXFP4 expert FFN: fused dequant + GEMV, HBM-bound.
//
// Replaces the reference's expert_linear4 + expert_act_pairs + expert_linear4 +
// moe_combine dispatch chain (Native/QwenNative/kernels.metal:1190-1220,
// :1333-1339, :185-194; driven from engine.mm:2198-2235) with two kernels:
//
//   gate_up_act : one workgroup = (pair, block of intermediate rows i). Each wave
//                 streams the gate row i and the up row I+i of its expert; a row of
//                 H/2 bytes is read by LPR lanes, 16 bytes (one 32-value E8M0
//                 group) per lane per load, GPL loads a lane, so a wave load is up to
//                 64 x 16 B, coalesced. Nibbles -> bf16 with the gfx950 scaled convert
//                 (scale folded in), dot2 against the bf16 input held in registers,
//                 segment reduction, then silu(gate) * up in the epilogue -> act (fp32).

//   down_combine: one workgroup = (token, block of output rows o). The four waves
//                 split the token's experts (routed + shared); each lane keeps its
//                 partial sums already scaled by the routing weight, so the
//                 cross-lane and cross-wave reductions happen once per output row:
//                 y[t,o] = sum_k w[t,k] * act_k . Wd_k[o] + gate(t) * act_s . Wd_s[o].
//                 The same kernel in per-pair mode writes each pair's row unweighted
//                 (the StreamingExperts [T, K, H] contract, qwen4_exp.py:853-904).
//
// Any hidden and intermediate size that is a multiple of 32 up to 16384 runs here (the
// reference's expert_linear4 takes any multiple of 32): a row of G = size / 32 groups is
// read by LPR lanes (a power of two) taking GPL groups each, LPR * GPL >= G, and the lanes
// past the row's last group load nothing and add nothing (lane_split).
#include <cmath>

#include "wm_common.h"
#include "moe_internal.h"

namespace wm {

// ---------------------------------------------------------------------------------
// The input row of a decode token as bf16 pairs: lane group `g` needs values
// [32 g, 32 g + 32) = 16 words; groups at or past `groups` (the row's end) read group 0.
// Every load in these kernels is issued unconditionally at an in-bounds address and its
// value masked where it is used (a scale of 0 for groups past a row's end): a load under a
// condition makes the compiler wait for it where the branches join, before the loads after
// it are issued.
template <int GPL, int LPR>
__device__ __forceinline__ void load_x_groups(const uint32_t* __restrict__ xrow, int gl, int groups,
                                              uint32_t (&xw)[GPL][16]) {
#pragma unroll
  for (int gp = 0; gp < GPL; ++gp) {
    const int g = gl + gp * LPR;
    const uint4* src = reinterpret_cast<const uint4*>(xrow + (g < groups ? g : 0) * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint4 v = src[q];
      xw[gp][4 * q + 0] = v.x;
      xw[gp][4 * q + 1] = v.y;
      xw[gp][4 * q + 2] = v.z;
      xw[gp][4 * q + 3] = v.w;
    }
  }
}

// Weight rows a gate_up wave reduces per pass (gate and up rows of RPW = ROWS / 2
// intermediate indices): one per lane slot when a wave load covers 8 or more rows,
// otherwise 8, fewer for wide rows so that x (16 GPL registers) and the row loads in
// flight (5 GPL registers per row step) stay within the register file.
__host__ __device__ constexpr int gate_up_rows(int lpr, int gpl) {
  return 64 / lpr >= 8 ? 64 / lpr : (64 / lpr >= 2 ? 8 : (gpl <= 3 ? 8 : gpl == 4 ? 6 : gpl == 5 ? 4 : 2));
}

// dot of one 32-value group: 16 weight bytes (4 words) against 16 bf16-pair words.
__device__ __forceinline__ float group_dot_bf16(uint4 w, float scale, const uint32_t (&xw)[16], float acc) {
  uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    wm_bf16x2 wv[4];
    fp4x8_to_bf16(words[j], scale, wv);
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = dot2_bf16(wv[m], bits_to_bf16x2(xw[4 * j + m]), acc);
  }
  return acc;
}

// One pair of the decode list: its token row and expert (or the shared expert); false
// for an id outside the table or an expert that is not resident (slot map entry < 0).
__device__ __forceinline__ bool decode_pair(int p, int tokens, int k, const int32_t* __restrict__ indices,
                                            const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared_opt,
                                            const wm_mxfp4_experts& shared, int& t, ExpertRegions& r) {
  bool resident;
  if (p < tokens * k) {
    t = p / k;
    int e = indices[p];
    if (e < 0 || e >= routed.experts) return false;
    r = expert_regions(routed, e, resident);
    return resident;
  }
  t = p - tokens * k;
  if (!shared_opt) return false;
  r = expert_regions(shared, 0, resident);
  return resident;
}

// grid: (ceil(I / (4 * RPW)), pairs), RPW = gate_up_rows(LPR, GPL) / 2. act[p, i] fp32.
template <int LPR, int GPL>
__global__ void __launch_bounds__(256) gate_up_act_kernel(const uint16_t* __restrict__ x, int tokens, int k,
                                                          const int32_t* __restrict__ indices, wm_mxfp4_experts routed,
                                                          wm_mxfp4_experts shared, int has_shared,
                                                          float* __restrict__ act) {
  constexpr int NS = 64 / LPR;              // rows a wave reads at once
  constexpr int ROWS = gate_up_rows(LPR, GPL);  // gate and up rows of RPW intermediate indices
  constexpr int RPW = ROWS / 2;
  constexpr int STEPS = (ROWS + NS - 1) / NS;
  __shared__ float sums[4][ROWS];
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int slot = lane / LPR, gl = lane % LPR;
  const int p = blockIdx.y;
  const int H = routed.hidden, I = routed.inter;
  int t;
  ExpertRegions r;
  if (!decode_pair(p, tokens, k, indices, routed, has_shared ? &shared : nullptr, shared, t, r)) {
    // Unknown or non-resident expert: its act row is zero and the down kernels skip the pair.
    for (int i = blockIdx.x * 4 * RPW + threadIdx.x; i < min(I, (int)(blockIdx.x + 1) * 4 * RPW); i += 256)
      act[(int64_t)p * I + i] = 0.0f;
    return;
  }
  const int up_first = has_shared && p >= tokens * k ? shared.up_first : routed.up_first;
  const float limit = has_shared && p >= tokens * k ? shared.swiglu_limit : routed.swiglu_limit;
  const int i_base = blockIdx.x * 4 * RPW + wave * RPW;

  const int G = H / 32;
  uint32_t xw[GPL][16];
  load_x_groups<GPL, LPR>(reinterpret_cast<const uint32_t*>(x) + (int64_t)t * (H / 2), gl, G, xw);

  uint4 wq[STEPS][GPL];
  uint32_t sb[STEPS][GPL];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    int q = st * NS + slot;
    int i = i_base + q / 2;
    bool ok = q < ROWS && i < I;
    // q even: gate row, q odd: up row (their order in the blob follows up_first).
    int row = ((q & 1) ^ up_first) ? I + i : i;
#pragma unroll
    for (int gp = 0; gp < GPL; ++gp) {
      const int g = gl + gp * LPR;
      const int rc = ok ? row : 0, gc = g < G ? g : 0;
      wq[st][gp] = gload16(r.gate_up + (int64_t)rc * (H / 2) + 16 * gc);
      sb[st][gp] = gload<uint8_t>(r.gate_up_scales + (int64_t)rc * G + gc);
    }
  }
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    const int q = st * NS + slot;
    const bool ok = q < ROWS && i_base + q / 2 < I;
    float acc = 0.0f;
#pragma unroll
    for (int gp = 0; gp < GPL; ++gp) {
      const bool valid = ok && gl + gp * LPR < G;
      acc = group_dot_bf16(wq[st][gp], valid ? e8m0_scale_operand(sb[st][gp]) : 0.0f, xw[gp], acc);
    }
    acc = segment_sum<LPR>(acc);
    if (gl == 0 && q < ROWS) sums[wave][q] = acc;
  }
  __syncthreads();
  if (lane < RPW) {
    int i = i_base + lane;
    if (i < I) {
      float g = sums[wave][2 * lane], u = sums[wave][2 * lane + 1];
      if (limit > 0.0f) {
        g = fminf(g, limit);
        u = fminf(fmaxf(u, -limit), limit);
      }
      act[(int64_t)p * I + i] = silu(g) * u;
    }
  }
}

// grid: combine mode (ceil(H / (NS * STEPS)), tokens); per-pair mode (ceil(H / (4 * NS * STEPS)), pairs).
// In combine mode the four waves split the token's experts; in per-pair mode they split the rows.
template <int LPR, int GPL, int STEPS, bool COMBINE>
__global__ void __launch_bounds__(256) down_kernel(const float* __restrict__ act, int tokens, int k,
                                                   const int32_t* __restrict__ indices,
                                                   const float* __restrict__ weights, wm_mxfp4_experts routed,
                                                   wm_mxfp4_experts shared, int has_shared,
                                                   const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ shared_gate,
                                                   uint16_t* __restrict__ y) {
  constexpr int NS = 64 / LPR;
  constexpr int OPW = NS * STEPS;           // output rows per wave
  __shared__ float partial[4][OPW];
  __shared__ float gate_value;
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int slot = lane / LPR, gl = lane % LPR;
  const int H = routed.hidden, I = routed.inter;
  const int G = I / 32;

  int o_base, first_entry, entry_step, n_entries, t;
  if (COMBINE) {
    t = blockIdx.y;
    o_base = blockIdx.x * OPW;
    n_entries = k + (has_shared ? 1 : 0);
    first_entry = wave;
    entry_step = 4;
  } else {
    t = blockIdx.y;  // the pair
    o_base = (blockIdx.x * 4 + wave) * OPW;
    n_entries = 1;
    first_entry = 0;
    entry_step = 1;
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

  float acc[STEPS];
#pragma unroll
  for (int st = 0; st < STEPS; ++st) acc[st] = 0.0f;

  for (int entry = first_entry; entry < n_entries; entry += entry_step) {
    int p;          // act row
    float w;        // weight of this expert's output
    ExpertRegions r;
    bool resident;
    if (COMBINE) {
      if (entry < k) {
        p = t * k + entry;
        int e = indices[p];
        if (e < 0 || e >= routed.experts) continue;
        r = expert_regions(routed, e, resident);
        w = weights[p];
      } else {
        p = tokens * k + t;
        r = expert_regions(shared, 0, resident);
        w = gate_value;
      }
      if (!resident) continue;  // a non-resident expert contributes nothing
    } else {
      p = t;
      if (p < tokens * k) {
        int e = indices[p];
        if (e < 0) return;  // a masked pair: its output row is left as it is (uniform per block)
        if (e >= routed.experts) break;  // zero row
        r = expert_regions(routed, e, resident);
      } else {
        r = expert_regions(shared, 0, resident);
      }
      if (!resident) break;  // zero row
      w = 1.0f;
    }
    // act values of this lane's groups: 32 floats per group.
    const float* arow = act + (int64_t)p * I;
    uint4 wq[STEPS][GPL];
    uint32_t sb[STEPS][GPL];
#pragma unroll
    for (int st = 0; st < STEPS; ++st) {
      int o = o_base + st * NS + slot;
#pragma unroll
      for (int gp = 0; gp < GPL; ++gp) {
        const int g = gl + gp * LPR;
        const int oc = o < H ? o : 0, gc = g < G ? g : 0;
        wq[st][gp] = gload16(r.down + (int64_t)oc * (I / 2) + 16 * gc);
        sb[st][gp] = gload<uint8_t>(r.down_scales + (int64_t)oc * G + gc);
      }
    }
#pragma unroll
    for (int gp = 0; gp < GPL; ++gp) {
      const int g = gl + gp * LPR;
      const float4* a4 = reinterpret_cast<const float4*>(arow + (g < G ? g : 0) * 32);
      float av[32];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        float4 v = a4[q];
        av[4 * q] = v.x; av[4 * q + 1] = v.y; av[4 * q + 2] = v.z; av[4 * q + 3] = v.w;
      }
#pragma unroll
      for (int st = 0; st < STEPS; ++st) {
        const bool valid = o_base + st * NS + slot < H && g < G;
        float scale = valid ? e8m0_scale_operand(sb[st][gp]) : 0.0f;
        uint32_t words[4] = {wq[st][gp].x, wq[st][gp].y, wq[st][gp].z, wq[st][gp].w};
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            wm_f32x2 wf;
            switch (b) {
              case 0: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[j], scale, 0); break;
              case 1: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[j], scale, 1); break;
              case 2: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[j], scale, 2); break;
              default: wf = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(words[j], scale, 3); break;
            }
            s = fmaf(wf[0], av[8 * j + 2 * b], s);
            s = fmaf(wf[1], av[8 * j + 2 * b + 1], s);
          }
        }
        acc[st] = fmaf(w, s, acc[st]);
      }
    }
  }
#pragma unroll
  for (int st = 0; st < STEPS; ++st) {
    float v = segment_sum<LPR>(acc[st]);
    if (gl == 0) partial[wave][st * NS + slot] = v;
  }
  __syncthreads();
  if (COMBINE) {
    if (threadIdx.x < OPW) {
      int o = o_base + threadIdx.x;
      if (o < H) {
        float v = partial[0][threadIdx.x] + partial[1][threadIdx.x] + partial[2][threadIdx.x] + partial[3][threadIdx.x];
        y[(int64_t)t * H + o] = f32_to_bf16_bits(v);
      }
    }
  } else {
    if (lane < OPW) {
      int o = o_base + lane;
      if (o < H) y[(int64_t)t * H + o] = f32_to_bf16_bits(partial[wave][lane]);
    }
  }
}

// ---------------------------------------------------------------------------------
// Launchers. A row of G groups is read by LPR lanes x GPL groups (lane_split).

// Every (LPR, GPL) lane_split can choose.
#define WM_LANE_SPLITS(X)                                                                          \
  X(4, 1) X(4, 3) X(4, 5) X(8, 1) X(8, 3) X(8, 5) X(16, 1) X(16, 3) X(16, 5) X(32, 1) X(32, 3) X(32, 5) \
  X(64, 1) X(64, 2) X(64, 3) X(64, 4) X(64, 5) X(64, 6) X(64, 7) X(64, 8)

// Lanes per row and groups per lane for rows of `dim` values (a multiple of 32): the split
// with the fewest idle lane groups, ties to the wider one (fewer loads per lane). False
// above 16384 values (512 groups).
static bool lane_split(int dim, int& lpr, int& gpl) {
  const int G = dim / 32;
  int best_waste = 1 << 30;
  lpr = gpl = 0;
#define WM_TRY(L, P)                                                  \
  if (L * P >= G && (L * P - G < best_waste || (L * P - G == best_waste && L > lpr))) { \
    best_waste = L * P - G;                                           \
    lpr = L;                                                          \
    gpl = P;                                                          \
  }
  WM_LANE_SPLITS(WM_TRY)
#undef WM_TRY
  return lpr > 0;
}

static void launch_gate_up(int lpr, int gpl, int pairs, int inter, hipStream_t s, const uint16_t* x, int tokens, int k,
                           const int32_t* indices, const wm_mxfp4_experts& routed, const wm_mxfp4_experts& shared,
                           int has_shared, float* act) {
#define WM_GU(L, G)                                                                                            \
  if (lpr == L && gpl == G) {                                                                                   \
    constexpr int RPW = gate_up_rows(L, G) / 2;                                                                 \
    hipLaunchKernelGGL((gate_up_act_kernel<L, G>), dim3((inter + 4 * RPW - 1) / (4 * RPW), pairs), dim3(256), 0, s, \
                       x, tokens, k, indices, routed, shared, has_shared, act);                                  \
    return;                                                                                                     \
  }
  WM_LANE_SPLITS(WM_GU)
#undef WM_GU
  fail("decode gate_up: unsupported hidden size");
}

template <int STEPS, bool COMBINE>
static void launch_down(int lpr, int gpl, dim3 grid, hipStream_t s, const float* act, int tokens, int k,
                        const int32_t* indices, const float* weights, const wm_mxfp4_experts& routed,
                        const wm_mxfp4_experts& shared, int has_shared, const uint16_t* x, const uint16_t* sg,
                        uint16_t* y) {
#define WM_DN(L, G)                                                                                            \
  if (lpr == L && gpl == G) {                                                                                   \
    hipLaunchKernelGGL((down_kernel<L, G, STEPS, COMBINE>), grid, dim3(256), 0, s, act, tokens, k, indices,     \
                       weights, routed, shared, has_shared, x, sg, y);                                          \
    return;                                                                                                     \
  }
  WM_LANE_SPLITS(WM_DN)
#undef WM_DN
  fail("decode down: unsupported intermediate size");
}

bool decode_mxfp4_supports(int hidden, int inter) {
  int l, g;
  return hidden % 32 == 0 && inter % 32 == 0 && lane_split(hidden, l, g) && lane_split(inter, l, g);
}

void decode_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                  const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                  uint16_t* y, bool combine, float* act, hipStream_t s) {
  const int H = routed.hidden, I = routed.inter;
  const int pairs = tokens * k + (shared ? tokens : 0);
  wm_mxfp4_experts sh = shared ? *shared : routed;
  int lpr_h, gpl_h, lpr_i, gpl_i;
  if (!lane_split(H, lpr_h, gpl_h) || !lane_split(I, lpr_i, gpl_i))
    fail("decode: hidden and intermediate must be at most 16384");
  launch_gate_up(lpr_h, gpl_h, pairs, I, s, x, tokens, k, indices, routed, sh, shared ? 1 : 0, act);
  check_launch("gate_up_act");
  constexpr int STEPS = 2;
  int opw = (64 / lpr_i) * STEPS;
  if (combine) {
    dim3 g2((H + opw - 1) / opw, tokens);
    launch_down<STEPS, true>(lpr_i, gpl_i, g2, s, act, tokens, k, indices, weights, routed, sh, shared ? 1 : 0, x,
                             shared_gate, y);
  } else {
    dim3 g2((H + 4 * opw - 1) / (4 * opw), tokens * k);
    launch_down<STEPS, false>(lpr_i, gpl_i, g2, s, act, tokens, k, indices, weights, routed, sh, 0, x, nullptr, y);
  }
  check_launch("down");
}

}  // namespace wm
