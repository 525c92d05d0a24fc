// Router kernels: softmax top-k (Qwen), scored top-k with bias-select and
// group-limited selection (DeepSeek), and the bf16 router linear.
// One wave64 per token; the top-k rule and register layout are in route_device.h.
#include <cmath>

#include "route_device.h"

namespace wm {

bool linear_bf16_mfma(const void* x, const void* w, int tokens, int hidden, int outputs, float* out, hipStream_t s);

constexpr int ROUTE_MAX_K = 32;

// The router kernels run a wave per token, four tokens to a 256-thread block. At 16K tokens
// x 512 experts they are bound by VALU and scalar issue (k rounds of a per-lane scan and a
// wave arg-max), not by the 33.5 MB of logits.
template <int PER_LANE>
__global__ void __launch_bounds__(256) route_softmax_topk_kernel(const float* __restrict__ logits, int tokens,
                                                                int experts, int k, int norm,
                                                                int32_t* __restrict__ indices,
                                                                float* __restrict__ weights,
                                                                float* __restrict__ probabilities) {
  __shared__ TopkScratch topk[4];
  const int t = blockIdx.x * 4 + threadIdx.x / 64, lane = threadIdx.x % 64;
  if (t >= tokens) return;
  const float* row = logits + (int64_t)t * experts;
  int sel;
  float w, full;
  wave_route_softmax<PER_LANE>(row, experts, k, norm != 0, lane, topk[threadIdx.x / 64], sel, w,
                               probabilities != nullptr, full);
  if (lane < k) {
    indices[(int64_t)t * k + lane] = sel;
    weights[(int64_t)t * k + lane] = w;
  }
  if (probabilities) {
    float top = row[__builtin_amdgcn_readlane(sel, 0)];
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts) probabilities[(int64_t)t * experts + e] = __expf(row[e] - top) / full;
    }
  }
}

// Scores of the DeepSeek gate in the stated arithmetic of route_device.h: sigmoid, or
// sqrt(softplus(l)) = sqrt(max(l, 0) + log1p(exp(-|l|))) (Native/DeepSeekNative/engine.mm:1875-1876).
__device__ __forceinline__ float score_fn(float l, int func) {
  return func == 1 ? sigmoid_defined(l) : sqrt_softplus_defined(l);
}

// FUNC: 0 softmax, 1 sigmoid, 2 sqrt-softplus (one instance each, so the score code of the
// others is not carried along). Every logit and bias load of a row is issued before any use.
template <int PER_LANE, int FUNC>
__global__ void __launch_bounds__(256) route_scored_kernel(const float* __restrict__ logits,
                                                          const float* __restrict__ bias, int tokens, int experts,
                                                          int k, float route_scale, int norm, int n_groups,
                                                          int topk_groups, int32_t* __restrict__ indices,
                                                          float* __restrict__ weights) {
  constexpr int func = FUNC;
  __shared__ float biased_all[4][64 * PER_LANE];
  __shared__ float score_all[4][64 * PER_LANE];
  __shared__ TopkScratch topk[4];
  const int wave = threadIdx.x / 64, t = blockIdx.x * 4 + wave, lane = threadIdx.x % 64;
  if (t >= tokens) return;
  float* biased_lds = biased_all[wave];  // each wave's own rows: LDS is shared only within the wave
  float* score_lds = score_all[wave];
  const float* row = logits + (int64_t)t * experts;
  float lg[PER_LANE], bs[PER_LANE];
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {  // in-bounds addresses: every load is unconditional
    const int e = min(r * 64 + lane, experts - 1);
    lg[r] = row[e];
    bs[r] = bias ? bias[e] : 0.0f;
  }
  float vals[PER_LANE];
  float top = 0.0f, denom = 1.0f;
  if constexpr (func == 0) {  // softmax scores need the row max and sum
    float m = -INFINITY;
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts) m = fmaxf(m, lg[r]);
    }
    int dummy = 0;
    wave_argmax(m, dummy);
    top = m;
    float part = 0.0f;
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts) part += exp_defined(lg[r] - top);
    }
    denom = segment_sum<64>(part);
  }
#pragma unroll
  for (int r = 0; r < PER_LANE; ++r) {
    int e = r * 64 + lane;
    if (e < experts) {
      float s = func == 0 ? exp_defined(lg[r] - top) / denom : score_fn(lg[r], func);
      float b = s + bs[r];
      score_lds[e] = s;
      biased_lds[e] = b;
      vals[r] = b;
    } else {
      vals[r] = -INFINITY;
    }
  }
  // a wave's LDS operations complete in order; the fence keeps the compiler from moving
  // the reads below above the writes
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (n_groups > 1) {
    int gsize = experts / n_groups;
    // A group's score is the sum of its two largest biased scores (DeepSeek-V3 rule).
    float gs[1] = {-INFINITY};
    if (gsize == 32 && experts % 64 == 0) {
      // Group 2 r + h is the lane half h of register r: the half's top two meet in five
      // xor butterflies (merging two pairs: a = max, b = max(min(a1, a2), max(b1, b2)), the
      // same multiset rule as the scan below, ties counted twice), then lanes 0 and 32 hold
      // each register's two group scores.
#pragma unroll
      for (int r = 0; r < PER_LANE; ++r) {
        float a = vals[r], b = -INFINITY;
#pragma unroll
        for (int m = 1; m < 32; m <<= 1) {
          const float oa = __shfl_xor(a, m, 64), ob = __shfl_xor(b, m, 64);
          b = fmaxf(fminf(a, oa), fmaxf(b, ob));
          a = fmaxf(a, oa);
        }
        const float sum = a + b;
        const float s0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 0));
        const float s1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sum), 32));
        gs[0] = lane == 2 * r ? s0 : (lane == 2 * r + 1 ? s1 : gs[0]);
      }
      if (lane >= n_groups) gs[0] = -INFINITY;
    } else if (lane < n_groups) {
      float a = -INFINITY, b = -INFINITY;
      for (int j = 0; j < gsize; ++j) {
        float v = biased_lds[lane * gsize + j];
        if (v > a) { b = a; a = v; }
        else if (v > b) b = v;
      }
      gs[0] = a + b;
    }
    int gsel;
    float gval;
    wave_topk<1>(gs, n_groups, topk_groups, lane, topk[wave], gsel, gval);
    uint64_t keep = 0;
    for (int j = 0; j < topk_groups; ++j) keep |= 1ull << __builtin_amdgcn_readlane(gsel, j);
#pragma unroll
    for (int r = 0; r < PER_LANE; ++r) {
      int e = r * 64 + lane;
      if (e < experts && !((keep >> (e / gsize)) & 1ull)) vals[r] = -INFINITY;
    }
  }
  int sel;
  float sel_val;
  wave_topk<PER_LANE>(vals, experts, k, lane, topk[wave], sel, sel_val);
  float mine = lane < k ? score_lds[lane < k ? sel : 0] : 0.0f;
  float sum = segment_sum<64>(mine);
  if (lane < k) {
    float w = mine;
    if (norm && k > 1) w = w / (sum + 1e-20f);
    indices[(int64_t)t * k + lane] = sel;
    weights[(int64_t)t * k + lane] = w * route_scale;
  }
}

// logits[t, e] = sum_h x[t, h] * w[e, h]; one wave per (e, t), lanes stride h in bf16 pairs.
__global__ void __launch_bounds__(256) linear_bf16_kernel(const uint32_t* __restrict__ x, const uint32_t* __restrict__ w,
                                                         int tokens, int hidden, int outputs, float* __restrict__ out) {
  int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  int e = blockIdx.x * 4 + wave, t = blockIdx.y;
  if (e >= outputs || t >= tokens) return;
  int pairs = hidden / 2;
  const uint32_t* xr = x + (int64_t)t * pairs;
  const uint32_t* wr = w + (int64_t)e * pairs;
  float acc = 0.0f;
  for (int p = lane; p < pairs; p += 64) acc = dot2_bf16(bits_to_bf16x2(xr[p]), bits_to_bf16x2(wr[p]), acc);
  acc = segment_sum<64>(acc);
  if (lane == 0) out[(int64_t)t * outputs + e] = acc;
}

// dot of 8 bf16 (one 16-byte chunk) against 8 bf16
__device__ __forceinline__ float dot8_bf16x(uint4 a, uint4 b, float acc) {
  acc = dot2_bf16(bits_to_bf16x2(a.x), bits_to_bf16x2(b.x), acc);
  acc = dot2_bf16(bits_to_bf16x2(a.y), bits_to_bf16x2(b.y), acc);
  acc = dot2_bf16(bits_to_bf16x2(a.z), bits_to_bf16x2(b.z), acc);
  return dot2_bf16(bits_to_bf16x2(a.w), bits_to_bf16x2(b.w), acc);
}

// Few tokens (<= TMAX): a wave takes LR_ROWS output rows and streams them once in 16-byte
// chunks (non-temporal loads: the rows are read once per call, 3% off the C5 verify step); each chunk of every token's x, loaded once per wave, meets all LR_ROWS rows, so x
// is read from the caches once per LR_ROWS rows (one x pass per row made x, not the
// weights, the larger read at 4 tokens). grid: ceil(outputs / (4 LR_ROWS)), 4 waves a block.
constexpr int LR_ROWS = 4;
template <int TMAX>
__global__ void __launch_bounds__(256) linear_rows_kernel(const uint4* __restrict__ x, const uint4* __restrict__ w,
                                                         int tokens, int chunks, int outputs, float* __restrict__ out) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int o0 = (blockIdx.x * 4 + wave) * LR_ROWS;
  if (o0 >= outputs) return;
  const uint4* wr[LR_ROWS];
#pragma unroll
  for (int r = 0; r < LR_ROWS; ++r) wr[r] = w + (int64_t)min(o0 + r, outputs - 1) * chunks;  // in bounds
  float acc[LR_ROWS][TMAX];
#pragma unroll
  for (int r = 0; r < LR_ROWS; ++r)
#pragma unroll
    for (int t = 0; t < TMAX; ++t) acc[r][t] = 0.0f;
#pragma unroll 2
  for (int c = lane; c < chunks; c += 64) {
    uint4 wv[LR_ROWS];
#pragma unroll
    for (int r = 0; r < LR_ROWS; ++r) wv[r] = gload16_nt(&wr[r][c]);
#pragma unroll
    for (int t = 0; t < TMAX; ++t) {
      if (t < tokens) {
        const uint4 xv = x[(int64_t)t * chunks + c];
#pragma unroll
        for (int r = 0; r < LR_ROWS; ++r) acc[r][t] = dot8_bf16x(wv[r], xv, acc[r][t]);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < LR_ROWS; ++r) {
#pragma unroll
    for (int t = 0; t < TMAX; ++t) {
      if (t < tokens) {  // uniform
        const float v = segment_sum<64>(acc[r][t]);
        if (lane == 0 && o0 + r < outputs) out[(int64_t)t * outputs + o0 + r] = v;
      }
    }
  }
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT int wm_route_softmax_topk(const float* logits, int32_t tokens, int32_t experts, int32_t k,
                                    int32_t norm_topk_prob, int32_t* indices, float* weights, float* probabilities,
                                    void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_route_softmax_topk: negative token count");
    if (experts < 1 || experts > 1024) fail("wm_route_softmax_topk: experts must be in 1..1024");
    if (k < 1 || k > ROUTE_MAX_K || k > experts) fail("wm_route_softmax_topk: k must be in 1..min(32, experts)");
    if (tokens == 0) return;
    if (!logits || !indices || !weights) fail("wm_route_softmax_topk: null pointer");
    hipStream_t s = as_stream(stream);
    int per_lane = (experts + 63) / 64;
#define WM_RS(P) hipLaunchKernelGGL(route_softmax_topk_kernel<P>, dim3((tokens + 3) / 4), dim3(256), 0, s, logits, tokens, experts, \
                                    k, norm_topk_prob, indices, weights, probabilities)
    if (per_lane <= 1) WM_RS(1);
    else if (per_lane <= 2) WM_RS(2);
    else if (per_lane <= 4) WM_RS(4);
    else if (per_lane <= 8) WM_RS(8);
    else WM_RS(16);
#undef WM_RS
    check_launch("route_softmax_topk");
  });
}

WM_EXPORT int wm_route_scored(const float* logits, const float* bias, int32_t tokens, int32_t experts, int32_t k,
                              int32_t func, float route_scale, int32_t norm_topk_prob, int32_t n_groups,
                              int32_t topk_groups, int32_t* indices, float* weights, void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_route_scored: negative token count");
    if (experts < 1 || experts > 1024) fail("wm_route_scored: experts must be in 1..1024");
    if (k < 1 || k > ROUTE_MAX_K || k > experts) fail("wm_route_scored: k must be in 1..min(32, experts)");
    if (func < 0 || func > 2) fail("wm_route_scored: func must be 0 (softmax), 1 (sigmoid) or 2 (sqrt-softplus)");
    if (n_groups < 1 || n_groups > 64 || experts % n_groups) fail("wm_route_scored: n_groups must divide experts (<= 64)");
    if (n_groups > 1 && experts / n_groups < 2) fail("wm_route_scored: groups need at least two experts");
    if (topk_groups < 1 || topk_groups > n_groups) fail("wm_route_scored: topk_groups must be in 1..n_groups");
    if (n_groups > 1 && k > topk_groups * (experts / n_groups)) fail("wm_route_scored: k exceeds the kept groups' experts");
    if (tokens == 0) return;
    if (!logits || !indices || !weights) fail("wm_route_scored: null pointer");
    hipStream_t s = as_stream(stream);
    int per_lane = (experts + 63) / 64;
#define WM_RS_F(P, F) hipLaunchKernelGGL((route_scored_kernel<P, F>), dim3((tokens + 3) / 4), dim3(256), 0, s, logits, bias, \
                                         tokens, experts, k, route_scale, norm_topk_prob, n_groups, topk_groups, indices, weights)
#define WM_RS(P) do { if (func == 0) WM_RS_F(P, 0); else if (func == 1) WM_RS_F(P, 1); else WM_RS_F(P, 2); } while (0)
    if (per_lane <= 1) WM_RS(1);
    else if (per_lane <= 2) WM_RS(2);
    else if (per_lane <= 4) WM_RS(4);
    else if (per_lane <= 8) WM_RS(8);
    else WM_RS(16);
#undef WM_RS
#undef WM_RS_F
    check_launch("route_scored");
  });
}

WM_EXPORT int wm_linear_bf16(const void* x, const void* w, int32_t tokens, int32_t hidden, int32_t outputs, float* out,
                             void* stream) {
  return guarded([&] {
    if (tokens < 0 || outputs < 0 || hidden < 2 || hidden % 2) fail("wm_linear_bf16: bad shape");
    if (tokens == 0 || outputs == 0) return;
    if (!x || !w || !out) fail("wm_linear_bf16: null pointer");
    // 64+ tokens: the router GEMM on MFMA (norm_router.hip); up to 16 tokens with 16-byte
    // rows: one pass over each weight row; else one wave per output
    if (linear_bf16_mfma(x, w, tokens, hidden, outputs, out, as_stream(stream))) return;
    if (tokens <= 16 && hidden % 8 == 0 && ((uintptr_t)x % 16) == 0 && ((uintptr_t)w % 16) == 0) {
      const dim3 grid((outputs + 4 * LR_ROWS - 1) / (4 * LR_ROWS));
      const int chunks = hidden / 8;
#define WM_LR(T) hipLaunchKernelGGL(linear_rows_kernel<T>, grid, dim3(256), 0, as_stream(stream), (const uint4*)x, \
                                    (const uint4*)w, tokens, chunks, outputs, out)
      if (tokens <= 1) WM_LR(1);
      else if (tokens <= 2) WM_LR(2);
      else if (tokens <= 4) WM_LR(4);
      else if (tokens <= 8) WM_LR(8);
      else WM_LR(16);
#undef WM_LR
      check_launch("linear_rows");
      return;
    }
    hipLaunchKernelGGL(linear_bf16_kernel, dim3((outputs + 3) / 4, tokens), dim3(256), 0, as_stream(stream),
                       (const uint32_t*)x, (const uint32_t*)w, tokens, hidden, outputs, out);
    check_launch("linear_bf16");
  });
}

}  // extern "C"
