// The decode stack: L MoE layers chained through a pre-norm residual,
//   x_l = rmsnorm(r_l) (bf16),  r_{l+1} = r_l + MoE_l(x_l),
// which is a decoder layer's MoE half (DecoderLayer.feed_forward,
// qwen4_exp.py:1127-1149) with attention left out. The native engine runs the
// same per-layer loop on the host (Native/QwenNative/engine.mm:1567-1588); here
// routing never leaves the device, so a step has no host synchronisation and a
// caller can capture it in one HIP graph.
#include <cmath>

#include "moe_internal.h"

namespace wm {

// r[t] += y[t] (when y is set); x[t] = bf16(r[t] / sqrt(mean(r[t]^2) + eps)). One workgroup per token.
__global__ void __launch_bounds__(256) residual_rmsnorm_kernel(float* __restrict__ r, const uint16_t* __restrict__ y,
                                                               int hidden, float eps, uint16_t* __restrict__ x) {
  __shared__ float partial[4];
  int t = blockIdx.x;
  float* rr = r + (int64_t)t * hidden;
  float sum = 0.0f;
  for (int i = threadIdx.x; i < hidden; i += 256) {
    float v = rr[i];
    if (y) {
      v += bf16_bits_to_f32(y[(int64_t)t * hidden + i]);
      rr[i] = v;
    }
    sum += v * v;
  }
  sum = segment_sum<64>(sum);
  if (threadIdx.x % 64 == 0) partial[threadIdx.x / 64] = sum;
  __syncthreads();
  float total = partial[0] + partial[1] + partial[2] + partial[3];
  float inv = rsqrtf(total / (float)hidden + eps);
  for (int i = threadIdx.x; i < hidden; i += 256) x[(int64_t)t * hidden + i] = f32_to_bf16_bits(rr[i] * inv);
}

// The same for hidden = 1024 PER: thread i holds columns 4 (i + 256 c) .. + 3 (c < PER) in
// registers, every load issued before the first use, so a token costs one memory round
// trip instead of one per 256 columns; r and y are read once.
template <int PER>
__global__ void __launch_bounds__(256) residual_rmsnorm_vec_kernel(float* __restrict__ r, const uint16_t* __restrict__ y,
                                                                   float eps, uint16_t* __restrict__ x) {
  __shared__ float partial[4];
  constexpr int H = 1024 * PER;
  const int t = blockIdx.x;
  float4* rr = reinterpret_cast<float4*>(r + (int64_t)t * H);
  float4 v[PER];
#pragma unroll
  for (int c = 0; c < PER; ++c) v[c] = rr[threadIdx.x + 256 * c];
  if (y) {
    const uint2* yy = reinterpret_cast<const uint2*>(y + (int64_t)t * H);
    uint2 yv[PER];
#pragma unroll
    for (int c = 0; c < PER; ++c) yv[c] = yy[threadIdx.x + 256 * c];
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      v[c].x += bf16_bits_to_f32(yv[c].x & 0xffffu);
      v[c].y += bf16_bits_to_f32(yv[c].x >> 16);
      v[c].z += bf16_bits_to_f32(yv[c].y & 0xffffu);
      v[c].w += bf16_bits_to_f32(yv[c].y >> 16);
      rr[threadIdx.x + 256 * c] = v[c];
    }
  }
  float sum = 0.0f;
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    sum += v[c].x * v[c].x;
    sum += v[c].y * v[c].y;
    sum += v[c].z * v[c].z;
    sum += v[c].w * v[c].w;
  }
  sum = segment_sum<64>(sum);
  if (threadIdx.x % 64 == 0) partial[threadIdx.x / 64] = sum;
  __syncthreads();
  const float total = partial[0] + partial[1] + partial[2] + partial[3];
  const float inv = rsqrtf(total / (float)H + eps);
  uint2* xx = reinterpret_cast<uint2*>(x + (int64_t)t * H);
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const uint32_t lo = f32_to_bf16_bits(v[c].x * inv) | ((uint32_t)f32_to_bf16_bits(v[c].y * inv) << 16);
    const uint32_t hi = f32_to_bf16_bits(v[c].z * inv) | ((uint32_t)f32_to_bf16_bits(v[c].w * inv) << 16);
    xx[threadIdx.x + 256 * c] = make_uint2(lo, hi);
  }
}

void residual_rmsnorm(float* r, const uint16_t* y, int tokens, int hidden, float eps, uint16_t* x, hipStream_t s) {
  const bool aligned = (uintptr_t)r % 16 == 0 && (uintptr_t)y % 8 == 0 && (uintptr_t)x % 8 == 0;
  if (aligned && hidden % 1024 == 0 && hidden / 1024 >= 1 && hidden / 1024 <= 8) {
    switch (hidden / 1024) {
#define WM_RN(P) case P: hipLaunchKernelGGL(residual_rmsnorm_vec_kernel<P>, dim3(tokens), dim3(256), 0, s, r, y, eps, x); break;
      WM_RN(1) WM_RN(2) WM_RN(3) WM_RN(4) WM_RN(5) WM_RN(6) WM_RN(7) WM_RN(8)
#undef WM_RN
    }
  } else {
    hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(tokens), dim3(256), 0, s, r, y, hidden, eps, x);
  }
  check_launch("residual_rmsnorm");
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT int wm_residual_rmsnorm(float* residual, const void* y, int32_t tokens, int32_t hidden, float eps, void* x,
                                  void* stream) {
  return guarded([&] {
    if (tokens < 0 || hidden < 1) fail("wm_residual_rmsnorm: bad shape");
    if (tokens == 0) return;
    if (!residual || !x) fail("wm_residual_rmsnorm: null pointer");
    residual_rmsnorm(residual, (const uint16_t*)y, tokens, hidden, eps, (uint16_t*)x, as_stream(stream));
  });
}

WM_EXPORT size_t wm_moe_stack_mxfp4_workspace_size(int32_t tokens, int32_t k, const wm_mxfp4_experts* experts) {
  if (!experts || tokens < 0 || k < 1) return 0;
  size_t routes = align256(sizeof(int32_t) * (size_t)tokens * k) + align256(sizeof(float) * (size_t)tokens * k);
  size_t io = 2 * align256(sizeof(uint16_t) * (size_t)tokens * experts->hidden);
  return routes + io + wm_moe_mxfp4_workspace_size(tokens, k, experts);
}

WM_EXPORT int wm_moe_stack_mxfp4(const float* logits, int32_t layers, int32_t tokens, int32_t k,
                                 int32_t norm_topk_prob, const wm_mxfp4_experts* experts,
                                 const wm_mxfp4_experts* shared, const void* const* shared_gates, float* residual,
                                 float eps, void* x_out, void* workspace, size_t workspace_bytes,
                                 int (*cancel)(void*), void* cancel_context, void* stream) {
  return guarded([&] {
    if (layers < 1 || tokens < 0 || k < 1) fail("wm_moe_stack_mxfp4: bad shape");
    if (!experts || !residual || !logits) fail("wm_moe_stack_mxfp4: null pointer");
    for (int l = 0; l < layers; ++l) {
      validate_experts(&experts[l], "stack routed experts", false);
      if (experts[l].tiled || (shared && shared[l].tiled))
        fail("wm_moe_stack_mxfp4: the decode stack takes tables in the row layout, not the prefill tile layout");
      if (experts[l].hidden != experts[0].hidden || experts[l].inter != experts[0].inter ||
          experts[l].experts != experts[0].experts)
        fail("wm_moe_stack_mxfp4: layers differ in shape");
      if (shared) validate_experts(&shared[l], "stack shared expert", true);
    }
    if (tokens == 0) return;
    if (workspace_bytes < wm_moe_stack_mxfp4_workspace_size(tokens, k, &experts[0]))
      fail("wm_moe_stack_mxfp4: workspace too small");
    hipStream_t s = as_stream(stream);
    const int H = experts[0].hidden, E = experts[0].experts;
    uint8_t* base = (uint8_t*)workspace;
    int32_t* idx = (int32_t*)base;
    base += align256(sizeof(int32_t) * (size_t)tokens * k);
    float* w = (float*)base;
    base += align256(sizeof(float) * (size_t)tokens * k);
    uint16_t* x = (uint16_t*)base;
    base += align256(sizeof(uint16_t) * (size_t)tokens * H);
    uint16_t* y = (uint16_t*)base;
    base += align256(sizeof(uint16_t) * (size_t)tokens * H);
    size_t rest = workspace_bytes - (size_t)(base - (uint8_t*)workspace);
    residual_rmsnorm(residual, nullptr, tokens, H, eps, x, s);
    for (int l = 0; l < layers; ++l) {
      // polled before each layer is enqueued, as the reference engine polls between layers
      // (Native/QwenNative/engine.h:112-113); earlier layers stay enqueued
      if (cancel && cancel(cancel_context))
        throw Cancelled("wm_moe_stack_mxfp4: cancelled before layer " + std::to_string(l));
      if (wm_route_softmax_topk(logits + (size_t)l * tokens * E, tokens, E, k, norm_topk_prob, idx, w, nullptr,
                                stream) != 0)
        fail(wm_last_error());
      if (wm_moe_mxfp4(x, tokens, idx, w, k, &experts[l], shared ? &shared[l] : nullptr,
                       shared_gates ? shared_gates[l] : nullptr, y, base, rest, stream) != 0)
        fail(wm_last_error());
      residual_rmsnorm(residual, y, tokens, H, eps, l + 1 == layers && x_out ? (uint16_t*)x_out : x, s);
    }
  });
}

}  // extern "C"
