// Combine of per-pair expert rows given in router order:
//   y[t, c] = sum_k w[t, k] * rows[t, k, c]  (+ add[t, c])
// with fp32 accumulation in k order and a bf16 result. This is SparseMoE._combine
// (runtime/deepseek_v4_ssd/qwen4_exp.py:1048-1051) and the DeepSeek _route_reduce
// (model.py:544-546) over the [T, K, H] output of wm_experts_mxfp4 / wm_experts_fp8, e.g.
// after a layer ran in two calls (ready experts first, the rest after their fills). The
// fused layer entry points (wm_moe_mxfp4 / wm_moe_fp8) combine inside their own kernels.
//
// HBM-bound: each thread owns 8 columns of one token, issues all K row loads of the token
// before summing (like the grouped path's combine), and writes one 16-byte bf16 chunk.
#include "wm_common.h"

namespace wm {

__global__ void __launch_bounds__(256) combine_pairs_kernel(const uint16_t* __restrict__ rows,
                                                            const float* __restrict__ weights, int k, int hidden,
                                                            const uint16_t* __restrict__ add,
                                                            uint16_t* __restrict__ y) {
  const int t = blockIdx.x;
  const int c8 = blockIdx.y * blockDim.x + threadIdx.x;
  if (c8 * 8 >= hidden) return;
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  constexpr int BATCH = 16;
  for (int j0 = 0; j0 < k; j0 += BATCH) {
    uint4 v[BATCH];
#pragma unroll
    for (int q = 0; q < BATCH; ++q)
      if (j0 + q < k) v[q] = reinterpret_cast<const uint4*>(rows + ((int64_t)t * k + j0 + q) * hidden)[c8];
#pragma unroll
    for (int q = 0; q < BATCH; ++q) {
      if (j0 + q < k) {  // pairs in order, as loaded
        const float w = weights[(int64_t)t * k + j0 + q];
        const uint32_t u[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          acc[2 * m] = fmaf(w, bf16_bits_to_f32(u[m] & 0xffffu), acc[2 * m]);
          acc[2 * m + 1] = fmaf(w, bf16_bits_to_f32(u[m] >> 16), acc[2 * m + 1]);
        }
      }
    }
  }
  if (add) {
    const uint4 a = reinterpret_cast<const uint4*>(add + (int64_t)t * hidden)[c8];
    const uint32_t u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      acc[2 * m] += bf16_bits_to_f32(u[m] & 0xffffu);
      acc[2 * m + 1] += bf16_bits_to_f32(u[m] >> 16);
    }
  }
  uint4 o;
  o.x = f32_to_bf16_bits(acc[0]) | ((uint32_t)f32_to_bf16_bits(acc[1]) << 16);
  o.y = f32_to_bf16_bits(acc[2]) | ((uint32_t)f32_to_bf16_bits(acc[3]) << 16);
  o.z = f32_to_bf16_bits(acc[4]) | ((uint32_t)f32_to_bf16_bits(acc[5]) << 16);
  o.w = f32_to_bf16_bits(acc[6]) | ((uint32_t)f32_to_bf16_bits(acc[7]) << 16);
  reinterpret_cast<uint4*>(y + (int64_t)t * hidden)[c8] = o;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT int wm_combine_pairs(const void* rows, const float* weights, int32_t tokens, int32_t k, int32_t hidden,
                               const void* add, void* y, void* stream) {
  return guarded([&] {
    if (tokens < 0 || k < 1 || k > 64 || hidden < 8 || hidden % 8) fail("wm_combine_pairs: bad shape");
    if (tokens == 0) return;
    if (!rows || !weights || !y) fail("wm_combine_pairs: null pointer");
    if (((uintptr_t)rows | (uintptr_t)y | (uintptr_t)add) % 16) fail("wm_combine_pairs: rows, add and y must be 16-byte aligned");
    hipLaunchKernelGGL(combine_pairs_kernel, dim3(tokens, (hidden / 8 + 255) / 256), dim3(256), 0, as_stream(stream),
                       (const uint16_t*)rows, weights, k, hidden, (const uint16_t*)add, (uint16_t*)y);
    check_launch("combine_pairs");
  });
}

}  // extern "C"
