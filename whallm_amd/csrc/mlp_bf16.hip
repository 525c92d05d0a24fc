// The reference's bf16 shared expert on the device:
//   y[t] = add[t] + g(t) * down(bf16(silu(x[t] . Wg^T) * (x[t] . Wu^T))),
//   g(t) = sigmoid(x[t] . gate_vec) (1 without a gate vector),
// the Qwen MLP (runtime/deepseek_v4_ssd/qwen4_exp.py:763-771) gated by
// shared_expert_gate (:1002-1003, :1045) and added to the routed combine; the native
// engine runs the same three linears with a mul_silu (Native/QwenNative/engine.mm:2075-2079).
// Weights are bf16 [I, H] (gate, up) and [H, I] (down), y = x W^T as mlx nn.Linear.
//
// Few tokens (decode, < 64): two HBM-bound GEMV kernels.
//   gate_up: a wave per intermediate row streams the gate and up rows (16 bytes per lane
//            per load) against every token's x, reduces, and writes the bf16 act; block 0
//            also computes each token's gate value.
//   down:    a wave per output row streams the down row against the tokens' act and writes
//            y = add + g * d (fp32 arithmetic, one bf16 rounding).
// 64+ tokens: the bf16 MFMA GEMM of the router (norm_router.hip) for the three linears,
// with an elementwise SwiGLU kernel between them and the gate / add in a final kernel.
#include <cmath>

#include "wm_common.h"

namespace wm {

bool linear_bf16_mfma(const void* x, const void* w, int tokens, int hidden, int outputs, float* out, hipStream_t s);
bool linear_bf16_mfma_fits(int tokens, int hidden);

constexpr int MLP_GEMV_MAX_TOKENS = 63;

// dot of 8 bf16 (one 16-byte chunk) against 8 bf16
__device__ __forceinline__ float dot8_bf16(uint4 a, uint4 b, float acc) {
  acc = dot2_bf16(bits_to_bf16x2(a.x), bits_to_bf16x2(b.x), acc);
  acc = dot2_bf16(bits_to_bf16x2(a.y), bits_to_bf16x2(b.y), acc);
  acc = dot2_bf16(bits_to_bf16x2(a.z), bits_to_bf16x2(b.z), acc);
  return dot2_bf16(bits_to_bf16x2(a.w), bits_to_bf16x2(b.w), acc);
}

// sigmoid(x[t] . v) by one wave (v may be null: 1).
__device__ __forceinline__ float wave_gate(const uint16_t* __restrict__ xr, const uint16_t* __restrict__ v, int hidden,
                                           int lane) {
  if (!v) return 1.0f;
  float a = 0.0f;
  for (int c = lane; c < hidden / 8; c += 64)
    a = dot8_bf16(reinterpret_cast<const uint4*>(xr)[c], reinterpret_cast<const uint4*>(v)[c], a);
  a = segment_sum<64>(a);
  return 1.0f / (1.0f + __expf(-a));
}

// grid: ceil(I / 4); wave w of block b owns intermediate row i = 4 b + w.
__global__ void __launch_bounds__(256) mlp_gate_up_gemv_kernel(const uint16_t* __restrict__ x, int tokens, int hidden,
                                                               int inter, const uint16_t* __restrict__ wg,
                                                               const uint16_t* __restrict__ wu,
                                                               const uint16_t* __restrict__ gate_vec,
                                                               uint16_t* __restrict__ act, float* __restrict__ gate) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int i = blockIdx.x * 4 + wave;
  if (blockIdx.x == 0)
    for (int t = wave; t < tokens; t += 4) {
      const float g = wave_gate(x + (int64_t)t * hidden, gate_vec, hidden, lane);
      if (lane == 0) gate[t] = g;
    }
  if (i >= inter) return;
  const uint4* gr = reinterpret_cast<const uint4*>(wg + (int64_t)i * hidden);
  const uint4* ur = reinterpret_cast<const uint4*>(wu + (int64_t)i * hidden);
  const int chunks = hidden / 8;
  for (int t = 0; t < tokens; ++t) {
    const uint4* xr = reinterpret_cast<const uint4*>(x + (int64_t)t * hidden);
    float g = 0.0f, u = 0.0f;
    for (int c = lane; c < chunks; c += 64) {
      const uint4 xv = xr[c];
      g = dot8_bf16(gr[c], xv, g);
      u = dot8_bf16(ur[c], xv, u);
    }
    g = segment_sum<64>(g);
    u = segment_sum<64>(u);
    if (lane == 0) act[(int64_t)t * inter + i] = f32_to_bf16_bits(silu(g) * u);
  }
}

// grid: ceil(H / 4); wave w of block b owns output row o = 4 b + w.
__global__ void __launch_bounds__(256) mlp_down_gemv_kernel(const uint16_t* __restrict__ act, int tokens, int hidden,
                                                            int inter, const uint16_t* __restrict__ wd,
                                                            const float* __restrict__ gate,
                                                            const uint16_t* __restrict__ add,
                                                            uint16_t* __restrict__ y) {
  const int wave = threadIdx.x / 64, lane = threadIdx.x % 64;
  const int o = blockIdx.x * 4 + wave;
  if (o >= hidden) return;
  const uint4* dr = reinterpret_cast<const uint4*>(wd + (int64_t)o * inter);
  const int chunks = inter / 8;
  for (int t = 0; t < tokens; ++t) {
    const uint4* ar = reinterpret_cast<const uint4*>(act + (int64_t)t * inter);
    float d = 0.0f;
    for (int c = lane; c < chunks; c += 64) d = dot8_bf16(dr[c], ar[c], d);
    d = segment_sum<64>(d);
    if (lane == 0) {
      float v = gate[t] * d;
      if (add) v += bf16_bits_to_f32(add[(int64_t)t * hidden + o]);
      y[(int64_t)t * hidden + o] = f32_to_bf16_bits(v);
    }
  }
}

// act[t, i] = bf16(silu(g[t, i]) * u[t, i]) for the MFMA path; one thread per element.
__global__ void __launch_bounds__(256) mlp_act_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                      int64_t n, uint16_t* __restrict__ act) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e < n) act[e] = f32_to_bf16_bits(silu(g[e]) * u[e]);
}

// gate[t] for the MFMA path: one wave per token.
__global__ void __launch_bounds__(64) mlp_gate_kernel(const uint16_t* __restrict__ x, int hidden,
                                                      const uint16_t* __restrict__ gate_vec, float* __restrict__ gate) {
  const float g = wave_gate(x + (int64_t)blockIdx.x * hidden, gate_vec, hidden, threadIdx.x);
  if (threadIdx.x == 0) gate[blockIdx.x] = g;
}

// y[t, o] = bf16(add[t, o] + gate[t] * d[t, o]); one thread per element.
__global__ void __launch_bounds__(256) mlp_out_kernel(const float* __restrict__ d, const float* __restrict__ gate,
                                                      const uint16_t* __restrict__ add, int hidden, int64_t n,
                                                      uint16_t* __restrict__ y) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= n) return;
  float v = gate[e / hidden] * d[e];
  if (add) v += bf16_bits_to_f32(add[e]);
  y[e] = f32_to_bf16_bits(v);
}

static size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

struct MlpLayout {
  size_t gate, act, g, u, d, total;
};

static MlpLayout mlp_layout(int tokens, int hidden, int inter) {
  MlpLayout p{};
  size_t at = 0;
  const size_t T = tokens > 0 ? (size_t)tokens : 1;
  p.gate = at; at += align256(sizeof(float) * T);
  p.act = at;  at += align256(sizeof(uint16_t) * T * inter);
  if (tokens > MLP_GEMV_MAX_TOKENS) {
    p.g = at; at += align256(sizeof(float) * T * inter);
    p.u = at; at += align256(sizeof(float) * T * inter);
    p.d = at; at += align256(sizeof(float) * T * hidden);
  }
  p.total = at;
  return p;
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_mlp_bf16_workspace_size(int32_t tokens, int32_t hidden, int32_t inter) {
  if (tokens < 0 || hidden < 1 || inter < 1) return 0;
  return mlp_layout(tokens, hidden, inter).total;
}

WM_EXPORT int wm_mlp_bf16(const void* x, int32_t tokens, int32_t hidden, int32_t inter, const void* gate_w,
                          const void* up_w, const void* down_w, const void* gate_vec, const void* add, void* y,
                          void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (tokens < 0 || hidden < 32 || hidden % 32 || inter < 32 || inter % 32)
      fail("wm_mlp_bf16: hidden and intermediate must be positive multiples of 32");
    if (tokens == 0) return;
    if (!x || !gate_w || !up_w || !down_w || !y || !workspace) fail("wm_mlp_bf16: null pointer");
    for (const void* p : {x, gate_w, up_w, down_w, gate_vec, add, (const void*)y, (const void*)workspace})
      if ((uintptr_t)p % 16) fail("wm_mlp_bf16: every tensor must be 16-byte aligned");
    const MlpLayout p = mlp_layout(tokens, hidden, inter);
    if (workspace_bytes < p.total) fail("wm_mlp_bf16: workspace too small");
    // every GEMM of the MFMA path is checked before the first launch, so a shape it cannot
    // hold launches nothing
    if (tokens > MLP_GEMV_MAX_TOKENS && (!linear_bf16_mfma_fits(tokens, hidden) || !linear_bf16_mfma_fits(tokens, inter)))
      fail("wm_mlp_bf16: hidden or intermediate too large for the MFMA GEMM's x tile (150 KB of LDS)");
    hipStream_t s = as_stream(stream);
    uint8_t* ws = (uint8_t*)workspace;
    float* gate = (float*)(ws + p.gate);
    uint16_t* act = (uint16_t*)(ws + p.act);
    const uint16_t *xb = (const uint16_t*)x, *gv = (const uint16_t*)gate_vec, *ab = (const uint16_t*)add;
    if (tokens <= MLP_GEMV_MAX_TOKENS) {
      hipLaunchKernelGGL(mlp_gate_up_gemv_kernel, dim3((inter + 3) / 4), dim3(256), 0, s, xb, tokens, hidden, inter,
                         (const uint16_t*)gate_w, (const uint16_t*)up_w, gv, act, gate);
      check_launch("mlp_gate_up_gemv");
      hipLaunchKernelGGL(mlp_down_gemv_kernel, dim3((hidden + 3) / 4), dim3(256), 0, s, act, tokens, hidden, inter,
                         (const uint16_t*)down_w, gate, ab, (uint16_t*)y);
      check_launch("mlp_down_gemv");
      return;
    }
    float* g = (float*)(ws + p.g);
    float* u = (float*)(ws + p.u);
    float* d = (float*)(ws + p.d);
    if (!linear_bf16_mfma(x, gate_w, tokens, hidden, inter, g, s) || !linear_bf16_mfma(x, up_w, tokens, hidden, inter, u, s))
      fail("wm_mlp_bf16: the gate/up GEMM does not support this shape");
    const int64_t ni = (int64_t)tokens * inter, nh = (int64_t)tokens * hidden;
    hipLaunchKernelGGL(mlp_act_kernel, dim3((unsigned)((ni + 255) / 256)), dim3(256), 0, s, g, u, ni, act);
    check_launch("mlp_act");
    hipLaunchKernelGGL(mlp_gate_kernel, dim3(tokens), dim3(64), 0, s, xb, hidden, gv, gate);
    check_launch("mlp_gate");
    if (!linear_bf16_mfma(act, down_w, tokens, inter, hidden, d, s))
      fail("wm_mlp_bf16: the down GEMM does not support this shape");
    hipLaunchKernelGGL(mlp_out_kernel, dim3((unsigned)((nh + 255) / 256)), dim3(256), 0, s, d, gate, ab, hidden, nh,
                       (uint16_t*)y);
    check_launch("mlp_out");
  });
}

}  // extern "C"
