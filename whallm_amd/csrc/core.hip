// Error state, version, and the standalone dequant kernels (formats).
#include <cmath>
#include <stdexcept>

#include "wm_common.h"

namespace wm {

static thread_local std::string g_error;

void set_error(const std::string& message) { g_error = message; }
void clear_error() { g_error.clear(); }
void fail(const std::string& message) { throw std::runtime_error(message); }
void check_hip(hipError_t status, const char* what) {
  if (status != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(status));
}
void check_launch(const char* kernel) {
  hipError_t status = hipGetLastError();
  if (status != hipSuccess) fail(std::string("launch of ") + kernel + " failed: " + hipGetErrorString(status));
}

// out[r, i] for 8 consecutive i of one packed word. Each thread decodes one word,
// with the same gfx950 scaled convert the GEMV and GEMM kernels use.
template <bool BF16>
__global__ void __launch_bounds__(256) dequant_mxfp4_kernel(const uint32_t* __restrict__ packed,
                                                           const uint8_t* __restrict__ scales, int64_t rows,
                                                           int64_t words_per_row, void* __restrict__ out) {
  int64_t w = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (w >= rows * words_per_row) return;
  int64_t r = w / words_per_row, c = w % words_per_row;
  uint32_t word = packed[w];
  float scale = e8m0_scale_operand(scales[r * (words_per_row / 4) + c / 4]);
  if (BF16) {
    wm_bf16x2 v[4];
    fp4x8_to_bf16(word, scale, v);
    uint4 o = make_uint4(bf16x2_to_bits(v[0]), bf16x2_to_bits(v[1]), bf16x2_to_bits(v[2]), bf16x2_to_bits(v[3]));
    reinterpret_cast<uint4*>(out)[w] = o;
  } else {
    float4* o = reinterpret_cast<float4*>(out) + 2 * w;
    wm_f32x2 a = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 0);
    wm_f32x2 b = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 1);
    wm_f32x2 c2 = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 2);
    wm_f32x2 d = __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(word, scale, 3);
    o[0] = make_float4(a[0], a[1], b[0], b[1]);
    o[1] = make_float4(c2[0], c2[1], d[0], d[1]);
  }
}

__global__ void __launch_bounds__(256) dequant_fp8_kernel(const uint8_t* __restrict__ w, const float* __restrict__ s,
                                                         int64_t rows, int64_t cols, float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  int64_t r = i / cols, c = i % cols;
  int64_t scale_cols = (cols + 127) / 128;
  out[i] = e4m3_to_f32(w[i]) * s[(r / 128) * scale_cols + c / 128];
}

// V4.1 FP8: out[r, c] = e4m3(w[r, c]) * 2^(s[r / 32, c / 32] - 127), the exact product.
__global__ void __launch_bounds__(256) dequant_fp8_e8m0_kernel(const uint8_t* __restrict__ w,
                                                              const uint8_t* __restrict__ s, int64_t rows,
                                                              int64_t cols, float* __restrict__ out) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * cols) return;
  int64_t r = i / cols, c = i % cols;
  out[i] = e4m3_to_f32(w[i]) * e8m0_value(s[(r / 32) * ((cols + 31) / 32) + c / 32]);
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT const char* wm_last_error(void) { return g_error.c_str(); }
WM_EXPORT const char* wm_version(void) { return "whallm_moe 0.1 gfx950"; }

WM_EXPORT int wm_dequant_mxfp4(const void* packed, const void* scales, int64_t rows, int64_t cols, void* out,
                               int out_bf16, void* stream) {
  return guarded([&] {
    if (!packed || !scales || !out) fail("wm_dequant_mxfp4: null pointer");
    if (rows < 0 || cols < 0 || cols % 32) fail("wm_dequant_mxfp4: cols must be a multiple of 32");
    int64_t words = rows * (cols / 8);
    if (words == 0) return;
    int64_t blocks = (words + 255) / 256;
    if (out_bf16)
      hipLaunchKernelGGL(dequant_mxfp4_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                         (const uint32_t*)packed, (const uint8_t*)scales, rows, cols / 8, out);
    else
      hipLaunchKernelGGL(dequant_mxfp4_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, as_stream(stream),
                         (const uint32_t*)packed, (const uint8_t*)scales, rows, cols / 8, out);
    check_launch("dequant_mxfp4");
  });
}

WM_EXPORT int wm_dequant_fp8_blocks(const void* weight, const float* scales, int64_t rows, int64_t cols, float* out,
                                    void* stream) {
  return guarded([&] {
    if (!weight || !scales || !out) fail("wm_dequant_fp8_blocks: null pointer");
    if (rows < 0 || cols < 0) fail("wm_dequant_fp8_blocks: negative size");
    int64_t n = rows * cols;
    if (n == 0) return;
    hipLaunchKernelGGL(dequant_fp8_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream),
                       (const uint8_t*)weight, scales, rows, cols, out);
    check_launch("dequant_fp8_blocks");
  });
}

WM_EXPORT int wm_dequant_fp8_e8m0(const void* weight, const void* scales, int64_t rows, int64_t cols, float* out,
                                  void* stream) {
  return guarded([&] {
    if (!weight || !scales || !out) fail("wm_dequant_fp8_e8m0: null pointer");
    if (rows < 0 || cols < 0) fail("wm_dequant_fp8_e8m0: negative size");
    int64_t n = rows * cols;
    if (n == 0) return;
    hipLaunchKernelGGL(dequant_fp8_e8m0_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream),
                       (const uint8_t*)weight, (const uint8_t*)scales, rows, cols, out);
    check_launch("dequant_fp8_e8m0");
  });
}

}  // extern "C"
