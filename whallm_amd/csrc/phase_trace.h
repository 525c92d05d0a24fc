// Trace hooks of the profiling build (whallm_amd/phase_trace.py compiles the persistent
// decode kernel with this header first; the library itself never includes it).
// WM_DS_TRACE stores s_memrealtime (100 MHz, one clock for the chip) and WM_DS_NOTE a value
// into wm_trace_buf[workgroup 256][layer 128][wave 4][point 16], lane 0 of each wave.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

__constant__ uint64_t* wm_trace_buf;

#define WM_DS_TRACE_AT(layer, point, value)                                                              \
  do {                                                                                                   \
    if ((threadIdx.x & 63) == 0) {                                                                       \
      uint64_t* tb_ = wm_trace_buf;                                                                      \
      if (tb_) tb_[(((size_t)blockIdx.x * 128 + (layer)) * 4 + threadIdx.x / 64) * 16 + (point)] = (value); \
    }                                                                                                    \
  } while (0)
#define WM_DS_TRACE(layer, point) WM_DS_TRACE_AT(layer, point, __builtin_amdgcn_s_memrealtime())
#define WM_DS_NOTE(layer, point, value) WM_DS_TRACE_AT(layer, point, (uint64_t)(value))

extern "C" __attribute__((visibility("default"))) int wm_trace_set(void* p) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(wm_trace_buf), &p, sizeof(p));
}
