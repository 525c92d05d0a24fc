// Trace hooks of the profiling build of the one-launch decode layer (whallm_amd/phase_trace.py
// compiles decode_layer.hip with this header first; the library itself never includes it).
// WM_DS_TRACE keeps s_memrealtime (100 MHz, one clock for the chip) of lane 0 of each wave in
// LDS, so a trace point adds no global store (whose completion a later s_waitcnt vmcnt would
// wait for); WM_DS_TRACE_FLUSH copies the points of the call to
// wm_trace_buf[workgroup 256][call slot 128][wave 4][point 16] at the end of the launch.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

__constant__ uint64_t* wm_trace_buf;

__device__ __forceinline__ uint64_t* wm_trace_lds() {
  __shared__ uint64_t points[4 * 16];
  return points;
}

#define WM_DS_TRACE(layer, point)                                                          \
  do {                                                                                     \
    if ((threadIdx.x & 63) == 0) wm_trace_lds()[(threadIdx.x / 64) * 16 + (point)] =       \
        __builtin_amdgcn_s_memrealtime();                                                  \
  } while (0)

#define WM_DS_TRACE_FLUSH(layer)                                                           \
  do {                                                                                     \
    uint64_t* tb_ = wm_trace_buf;                                                          \
    if (tb_ && (threadIdx.x & 63) < 16)                                                    \
      tb_[(((size_t)blockIdx.x * 128 + (layer)) * 4 + threadIdx.x / 64) * 16 + (threadIdx.x & 63)] = \
          wm_trace_lds()[(threadIdx.x / 64) * 16 + (threadIdx.x & 63)];                  \
  } while (0)

extern "C" __attribute__((visibility("default"))) int wm_trace_set(void* p) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(wm_trace_buf), &p, sizeof(p));
}
