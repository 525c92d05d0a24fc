// Internal interfaces between the MoE kernel files of libwhallm_moe.
#pragma once

#include "wm_common.h"

namespace wm {

// Device addresses of one expert's four regions.
struct ExpertRegions {
  const uint8_t* gate_up;
  const uint8_t* gate_up_scales;
  const uint8_t* down;
  const uint8_t* down_scales;
};

// Regions of expert e. A slot map entry below 0 means the expert is not resident: the
// regions then point at slot 0 (so no access leaves the pool) and `resident` is false;
// every kernel makes such a pair contribute nothing.
__device__ __forceinline__ ExpertRegions expert_regions(const wm_mxfp4_experts& t, int e, bool& resident) {
  int64_t slot = t.slots ? t.slots[e] : e;
  resident = slot >= 0;
  if (slot < 0) slot = 0;
  ExpertRegions r;
  r.gate_up = (const uint8_t*)t.gate_up + slot * t.gate_up_stride;
  r.gate_up_scales = (const uint8_t*)t.gate_up_scales + slot * t.gate_up_scales_stride;
  r.down = (const uint8_t*)t.down + slot * t.down_stride;
  r.down_scales = (const uint8_t*)t.down_scales + slot * t.down_scales_stride;
  return r;
}

// Device addresses of one FP8 expert (w13 = gate/up rows, w2 = down; block scales fp32
// 128x128 or E8M0 32x32 bytes, by the table's scale_format).
struct Fp8Regions {
  const uint8_t* w13;
  const uint8_t* w13_scales;
  const uint8_t* w2;
  const uint8_t* w2_scales;
};

__device__ __forceinline__ Fp8Regions fp8_regions(const wm_fp8_experts& t, int e, bool& resident) {
  int64_t slot = t.slots ? t.slots[e] : e;
  resident = slot >= 0;
  if (slot < 0) slot = 0;  // not resident: slot 0's address, and the pair contributes nothing
  Fp8Regions r;
  r.w13 = (const uint8_t*)t.w13 + slot * t.w13_stride;
  r.w13_scales = (const uint8_t*)t.w13_scales + slot * t.w13_scales_stride;
  r.w2 = (const uint8_t*)t.w2 + slot * t.w2_stride;
  r.w2_scales = (const uint8_t*)t.w2_scales + slot * t.w2_scales_stride;
  return r;
}

// Host-side checks of an expert table; raises on a bad shape.
void validate_experts(const wm_mxfp4_experts* e, const char* what, bool shared);

// Whether the decode kernels take this shape (multiples of 32 up to 16384).
bool decode_mxfp4_supports(int hidden, int inter);

// Decode path (small T): gate_up_act into `act` [(T*K + T_shared), I] fp32, then
// down (combined into y [T, H] bf16, or per pair into y [T*K, H] bf16).
void decode_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                  const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                  uint16_t* y, bool combine, float* act, hipStream_t s);

// Prefill path (grouped GEMM). `ws` holds the permute and activation buffers.
size_t prefill_workspace_size(int tokens, int k, const wm_mxfp4_experts& e, bool has_shared);
void prefill_mxfp4(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                   const wm_mxfp4_experts& routed, const wm_mxfp4_experts* shared, const uint16_t* shared_gate,
                   uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s);

// FP8 expert FFN (hidden and intermediate multiples of 128; up to 8192 for decode).
void decode_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                uint16_t* y, bool combine, uint16_t* act, hipStream_t s);  // act: bf16 [pairs, I]
size_t prefill_fp8_workspace_size(int tokens, int k, const wm_fp8_experts& e, bool has_shared);
void prefill_fp8(const uint16_t* x, int tokens, const int32_t* indices, const float* weights, int k,
                 const wm_fp8_experts& routed, const wm_fp8_experts* shared, const uint16_t* shared_gate,
                 uint16_t* y, bool combine, void* ws, size_t ws_bytes, hipStream_t s);

// The one-launch decode layer (decode_layer.hip): shapes with a fused instantiation.
bool moe_layer_fused_supports(int hidden, int inter, int k);

// Pairs at or below this count take the decode path.
constexpr int DECODE_MAX_PAIRS = 256;

}  // namespace wm
