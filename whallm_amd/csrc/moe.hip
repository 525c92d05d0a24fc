// C-ABI entry points of the MXFP4 MoE layer: argument checks, path choice
// (fused dequant-GEMV for decode, MFMA grouped GEMM for prefill) and workspace sizing.
#include <mutex>
#include <string>

#include "moe_internal.h"

namespace wm {

void validate_experts(const wm_mxfp4_experts* e, const char* what, bool shared) {
  std::string w(what);
  if (!e) fail(w + ": expert table is null");
  if (!e->gate_up || !e->gate_up_scales || !e->down || !e->down_scales) fail(w + ": expert region pointer is null");
  if (e->hidden < 32 || e->hidden % 32) fail(w + ": hidden must be a positive multiple of 32");
  if (e->inter < 32 || e->inter % 32) fail(w + ": intermediate must be a positive multiple of 32");
  if (!shared && (e->experts < 1 || e->experts > 1024)) fail(w + ": expert count must be in 1..1024");
  if (e->gate_up_stride < 0 || e->gate_up_scales_stride < 0 || e->down_stride < 0 || e->down_scales_stride < 0)
    fail(w + ": negative stride");
  if (e->swiglu_limit < 0.0f) fail(w + ": swiglu_limit must be >= 0");
  // 16-byte weight loads and 2-byte scale loads.
  auto aligned = [](const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; };
  if (!aligned(e->gate_up, 16) || !aligned(e->down, 16) || e->gate_up_stride % 16 || e->down_stride % 16)
    fail(w + ": weight regions and strides must be 16-byte aligned");
  if (!aligned(e->gate_up_scales, 2) || !aligned(e->down_scales, 2) || e->gate_up_scales_stride % 2 ||
      e->down_scales_stride % 2)
    fail(w + ": scale regions and strides must be 2-byte aligned");
}

static void validate_pair(const wm_mxfp4_experts* routed, const wm_mxfp4_experts* shared) {
  validate_experts(routed, "routed experts", false);
  if (routed->tiled && (routed->hidden % 128 || routed->inter % 128))
    fail("routed experts: the prefill tile layout needs hidden and intermediate multiples of 128");
  if (shared) {
    validate_experts(shared, "shared expert", true);
    if (shared->hidden != routed->hidden) fail("shared expert: hidden differs from the routed experts");
    if (shared->inter != routed->inter)
      fail("shared expert: intermediate must equal the routed experts' (one act buffer layout)");
    if ((shared->tiled != 0) != (routed->tiled != 0))
      fail("shared expert: the routed and shared tables must both be in the row layout or both tiled");
  }
}

static bool use_decode(int tokens, int k) { return (int64_t)tokens * k <= DECODE_MAX_PAIRS; }
// Tables in the prefill tile layout always take the grouped GEMM, and so do shapes the decode
// kernels do not take (above 16384).
static bool use_decode(int tokens, int k, const wm_mxfp4_experts& e) {
  return !e.tiled && use_decode(tokens, k) && decode_mxfp4_supports(e.hidden, e.inter);
}

static void validate_fp8(const wm_fp8_experts* e, const char* what, bool shared) {
  std::string w(what);
  if (!e) fail(w + ": expert table is null");
  if (!e->w13 || !e->w13_scales || !e->w2 || !e->w2_scales) fail(w + ": expert region pointer is null");
  if (e->hidden < 128 || e->hidden % 128) fail(w + ": hidden must be a positive multiple of 128");
  if (e->inter < 128 || e->inter % 128) fail(w + ": intermediate must be a positive multiple of 128");
  if (!shared && (e->experts < 1 || e->experts > 1024)) fail(w + ": expert count must be in 1..1024");
  if (e->w13_stride < 0 || e->w13_scales_stride < 0 || e->w2_stride < 0 || e->w2_scales_stride < 0)
    fail(w + ": negative stride");
  if (e->swiglu_limit < 0.0f) fail(w + ": swiglu_limit must be >= 0");
  if (e->scale_format != 0 && e->scale_format != 1)
    fail(w + ": scale_format must be 0 (fp32 128x128 blocks) or 1 (E8M0 32x32 blocks)");
  auto aligned = [](const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; };
  if (!aligned(e->w13, 16) || !aligned(e->w2, 16) || e->w13_stride % 16 || e->w2_stride % 16)
    fail(w + ": weight regions and strides must be 16-byte aligned");
  if (!aligned(e->w13_scales, 4) || !aligned(e->w2_scales, 4) || e->w13_scales_stride % 4 || e->w2_scales_stride % 4)
    fail(w + ": scale regions and strides must be 4-byte aligned");
}

static void validate_fp8_pair(const wm_fp8_experts* routed, const wm_fp8_experts* shared) {
  validate_fp8(routed, "routed experts", false);
  if (shared) {
    validate_fp8(shared, "shared expert", true);
    if (shared->hidden != routed->hidden || shared->inter != routed->inter)
      fail("shared expert: hidden and intermediate must equal the routed experts'");
    if ((shared->tiled != 0) != (routed->tiled != 0))
      fail("shared expert: the routed and shared tables must both be in the row layout or both tiled");
    if (shared->scale_format != routed->scale_format)
      fail("shared expert: the routed and shared tables must share a scale format");
  }
}

// The fused GEMV handles hidden / intermediate (multiples of 128) up to 8192 in the row
// layout; larger shapes, tables in the prefill tile layout and larger batches take the
// grouped GEMM.
static bool use_decode_fp8(int tokens, int k, const wm_fp8_experts& e) {
  return !e.tiled && use_decode(tokens, k) && e.hidden <= 8192 && e.inter <= 8192;
}

static size_t decode_workspace(int tokens, int k, const wm_mxfp4_experts& e) {
  return sizeof(float) * (size_t)(tokens * k + tokens) * e.inter;
}

// Scratch of the allocation-free entry point: the decode path's act rows live in this
// file-scope device array instead of a caller workspace. Each GPU holds its own copy for
// the life of the process. Host code never passes the array's name to a kernel (on the
// host it is only a stand-in for the symbol): the device address is looked up once per
// device with hipGetSymbolAddress, with that device current, and kept here.
constexpr size_t kNoAllocScratchBytes = (size_t)4 << 20;
__device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];
static void* g_scratch_ptr[64];
static std::mutex g_scratch_mu;

static void* scratch_for_current_device() {
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) fail("wm_moe_mxfp4_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    if (!ptr) fail("wm_moe_mxfp4_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = ptr;
  }
  return g_scratch_ptr[dev];
}

}  // namespace wm

using namespace wm;

extern "C" {

WM_EXPORT size_t wm_moe_mxfp4_workspace_size(int32_t tokens, int32_t k, const wm_mxfp4_experts* experts) {
  if (!experts || tokens < 0 || k < 1) return 0;
  if (use_decode(tokens, k, *experts)) return decode_workspace(tokens, k, *experts) + 256;
  return prefill_workspace_size(tokens, k, *experts, true) + 256;
}

WM_EXPORT int wm_moe_mxfp4(const void* x, int32_t tokens, const int32_t* indices, const float* weights, int32_t k,
                           const wm_mxfp4_experts* experts, const wm_mxfp4_experts* shared, const void* shared_gate,
                           void* y, void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_moe_mxfp4: negative token count");
    if (k < 1 || k > 32) fail("wm_moe_mxfp4: k must be in 1..32");
    validate_pair(experts, shared);
    if (tokens == 0) return;
    if (!x || !indices || !weights || !y) fail("wm_moe_mxfp4: null pointer");
    if (workspace_bytes < wm_moe_mxfp4_workspace_size(tokens, k, experts) - 256 || !workspace)
      fail("wm_moe_mxfp4: workspace too small");
    hipStream_t s = as_stream(stream);
    if (use_decode(tokens, k, *experts))
      decode_mxfp4((const uint16_t*)x, tokens, indices, weights, k, *experts, shared, (const uint16_t*)shared_gate,
                    (uint16_t*)y, true, (float*)workspace, s);
    else
      prefill_mxfp4((const uint16_t*)x, tokens, indices, weights, k, *experts, shared, (const uint16_t*)shared_gate,
                    (uint16_t*)y, true, workspace, workspace_bytes, s);
  });
}

WM_EXPORT size_t wm_moe_mxfp4_noalloc_max_bytes(void) { return kNoAllocScratchBytes; }

WM_EXPORT int wm_moe_mxfp4_noalloc(const void* x, int32_t tokens, const int32_t* indices, const float* weights,
                                   int32_t k, const wm_mxfp4_experts* experts, const wm_mxfp4_experts* shared,
                                   const void* shared_gate, void* y, void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_moe_mxfp4_noalloc: negative token count");
    if (k < 1 || k > 32) fail("wm_moe_mxfp4_noalloc: k must be in 1..32");
    validate_pair(experts, shared);
    if (tokens == 0) return;
    if (!x || !indices || !weights || !y) fail("wm_moe_mxfp4_noalloc: null pointer");
    if (!use_decode(tokens, k, *experts))
      fail("wm_moe_mxfp4_noalloc: only calls that take the decode path (tokens * k <= 256, row layout)");
    const size_t need = decode_workspace(tokens, k, *experts);
    if (need > kNoAllocScratchBytes)
      fail("wm_moe_mxfp4_noalloc: the call needs " + std::to_string(need) + " bytes of scratch, more than the " +
           std::to_string(kNoAllocScratchBytes) + " it has");
    void* ws = scratch_for_current_device();
    decode_mxfp4((const uint16_t*)x, tokens, indices, weights, k, *experts, shared, (const uint16_t*)shared_gate,
                 (uint16_t*)y, true, (float*)ws, as_stream(stream));
  });
}

WM_EXPORT int wm_experts_mxfp4(const void* x, int32_t tokens, const int32_t* indices, int32_t k,
                               const wm_mxfp4_experts* experts, void* out, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_experts_mxfp4: negative token count");
    if (k < 1 || k > 32) fail("wm_experts_mxfp4: k must be in 1..32");
    validate_pair(experts, nullptr);
    if (tokens == 0) return;
    if (!x || !indices || !out) fail("wm_experts_mxfp4: null pointer");
    if (workspace_bytes < wm_moe_mxfp4_workspace_size(tokens, k, experts) - 256 || !workspace)
      fail("wm_experts_mxfp4: workspace too small");
    hipStream_t s = as_stream(stream);
    if (use_decode(tokens, k, *experts))
      decode_mxfp4((const uint16_t*)x, tokens, indices, nullptr, k, *experts, nullptr, nullptr, (uint16_t*)out, false,
                   (float*)workspace, s);
    else
      prefill_mxfp4((const uint16_t*)x, tokens, indices, nullptr, k, *experts, nullptr, nullptr, (uint16_t*)out,
                    false, workspace, workspace_bytes, s);
  });
}

WM_EXPORT size_t wm_moe_fp8_workspace_size(int32_t tokens, int32_t k, const wm_fp8_experts* experts) {
  if (!experts || tokens < 0 || k < 1) return 0;
  if (use_decode_fp8(tokens, k, *experts))  // act rows, bf16
    return sizeof(uint16_t) * (size_t)(tokens * k + tokens) * experts->inter + 256;
  return prefill_fp8_workspace_size(tokens, k, *experts, true) + 256;
}

WM_EXPORT int wm_moe_fp8(const void* x, int32_t tokens, const int32_t* indices, const float* weights, int32_t k,
                         const wm_fp8_experts* experts, const wm_fp8_experts* shared, const void* shared_gate, void* y,
                         void* workspace, size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_moe_fp8: negative token count");
    if (k < 1 || k > 32) fail("wm_moe_fp8: k must be in 1..32");
    validate_fp8_pair(experts, shared);
    if (tokens == 0) return;
    if (!x || !indices || !weights || !y) fail("wm_moe_fp8: null pointer");
    if (workspace_bytes < wm_moe_fp8_workspace_size(tokens, k, experts) - 256 || !workspace)
      fail("wm_moe_fp8: workspace too small");
    hipStream_t s = as_stream(stream);
    if (use_decode_fp8(tokens, k, *experts))
      decode_fp8((const uint16_t*)x, tokens, indices, weights, k, *experts, shared, (const uint16_t*)shared_gate,
                 (uint16_t*)y, true, (uint16_t*)workspace, s);
    else
      prefill_fp8((const uint16_t*)x, tokens, indices, weights, k, *experts, shared, (const uint16_t*)shared_gate,
                  (uint16_t*)y, true, workspace, workspace_bytes, s);
  });
}

WM_EXPORT int wm_experts_fp8(const void* x, int32_t tokens, const int32_t* indices, int32_t k,
                             const wm_fp8_experts* experts, void* out, void* workspace, size_t workspace_bytes,
                             void* stream) {
  return guarded([&] {
    if (tokens < 0) fail("wm_experts_fp8: negative token count");
    if (k < 1 || k > 32) fail("wm_experts_fp8: k must be in 1..32");
    validate_fp8_pair(experts, nullptr);
    if (tokens == 0) return;
    if (!x || !indices || !out) fail("wm_experts_fp8: null pointer");
    if (workspace_bytes < wm_moe_fp8_workspace_size(tokens, k, experts) - 256 || !workspace)
      fail("wm_experts_fp8: workspace too small");
    hipStream_t s = as_stream(stream);
    if (use_decode_fp8(tokens, k, *experts))
      decode_fp8((const uint16_t*)x, tokens, indices, nullptr, k, *experts, nullptr, nullptr, (uint16_t*)out, false,
                 (uint16_t*)workspace, s);
    else
      prefill_fp8((const uint16_t*)x, tokens, indices, nullptr, k, *experts, nullptr, nullptr, (uint16_t*)out, false,
                  workspace, workspace_bytes, s);
  });
}

}  // extern "C"
