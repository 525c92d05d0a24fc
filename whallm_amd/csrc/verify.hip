// The MTP verify round's expert half as one C entry point: the drafts and the accepted token
// (M <= 16 rows) through L FP8 MoE layers with their pre-norm residual glue, the LM head, and
// greedy acceptance. The reference's verify call (wq_verify, Native/QwenNative/capi.h:57;
// native_qwen.py:604-656) runs the whole model on the rows, the experts through the pair path
// (engine.mm:869, :2198-2235), and the caller accepts with Sampler.verify
// (native_qwen.py:389-408); attention and the KV state (and so wq_draft / wq_commit) are not
// on the expert path. Here each layer l is
//   x_l = bf16(rmsnorm(r_l)),  (idx, w) = scored routing of the layer's router logits,
//   r_{l+1} = r_l + MoE_l(x_l),
// then logits = x_L . head^T (fp32) and (accepted drafts, next token). Every step is an
// existing library kernel on the caller's stream (no host synchronisation), so a call can be
// captured in a HIP graph.
#include <string>

#include "moe_internal.h"

using namespace wm;

namespace {

struct VerifyScratch {
  size_t x, y, idx, w, moe, mtp, total;
};

VerifyScratch verify_scratch(int32_t rows, int32_t hidden, int32_t k, int32_t vocab, const wm_fp8_experts* experts) {
  auto al = [](size_t n) { return (n + 255) & ~(size_t)255; };
  VerifyScratch s;
  size_t at = 0;
  s.x = at;   at += al((size_t)rows * hidden * 2);
  s.y = at;   at += al((size_t)rows * hidden * 2);
  s.idx = at; at += al((size_t)rows * k * 4);
  s.w = at;   at += al((size_t)rows * k * 4);
  s.moe = at; at += al(wm_moe_fp8_workspace_size(rows, k, experts));
  s.mtp = at; at += al(wm_mtp_workspace_size(rows - 1, vocab));
  s.total = at;
  return s;
}

void check_call(int rc, const char* what) {
  if (rc != 0) fail(std::string("wm_verify_step_fp8: ") + what + ": " + wm_last_error());
}

}  // namespace

extern "C" {

WM_EXPORT size_t wm_verify_step_fp8_workspace_size(int32_t rows, int32_t k, int32_t vocab,
                                                   const wm_fp8_experts* experts) {
  if (rows < 1 || rows > 16 || k < 1 || vocab < 1 || !experts) return 0;
  return verify_scratch(rows, experts->hidden, k, vocab, experts).total;
}

WM_EXPORT int wm_verify_step_fp8(int32_t layers, const float* router_logits, float* residual, int32_t rows,
                                 const wm_fp8_experts* tables, const wm_fp8_experts* shared,
                                 const float* const* biases, int32_t k, int32_t func, float route_scale,
                                 int32_t n_groups, int32_t topk_groups, float eps, const void* head, int32_t vocab,
                                 const int32_t* drafts, float* logits, int32_t* acceptance, void* workspace,
                                 size_t workspace_bytes, void* stream) {
  return guarded([&] {
    if (layers < 1 || !tables) fail("wm_verify_step_fp8: at least one layer table is required");
    if (rows < 1 || rows > 16) fail("wm_verify_step_fp8: rows must be in 1..16 (the token and up to 15 drafts)");
    if (!router_logits || !residual || !head || !logits || !acceptance || !workspace || (rows > 1 && !drafts))
      fail("wm_verify_step_fp8: null pointer");
    const int H = tables[0].hidden, E = tables[0].experts;
    for (int l = 0; l < layers; ++l)
      if (tables[l].hidden != H || tables[l].experts != E)
        fail("wm_verify_step_fp8: the layers' tables differ in hidden size or expert count");
    if (workspace_bytes < wm_verify_step_fp8_workspace_size(rows, k, vocab, &tables[0]) || (uintptr_t)workspace % 256)
      fail("wm_verify_step_fp8: workspace too small or not 256-byte aligned");
    const VerifyScratch s = verify_scratch(rows, H, k, vocab, &tables[0]);
    uint8_t* base = static_cast<uint8_t*>(workspace);
    void* x = base + s.x;
    void* y = base + s.y;
    int32_t* idx = reinterpret_cast<int32_t*>(base + s.idx);
    float* w = reinterpret_cast<float*>(base + s.w);
    const size_t moe_bytes = s.mtp - s.moe;
    check_call(wm_residual_rmsnorm(residual, nullptr, rows, H, eps, x, stream), "residual_rmsnorm");
    for (int l = 0; l < layers; ++l) {
      check_call(wm_route_scored(router_logits + (size_t)l * rows * E, biases ? biases[l] : nullptr, rows, E, k, func,
                                 route_scale, 1, n_groups, topk_groups, idx, w, stream),
                 "route_scored");
      check_call(wm_moe_fp8(x, rows, idx, w, k, &tables[l], shared ? &shared[l] : nullptr, nullptr, y, base + s.moe,
                            moe_bytes, stream),
                 "moe_fp8");
      check_call(wm_residual_rmsnorm(residual, y, rows, H, eps, x, stream), "residual_rmsnorm");
    }
    check_call(wm_linear_bf16(x, head, rows, H, vocab, logits, stream), "linear_bf16 (LM head)");
    check_call(wm_mtp_verify_greedy(logits, drafts, rows - 1, vocab, acceptance, base + s.mtp,
                                    s.total - s.mtp, stream),
               "mtp_verify_greedy");
  });
}

}  // extern "C"
