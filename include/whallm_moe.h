/* C interface of the MI355X (gfx950) MoE expert-path library, libwhallm_moe.so.
 *
 * Conventions (mirroring Native/QwenNative/capi.h:1-5 and capi.mm:20-37):
 *  - every entry point returns int: 0 on success, 1 on an error whose message
 *    wm_last_error() returns (per calling thread), 2 when the caller's cancel hook
 *    stopped the call; nothing is launched when an argument check fails; after a
 *    nonzero status of a call that carries state (a decode stack, a residual), that
 *    state must be reset before it is used again;
 *  - pointers are device pointers unless named host_*; sizes are element counts;
 *  - `stream` is a hipStream_t (NULL = the default stream); work is enqueued,
 *    not waited for. Outputs are caller-owned and valid once the stream reaches
 *    them; inputs must stay valid until then;
 *  - calls that share a workspace or a slot arena from more than one thread
 *    at a time race: one thread per handle / workspace, as in the reference.
 *
 * Weight layout (HBM): each expert is the reference's Qwen blob regions
 * (runtime/deepseek_v4_ssd/manifest.py:37-42): gate_up [2I, H/8] u32 words of
 * eight E2M1 nibbles (value i = nibble i % 8, low first), gate_up scales
 * [2I, H/32] E8M0 bytes, down [H, I/8] u32, down scales [H, I/32] u8.
 * An expert table locates expert e's regions at base + slot(e) * stride, which
 * covers both per-slot blobs (stride = blob size) and the region-major layer
 * buffers of expert_layout.py:83-119 (stride = region size).
 *
 * Expert ids and residency: a pair whose id is outside [0, experts) or whose slot map
 * entry is negative (an expert that is not resident) contributes nothing to a layer
 * output and gives a zero row in the per-pair (router order) outputs; a pair with a
 * negative id leaves its per-pair output row unwritten, so a layer can be run in two
 * calls over complementary pair masks (ready experts first, the rest after their fills).
 */
#ifndef WHALLM_MOE_H
#define WHALLM_MOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
#define WM_EXPORT __attribute__((visibility("default")))
extern "C" {
#else
#define WM_EXPORT
#endif

/* MXFP4 expert set. gate rows first (Qwen, qwen4_exp.py:816-818) unless up_first
 * (DeepSeek w13 = [w3; w1], expert_layout.py:43-51, model.py:516-523). */
typedef struct wm_mxfp4_experts {
  const void* gate_up;
  const void* gate_up_scales;
  const void* down;
  const void* down_scales;
  int64_t gate_up_stride;        /* bytes between consecutive slots */
  int64_t gate_up_scales_stride;
  int64_t down_stride;
  int64_t down_scales_stride;
  const int32_t* slots;          /* device map expert -> slot, or NULL for slot = expert */
  int32_t experts;               /* routed experts addressable through `slots` */
  int32_t hidden;                /* H: multiple of 32 */
  int32_t inter;                 /* I: multiple of 32 */
  int32_t up_first;
  float swiglu_limit;            /* 0: plain SwiGLU; > 0: clamped (deepseek_v41/moe.py:30-43) */
  int32_t tiled;                 /* 0: the reference's row layout; 1: prefill tile layout
                                    (wm_repack_prefill_mxfp4), grouped-GEMM path only */
  int32_t act_terms;             /* grouped GEMM's activation terms: 0 two E4M3 terms per
                                    32-value block (bf16-exact above 2^-13 of the block max,
                                    fp4 x fp8 MFMA rate); 1 two E2M3 terms (~7 significant bits
                                    of the block max, twice the MFMA rate for MXFP4 weights) */
} wm_mxfp4_experts;

/* FP8-E4M3 expert set. scale_format 0: fp32 128x128 block scales (the DeepSeek-V3 / MiMo
 * checkpoints, mimo/weights.py:17-43): w13 [2I, H] bytes (gate rows first unless up_first),
 * scales fp32 [ceil(2I/128), ceil(H/128)]; w2 [H, I] bytes, scales [ceil(H/128), ceil(I/128)].
 * scale_format 1: one E8M0 byte (2^(b-127)) per 32x32 block (the V4.1 release,
 * deepseek_v41/dequant.py:45-50; Native/DeepSeekNative/kernels.metal:17-28): scales u8
 * [2I/32, H/32] and [H/32, I/32]. H and I must be multiples of 128. */
typedef struct wm_fp8_experts {
  const void* w13;
  const void* w13_scales;
  const void* w2;
  const void* w2_scales;
  int64_t w13_stride, w13_scales_stride, w2_stride, w2_scales_stride;
  const int32_t* slots;
  int32_t experts;
  int32_t hidden;
  int32_t inter;
  int32_t up_first;
  float swiglu_limit;
  int32_t tiled;                 /* 0: the reference's row layout; 1: prefill tile layout of the
                                    weight bytes (wm_repack_prefill_fp8), grouped-GEMM path only */
  int32_t scale_format;          /* 0: fp32 128x128 blocks; 1: E8M0 32x32 blocks */
  int32_t act_terms;             /* as wm_mxfp4_experts.act_terms (fp8 x fp8 and fp8 x fp6 run at
                                    the same MFMA rate) */
} wm_fp8_experts;

/* Message of the last failed call on this thread ("" when none). */
WM_EXPORT const char* wm_last_error(void);
/* Library version string; no device work. */
WM_EXPORT const char* wm_version(void);

/* ---- formats --------------------------------------------------------------
 * out[r, i] = e2m1(nibble) * 2^(scale[r, i/32] - 127) as fp32 (bf16 when out_bf16);
 * scale byte 0 -> 2^-127 (a denormal), 255 -> NaN (OCP MX). Replaces the reference's unpack_fp4 /
 * dequant_fp4 / e8m0_to_float (deepseek_v41/dequant.py:33-68) and mx.dequantize. */
WM_EXPORT int wm_dequant_mxfp4(const void* packed, const void* scales, int64_t rows, int64_t cols,
                               void* out, int out_bf16, void* stream);
/* out[r, c] = e4m3(w[r, c]) * scales[r/128, c/128] (fp32); decode_fp8_blocks
 * (mimo/weights.py:17-43) without the bf16 rounding. */
WM_EXPORT int wm_dequant_fp8_blocks(const void* weight, const float* scales, int64_t rows, int64_t cols,
                                    float* out, void* stream);
/* out[r, c] = e4m3(w[r, c]) * 2^(scales[r/32, c/32] - 127) as fp32 (exact), scales E8M0 u8
 * [ceil(rows/32), ceil(cols/32)]: dequant_fp8 of the V4.1 release (deepseek_v41/dequant.py:45-50)
 * before its cast to the output dtype; e8m0_256 x fp8x4 of Native/DeepSeekNative/kernels.metal:17-28.
 * Scale byte 255 gives NaN (OCP MX). */
WM_EXPORT int wm_dequant_fp8_e8m0(const void* weight, const void* scales, int64_t rows, int64_t cols, float* out,
                                  void* stream);

/* ---- routing --------------------------------------------------------------
 * logits [T, E] fp32 -> indices [T, K] int32 (descending, ties -> lower index)
 * and weights [T, K] fp32 = softmax over the kept logits (norm_topk_prob) or the
 * full softmax probability; probabilities (nullable) receives the full softmax [T, E].
 * SparseMoE.route/_gates (qwen4_exp.py:1009-1046), native host top-k
 * (Native/QwenNative/engine.mm:2086-2100). E <= 1024, K <= 32. */
WM_EXPORT int wm_route_softmax_topk(const float* logits, int32_t tokens, int32_t experts, int32_t k,
                                    int32_t norm_topk_prob, int32_t* indices, float* weights, float* probabilities,
                                    void* stream);
/* DeepSeek routing: s = f(logits) (func 0 softmax, 1 sigmoid, 2 sqrt-softplus),
 * select on s + bias (bias may be NULL), w = s[idx] / (sum + 1e-20) * route_scale.
 * Gate.__call__ (deepseek_v41/moe.py:58-74), native route (Native/DeepSeekNative/engine.mm:1863-1889).
 * n_groups > 1 adds DeepSeek-V3 group-limited selection (no reference counterpart). */
WM_EXPORT int wm_route_scored(const float* logits, const float* bias, int32_t tokens, int32_t experts,
                              int32_t k, int32_t func, float route_scale, int32_t norm_topk_prob,
                              int32_t n_groups, int32_t topk_groups, int32_t* indices, float* weights,
                              void* stream);
/* logits[t, e] = x[t] . w[e] for bf16 x [T, H] and bf16 w [E, H], fp32 out: the
 * router linear (SparseMoE.gate, qwen4_exp.py:1000; linear_bf16,
 * Native/QwenNative/kernels.metal:18-67). 64+ tokens with hidden a multiple of 32 run on
 * bf16 MFMA (the GEMM of wm_norm_router); fewer run one wave per output. */
WM_EXPORT int wm_linear_bf16(const void* x, const void* w, int32_t tokens, int32_t hidden, int32_t outputs,
                             float* out, void* stream);

/* ---- permute --------------------------------------------------------------
 * Stable sort of the T*K (token, k) pairs by expert (mlx-lm _gather_sort as used at
 * qwen4_exp.py:865-868; native tile build Native/QwenNative/engine.mm:2104-2126).
 * order[r] = pair of permuted row r, inverse[p] = row of pair p, offsets[E+1],
 * tiles[n][2] = (expert, first row) of each tile_rows-row tile, tile_count[1].
 * max tiles = ceil(T*K / tile_rows) + E. workspace: wm_permute_workspace_size bytes. */
WM_EXPORT size_t wm_permute_workspace_size(int64_t pairs, int32_t experts);
WM_EXPORT int wm_permute(const int32_t* indices, int64_t pairs, int32_t experts, int32_t tile_rows,
                         int32_t* order, int32_t* inverse, int32_t* offsets, int32_t* tiles,
                         int32_t* tile_count, void* workspace, size_t workspace_bytes, void* stream);

/* ---- MXFP4 expert FFN -----------------------------------------------------
 * One MoE layer, Qwen form (SparseMoE.__call__, qwen4_exp.py:1015-1051):
 *   y[t] = sum_k weights[t,k] * FFN_{indices[t,k]}(x[t]) + sigmoid(x[t] . shared_gate) * FFN_shared(x[t])
 * x, y bf16 [T, H]; shared may be NULL (no shared term) and shared_gate NULL
 * (ungated shared expert, the DeepSeek form, model.py:540-541).
 * Decode path (fused dequant-GEMV) for T*K <= 256, MFMA grouped GEMM otherwise.
 * workspace: wm_moe_mxfp4_workspace_size bytes. */
WM_EXPORT size_t wm_moe_mxfp4_workspace_size(int32_t tokens, int32_t k, const wm_mxfp4_experts* experts);
WM_EXPORT int wm_moe_mxfp4(const void* x, int32_t tokens, const int32_t* indices, const float* weights,
                           int32_t k, const wm_mxfp4_experts* experts, const wm_mxfp4_experts* shared,
                           const void* shared_gate, void* y, void* workspace, size_t workspace_bytes,
                           void* stream);
/* wm_moe_mxfp4 without a workspace and without any allocation, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference. Its scratch (the decode path's act rows) is
 * a file-scope device array of wm_moe_mxfp4_noalloc_max_bytes() = 4 MiB per GPU, held until
 * the process ends; its address is looked up on a device's first call. Only calls that take
 * the decode path (tokens * k <= 256, row layout) and need at most that much scratch
 * (4 * (tokens * (k + 1)) * inter bytes) are accepted; others fail with a message. Every
 * call on one GPU shares its array, so calls that may overlap on one GPU (other streams,
 * other threads) race; calls ordered on one stream do not. Same results as wm_moe_mxfp4. */
WM_EXPORT size_t wm_moe_mxfp4_noalloc_max_bytes(void);
WM_EXPORT int wm_moe_mxfp4_noalloc(const void* x, int32_t tokens, const int32_t* indices, const float* weights,
                                   int32_t k, const wm_mxfp4_experts* experts, const wm_mxfp4_experts* shared,
                                   const void* shared_gate, void* y, void* stream);
/* Per-pair expert outputs in router order, out bf16 [T, K, H]: the
 * StreamingExperts.__call__ contract (qwen4_exp.py:853-904) and
 * _StreamingSwitchGLU.__call__ (model.py:325-385). Same workspace size. */
WM_EXPORT int wm_experts_mxfp4(const void* x, int32_t tokens, const int32_t* indices, int32_t k,
                               const wm_mxfp4_experts* experts, void* out, void* workspace,
                               size_t workspace_bytes, void* stream);
/* Prefill tile layout: writes every expert of src (resolved through src->slots) into the
 * caller's four device regions, one expert after another with the region sizes of the
 * row layout (2I*H/2, 2I*H/32, H*I/2, H*I/32 bytes), the same bytes reordered so that the
 * grouped GEMM reads each 16-row group's 128-wide K step as one contiguous KB and each
 * step's scale bytes of all rows as one run:
 *   weights [K/128 steps][rows/16 groups][4 x 16 bytes of the step][16 rows][16 bytes]
 *   scales  [K/128 steps][rows][4 E8M0 bytes of the step]
 * (gate_up: rows 2I, K = H; down: rows H, K = I; H and I multiples of 128). Describe the
 * result with slots = NULL, the region sizes as strides and tiled = 1; such a table always
 * takes the grouped-GEMM path. The counterpart of the reference's install-time expert blob
 * repack (Repacker.run / convert, Sources/DeepSeekRepack/Repacker.swift:17-124, :601-715),
 * for this GPU's loads. */
WM_EXPORT int wm_repack_prefill_mxfp4(const wm_mxfp4_experts* src, void* gate_up, void* gate_up_scales,
                                      void* down, void* down_scales, void* stream);

/* Combine of per-pair rows [T, K, H] bf16 in router order (the output of
 * wm_experts_mxfp4 / wm_experts_fp8): y[t] = sum_k weights[t, k] * rows[t, k] (+ add[t]),
 * fp32 in k order, bf16 out; add (nullable) bf16 [T, H], e.g. the gated shared expert.
 * SparseMoE._combine (qwen4_exp.py:1048-1051) and _route_reduce + shared (model.py:540-546).
 * rows, add and y 16-byte aligned, hidden a multiple of 8, k <= 64. */
WM_EXPORT int wm_combine_pairs(const void* rows, const float* weights, int32_t tokens, int32_t k, int32_t hidden,
                               const void* add, void* y, void* stream);

/* The reference's bf16 shared expert: y[t] = add[t] + g(t) * down(silu(x[t] gate_w^T) * (x[t] up_w^T)),
 * g(t) = sigmoid(x[t] . gate_vec) (1 when gate_vec is NULL), the act rounded to bf16 once.
 * MLP (qwen4_exp.py:763-771) with shared_expert_gate (:1002-1003, :1045); native
 * engine.mm:2075-2079. x [T, H], gate_w / up_w [I, H], down_w [H, I], gate_vec [H], add and y
 * [T, H], all bf16 and 16-byte aligned; add (nullable) may alias y. H and I multiples of
 * 32. Fewer than 64 tokens run two GEMV kernels, more the bf16 MFMA GEMM of wm_linear_bf16.
 * workspace: wm_mlp_bf16_workspace_size bytes. */
WM_EXPORT size_t wm_mlp_bf16_workspace_size(int32_t tokens, int32_t hidden, int32_t inter);
WM_EXPORT int wm_mlp_bf16(const void* x, int32_t tokens, int32_t hidden, int32_t inter, const void* gate_w,
                          const void* up_w, const void* down_w, const void* gate_vec, const void* add, void* y,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- FP8-E4M3 expert FFN (fp32 128x128 block scales) ----------------------
 * The DeepSeek-V3 expert format (runtime/deepseek_v4_ssd/mimo/weights.py:17-43):
 * SharedExpert / routed experts of deepseek_v41/moe.py:77-93, y = W2(swiglu(W1 x, W3 x)),
 * clamped when swiglu_limit > 0 (moe.py:30-43). Same contract as wm_moe_mxfp4 /
 * wm_experts_mxfp4 (shared_gate NULL = the ungated DeepSeek shared expert, model.py:540-541).
 * Fused dequant-GEMV for T*K <= 256 when hidden and intermediate are multiples of 1024;
 * grouped MFMA GEMM otherwise (multiples of 128). Replaces the FP8 expert linears
 * (Native/DeepSeekNative/kernels.metal:82-124) and the install-time FP8 decode
 * (Sources/DeepSeekRepack/Repacker.swift:622-627). */
WM_EXPORT size_t wm_moe_fp8_workspace_size(int32_t tokens, int32_t k, const wm_fp8_experts* experts);
WM_EXPORT int wm_moe_fp8(const void* x, int32_t tokens, const int32_t* indices, const float* weights, int32_t k,
                         const wm_fp8_experts* experts, const wm_fp8_experts* shared, const void* shared_gate,
                         void* y, void* workspace, size_t workspace_bytes, void* stream);
WM_EXPORT int wm_experts_fp8(const void* x, int32_t tokens, const int32_t* indices, int32_t k,
                             const wm_fp8_experts* experts, void* out, void* workspace, size_t workspace_bytes,
                             void* stream);
/* Prefill tile layout of FP8 weights: writes every expert of src (resolved through
 * src->slots) into the caller's four device regions, one expert after another with the
 * region sizes of the row layout (2I*H, 4*(2I/128)*(H/128), H*I, 4*(H/128)*(I/128) bytes):
 * the weight bytes reordered so that the grouped GEMM reads each 16-row group's 128-wide
 * K step as two contiguous KB, the block scales copied unchanged:
 *   weights [K/128 steps][rows/16 groups][8 x 16 bytes of the step][16 rows][16 bytes]
 * (w13: rows 2I, K = H; w2: rows H, K = I; H and I multiples of 128). Describe the result
 * with slots = NULL, the region sizes as strides and tiled = 1; such a table always takes
 * the grouped-GEMM path. The counterpart of the reference's install-time FP8 expert
 * repack (Sources/DeepSeekRepack/Repacker.swift:601-715), for this GPU's loads. */
WM_EXPORT int wm_repack_prefill_fp8(const wm_fp8_experts* src, void* w13, void* w13_scales, void* w2,
                                    void* w2_scales, void* stream);

/* ---- the prefill GEMMs' activation terms ------------------------------------
 * x [rows, hidden] bf16 (hidden a multiple of 128, 16-byte aligned) -> out [rows][hidden/128]
 * [208 bytes]: per 128-wide K step, for each of its four 32-value blocks the hi and the lo
 * E2M3 terms (32 six-bit fields each, field k at bits 6k..6k+5), then the four hi and the
 * four lo E8M0 exponents, then 8 bytes of padding (not written). hi = e2m3(x / 2^(s-127))
 * with the block maximum in [4, 8) at that scale; lo the same for the exact residual. No
 * counterpart in the reference: the format in which the grouped GEMMs read activations,
 * exposed so callers can prepare rows once and so the tests can check it byte for byte. */
WM_EXPORT int wm_split_rows_e2m3(const void* x, int32_t rows, int32_t hidden, void* out, void* stream);
/* x [rows, hidden] bf16 -> the grouped GEMM's bf16-exact split rows: terms [rows][hidden/128]
 * [256 bytes] (per 128-wide step the hi terms of K 0..127 in K order, then the lo terms) and
 * scales [rows][hidden/128] u32 (the step's 4 hi E8M0 bytes; the lo scale is hi - 4). Per
 * 32-value block hi = e4m3(x / 2^(s-127)), s = max(e(max |x|) - 7, 5), lo = e4m3((x /
 * 2^(s-127) - hi) * 16), round to nearest even. No counterpart in the reference (its
 * activations stay bf16 / fp32); exposed for the bit-exact test of the split. */
WM_EXPORT int wm_split_rows_e4m3(const void* x, int32_t rows, int32_t hidden, void* terms, void* scales, void* stream);

/* ---- measurement ----------------------------------------------------------
 * When enabled, every later wm_moe_mxfp4 / wm_experts_mxfp4 / wm_moe_fp8 / wm_experts_fp8
 * call that takes the grouped-GEMM path records events on its stream around the gate_up
 * and the down GEMM; wm_kernel_timing_ms waits for the latest call's events and returns
 * (gate_up ms, down ms). No counterpart in the reference (a benchmark hook; one set of
 * events per device, so concurrent calls overwrite each other's). */
WM_EXPORT int wm_set_kernel_timing(int enable);
WM_EXPORT int wm_kernel_timing_ms(float* out2);

/* ---- decode stack ---------------------------------------------------------
 * r[t] += y[t] (y nullable), x[t] = bf16(r[t] / sqrt(mean(r[t]^2) + eps)): the
 * pre-norm residual between MoE layers (DecoderLayer.feed_forward, qwen4_exp.py:1127-1149,
 * without attention). residual fp32 [T, H], y and x bf16 [T, H]. */
WM_EXPORT int wm_residual_rmsnorm(float* residual, const void* y, int32_t tokens, int32_t hidden, float eps,
                                  void* x, void* stream);
/* The step before the MoE fused into one launch: v = residual + y (y nullable),
 * x = bf16(v * rsqrt(mean(v^2) + eps) * norm_weight) (norm_weight nullable: unit),
 * logits[t, e] = x[t] . router[e] (fp32 [T, E]) and shared_logit[t] = x[t] . shared_gate
 * (both nullable together). residual_out (nullable, must not overlap residual) receives v.
 * bf16 y [T, H], norm_weight [H], router [E, H], shared_gate [H]; every pointer 16-byte
 * aligned, hidden a multiple of 8. router_packed (nullable) is the same rows from
 * wm_repack_router, router_packed_bytes its size; the prefill path (16+ tokens) then reads
 * it instead of router. Replaces the norm dispatch and the router / shared-gate linears
 * before the expert step (Native/QwenNative/engine.mm:2074-2079; SparseMoE.gate and
 * shared_expert_gate, qwen4_exp.py:1000-1003); routing follows with wm_route_softmax_topk or
 * wm_route_scored on the device. */
WM_EXPORT int wm_norm_router(const float* residual, const void* y, const void* norm_weight, int32_t tokens,
                             int32_t hidden, float eps, const void* router, int32_t experts, const void* shared_gate,
                             const void* router_packed, size_t router_packed_bytes, void* x,
                             float* residual_out, float* logits, float* shared_logit, void* stream);
/* The router rows (and the shared gate row when shared_gate is set) in the fragment order of
 * wm_norm_router's prefill GEMM: [ceil((E + gate) / 16) + gate][H / 32][64] x 16 bytes,
 * zero-padded rows (the spare group with a gate makes the size tell whether it is packed). A one-time repack, like the prefill tile layout of the experts (no reference
 * counterpart: the reference's router weight stays [E, H]). hidden a multiple of 32. */
WM_EXPORT size_t wm_router_packed_bytes(int32_t experts, int32_t hidden, int32_t has_gate);
WM_EXPORT int wm_repack_router(const void* router, const void* shared_gate, int32_t experts, int32_t hidden,
                               void* packed, void* stream);
/* `layers` MoE layers chained as x_l = rmsnorm(r_l), r_{l+1} = r_l + MoE_l(x_l), routing
 * from logits [layers, T, E] on the device (no host synchronisation; graph-capturable).
 * experts / shared / shared_gates are host arrays of `layers` entries (shared and
 * shared_gates nullable). The per-layer loop of the native engine
 * (Native/QwenNative/engine.mm:1567-1588, experts() at :2073-2236). x_out (nullable)
 * receives the last rmsnorm(r_L). cancel (nullable) is the reference's cancel callback
 * (wq_cancel_fn, Native/QwenNative/capi.h:36-37; Engine::set_cancel, engine.h:112-113):
 * it is called with cancel_context before each layer is enqueued, and a nonzero return
 * stops the call with status 2; the layers already enqueued still run, so the residual
 * must then be restored by the caller. */
WM_EXPORT size_t wm_moe_stack_mxfp4_workspace_size(int32_t tokens, int32_t k, const wm_mxfp4_experts* experts);
WM_EXPORT int wm_moe_stack_mxfp4(const float* logits, int32_t layers, int32_t tokens, int32_t k,
                                 int32_t norm_topk_prob, const wm_mxfp4_experts* experts,
                                 const wm_mxfp4_experts* shared, const void* const* shared_gates,
                                 float* residual, float eps, void* x_out, void* workspace,
                                 size_t workspace_bytes, int (*cancel)(void*), void* cancel_context,
                                 void* stream);

/* ---- persistent decode (one kernel per token through every layer) ----------
 * Per-layer descriptor of the persistent decode kernel. Routed experts keep the
 * reference gate_up region ([2I, H/8] u32 + [2I, H/32] u8 per expert); the down
 * region is repacked slice-major for it (wm_repack_down_slices): [8][H][I/16 bytes]
 * words and [8][H][I/256] scale bytes per expert, slice s holding columns
 * [s*I/8, (s+1)*I/8). The shared expert (one, always on) uses the same layouts and
 * is gated by sigmoid(x . shared_gate) (NULL gate: weight 1). */
typedef struct wm_decode_layer {
  const void* gate_up;
  const void* gate_up_scales;
  const void* down;               /* slice-major */
  const void* down_scales;        /* slice-major */
  int64_t gate_up_stride, gate_up_scales_stride, down_stride, down_scales_stride;
  const int32_t* slots;           /* NULL: slot = expert */
  const void* shared_gate_up;
  const void* shared_gate_up_scales;
  const void* shared_down;        /* slice-major */
  const void* shared_down_scales; /* slice-major */
  const void* shared_gate;        /* bf16 [H] or NULL */
} wm_decode_layer;

/* Repacks `experts` down regions from the reference row-major layout ([H, I/8] u32 +
 * [H, I/32] u8, consecutive experts `src_stride` / `src_scales_stride` bytes apart) into
 * the slice-major layout above (dst experts dense: H*I/2 and H*I/32 bytes apart). */
WM_EXPORT int wm_repack_down_slices(const void* src, const void* src_scales, int64_t src_stride,
                                    int64_t src_scales_stride, int32_t experts, int32_t hidden, int32_t inter,
                                    void* dst, void* dst_scales, void* stream);

/* Bytes of the persistent decode state (message buffers and per-workgroup epochs);
 * the caller zero-fills it once and passes the same buffer to every call. */
WM_EXPORT size_t wm_decode_state_size(int32_t layers, int32_t experts);
/* One token through `layers` MoE layers in one persistent launch of 256 workgroups
 * (8 XCDs x 32): x_l = rmsnorm(r_l); r_{l+1} = r_l + bf16(MoE_l(x_l)) with top-k
 * softmax routing from logits [layers, E] (fp32). layers_dev: device array of
 * wm_decode_layer. residual fp32 [H] in/out; x_out (nullable) bf16 rmsnorm(r_L).
 * Supports hidden 2048, inter 512, k <= 11, one token.
 * down_row_layout: 0 when every descriptor's down regions are slice-major
 * (wm_repack_down_slices), 1 when they are in the reference row layout (e.g. the blobs
 * of a slot cache, read in place).
 * cancel (nullable): an int32 the host may set while the launch runs (pinned host
 * memory, or device memory written from another stream); it is read once per layer,
 * and a nonzero value ends the launch after that layer with status 2 (the device
 * counterpart of the reference's per-layer cancel poll, Native/QwenNative/capi.h:36-37).
 * The launch runs asynchronously, so the outcome is in the state's status word
 * (wm_decode_status_offset): 0 done, 1 a message wait ran out, 2 cancelled, 3 a selected
 * expert is not resident (negative slot map entry; checked before any layer runs), 4 no
 * valid route (a layer's logits row has fewer than k selectable values, e.g. NaN logits;
 * checked before any layer runs).
 * A launch that ends with a nonzero status leaves residual and x_out unchanged; the
 * state must then be zero-filled again. Calls that share a state buffer must be
 * stream-ordered.
 * residual_trace (nullable): fp32 [layers, H] receives the residual after every layer
 * (row l = r_{l+1}), for per-layer verification; no counterpart in the reference. */
WM_EXPORT int wm_moe_decode_persistent_mxfp4(const float* logits, int32_t layers, int32_t experts, int32_t k,
                                             int32_t hidden, int32_t inter, const wm_decode_layer* layers_dev,
                                             float* residual, float eps, void* x_out, void* state,
                                             size_t state_bytes, int32_t down_row_layout, const int32_t* cancel,
                                             float* residual_trace, void* stream);
/* Byte offset of the state buffer's int32 status word (0 = healthy; see above). */
WM_EXPORT size_t wm_decode_status_offset(int32_t layers, int32_t experts);

/* One MoE decode layer for one token in one launch: x = bf16(rmsnorm(residual) * norm_weight)
 * (norm_weight nullable: unit), logits = x . router^T (bf16 [experts, hidden]), softmax top-k
 * (norm_topk_prob), y = sum_k w_k FFN_k(x) + sigmoid(x . shared_gate) FFN_shared(x) (shared and
 * shared_gate nullable; a null gate leaves the shared expert ungated), residual_out = residual
 * + bf16(y) (nullable; may alias residual). The decoder layer's MoE half between its attention
 * blocks, called once per layer (DecoderLayer.feed_forward -> SparseMoE, qwen4_exp.py:1146,
 * :1036-1051; the native engine's expert step with its router GEMV and shared gate,
 * Native/QwenNative/engine.mm:2073-2236). Optional outputs: y bf16 [hidden], x_out bf16
 * [hidden], logits_out fp32 [experts], indices_out int32 [k], weights_out fp32 [k].
 * Shapes with a fused kernel (hidden / intermediate 2048 / 512 and 1024 / 512, k <= 11) run
 * as one launch whose outcome is in the state's status word (wm_moe_layer_decode_status_offset:
 * 0 done, 1 a grid-wide wait ran out, 4 no valid route: fewer than k selectable logits, e.g.
 * NaN; after a nonzero status residual_out and y are not written and the state must be
 * zero-filled again); other shapes run norm_router, the router, the decode GEMV kernels and the
 * residual add (errors returned at once). state: wm_moe_layer_decode_state_size bytes,
 * zero-filled before the first call, reused by calls in stream order (one call at a time).
 * Tables in the row layout; experts <= 1024; vectors and router 16-byte aligned. */
WM_EXPORT size_t wm_moe_layer_decode_state_size(int32_t experts, int32_t hidden, int32_t inter, int32_t k);
WM_EXPORT size_t wm_moe_layer_decode_status_offset(int32_t experts, int32_t inter);
WM_EXPORT int wm_moe_layer_decode(const float* residual, float* residual_out, const void* norm_weight, float eps,
                                  const void* router, const void* shared_gate, int32_t experts, int32_t k,
                                  int32_t norm_topk_prob, const wm_mxfp4_experts* routed,
                                  const wm_mxfp4_experts* shared, void* y, void* x_out, float* logits_out,
                                  int32_t* indices_out, float* weights_out, void* state, size_t state_bytes,
                                  void* stream);
/* 1 when the current device runs block b of the persistent launch on XCC b % 8, so
 * messages read only within one XCD use XCD-local stores; 0 when it does not (the
 * persistent launch then uses device-scope stores throughout); -1 on error. Checked
 * once per device with a probe launch on `stream` (it allocates and synchronises; a
 * persistent launch into a stream being captured skips the probe and uses device-scope
 * stores unless this was called before). No counterpart in the reference (an MI355X
 * placement detail of the persistent decode). */
WM_EXPORT int wm_decode_xcd_local(void* stream);

/* ---- HBM expert slot cache ----------------------------------------------------
 * The reference's expert arena (Native/QwenNative/engine.mm:649-778; ExpertCache,
 * runtime/deepseek_v4_ssd/expert_cache.py:1465-1945) on MI355X: `slots` expert blobs of
 * blob_bytes (the Qwen blob, manifest.py:41-45: gate_up | gate_up scales | down |
 * down scales) in caller-owned device memory, filled from a caller-owned pinned host pool
 * [files][experts][blob_bytes] (hipHostMalloc; the stand-in for the SSD expert files).
 * Replacement: LFU (use count, then oldest stamp), never a slot handed out by the same
 * plan; use counts halve every max(8 * slots, 64) touches (ExpertArena::victim/touch).
 * Opaque handle; errors as in the reference's C ABI (capi.h): int status, message at
 * wm_slot_cache_error(handle). One thread per handle. */
typedef struct wm_slot_cache wm_slot_cache;
/* device_slots NULL: policy only (plan works, acquire fails; no device calls at all).
 * device_map (nullable): device int32 [files * experts], expert -> slot of each file,
 * refreshed by acquire for the experts it hands out (the `slots` of wm_mxfp4_experts).
 * Returns NULL on failure with the message in err. Replaces ExpertArena's constructor
 * (engine.mm:653-659) and ExpertCache's slot pool (expert_cache.py:488-610). */
WM_EXPORT wm_slot_cache* wm_slot_cache_open(int32_t slots, int64_t blob_bytes, int32_t files, int32_t experts,
                                            void* device_slots, int32_t* device_map, const void* host_pool,
                                            char* err, size_t err_size);
WM_EXPORT void wm_slot_cache_close(wm_slot_cache* cache);
WM_EXPORT const char* wm_slot_cache_error(const wm_slot_cache* cache);
/* Slots for experts[n] (host ids) of `file`; out_filled[i] = 1 where the expert was missing
 * and took a slot (ExpertArena::plan, engine.mm:679-707). No copies. Host arrays. */
WM_EXPORT int wm_slot_cache_plan(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                 int32_t* out_slots, int32_t* out_filled);
/* plan + fill the misses from the host pool with hipMemcpyAsync on the cache's copy stream
 * (ExpertArena::acquire/load, engine.mm:671-722; ExpertCache.get_many, expert_cache.py:1465-1530).
 * The copy stream waits for the work already on compute_stream; compute_stream then waits
 * for the fills, so work enqueued after this call sees the experts resident. */
WM_EXPORT int wm_slot_cache_acquire(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                    int32_t* out_slots, void* compute_stream);
/* Cached-first acquire (the native engine's ready-then-late pair order,
 * Native/QwenNative/engine.mm:2204-2234; ExpertCache.iter_ready, expert_cache.py:1541-1645):
 * plan as wm_slot_cache_acquire and enqueue the misses' fills on the copy stream (after the
 * work already on compute_stream), but do not make compute_stream wait for them.
 * out_ready[i] = 1 where the expert was already resident: work enqueued on compute_stream
 * right away may read those experts (no fill of the plan touches their slots), e.g. a layer
 * call whose other pairs are masked with id -1. wm_slot_cache_wait_fills then makes
 * compute_stream wait for the fills, after which the remaining pairs may run. An expert
 * whose slot an earlier acquire_ready is still filling (no wait_fills since) is not ready;
 * wm_slot_cache_acquire waits for such fills as well, even when every expert is a hit. */
WM_EXPORT int wm_slot_cache_acquire_ready(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                          int32_t* out_slots, int32_t* out_ready, void* compute_stream);
/* wm_slot_cache_acquire_ready for one call's pairs in the reference's order (the ready pairs
 * are submitted before the reads, Native/QwenNative/engine.mm:2204-2230): plans `experts`
 * (the call's unique ids, host), then on compute_stream splits the device pair ids
 * indices [pairs] into ready_indices (the id where its expert is ready, else -1) and
 * late_indices (the rest; device arrays of `pairs`), with no host -> device copy. The copy
 * stream is ordered after compute_stream's work up to the split, but the fills are held
 * back until wm_slot_cache_start_fills, so the caller enqueues its ready-pair kernels
 * first and they run under the copies; any later call on the cache (wm_slot_cache_wait_fills
 * included) starts held fills the caller has not started. A slot filled by an earlier
 * acquire_ready that no wait_fills has covered is not ready. Order: acquire_split, the
 * ready pairs, start_fills, wait_fills, the late pairs. At most 1024 experts. */
WM_EXPORT int wm_slot_cache_acquire_split(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                          int32_t* out_slots, int32_t* out_ready, const int32_t* indices,
                                          int64_t pairs, int32_t* ready_indices, int32_t* late_indices,
                                          void* compute_stream);
/* Enqueues the fills wm_slot_cache_acquire_split held back (no-op when there are none): the
 * reads the native engine submits after the ready pairs (engine.mm:2225-2231). */
WM_EXPORT int wm_slot_cache_start_fills(wm_slot_cache* cache);
WM_EXPORT int wm_slot_cache_wait_fills(wm_slot_cache* cache, void* compute_stream);
/* Route mode (ExpertCache with eviction_policy "route", expert_cache.py:1131-1181): scores
 * [files * experts] (host, the route policy's retention scores) and quotas [files] (its
 * per-file slot targets) are copied; later victims are the resident expert with the lowest
 * (tier, score, last access), tier 0 = files over quota (or the incoming file at quota),
 * never one handed out by the same plan. scores NULL returns to LFU. Call again after each
 * rebalance of the policy (RouteCachePolicy.rebalance, route_cache.py:68-95). */
WM_EXPORT int wm_slot_cache_set_route(wm_slot_cache* cache, const double* scores, const int32_t* quotas);
/* The whole file (experts * blob_bytes) from the host pool into device buffer dst with one
 * hipMemcpyAsync on the copy stream, after the work already on compute_stream (which may
 * still read dst): the reference's background whole-layer read into one of two layer
 * buffers (wait_layer / read_layer, engine.mm:1647-1661). */
WM_EXPORT int wm_slot_cache_read_layer(wm_slot_cache* cache, int32_t file, void* dst, void* compute_stream);
/* compute_stream waits for the last read_layer of `file`. */
WM_EXPORT int wm_slot_cache_wait_layer(wm_slot_cache* cache, int32_t file, void* compute_stream);
/* Prompt-tail seeding (seed_layer, engine.mm:1664-1678; hot_tail_experts,
 * qwen_streaming_policy.py:23-45): plan experts[n] of `file` in the given order (least
 * valuable first), set their use counts to uses[n] (nullable), and fill the misses from
 * `layer` (a device copy of the whole file, as read_layer writes it) device to device on the
 * copy stream; compute_stream then waits for them. out_slots[n] receives the slots. */
WM_EXPORT int wm_slot_cache_seed(wm_slot_cache* cache, int32_t file, const int32_t* experts, const int32_t* uses,
                                 int32_t n, const void* layer, int32_t* out_slots, void* compute_stream);
/* One plan over several files (layers): n_files requests, request r = counts[r] experts of
 * files[r], the experts (host ids) and out_slots concatenated in request order. Every slot
 * the plan hands out is protected from its own evictions, so all requested experts are
 * resident together afterwards, as one launch over several layers (the persistent decode
 * stack) needs. Fills and map refreshes as wm_slot_cache_acquire. */
WM_EXPORT int wm_slot_cache_acquire_files(wm_slot_cache* cache, int32_t n_files, const int32_t* files,
                                          const int32_t* counts, const int32_t* experts, int32_t* out_slots,
                                          void* compute_stream);
/* The listed experts (host ids, sorted and unique) of `file` from the host pool into dst at
 * their offsets in the file (blob e at e * blob_bytes), one copy per run of consecutive ids
 * of at most 32 blobs, on the copy stream after the work already on compute_stream; the
 * reference's prefill reads of the routed experts (expert_cache.py:2062-2085, batched by
 * contiguous_batches, qwen_streaming_policy.py:7-20). wm_slot_cache_wait_layer waits for it. */
WM_EXPORT int wm_slot_cache_read_experts(wm_slot_cache* cache, int32_t file, const int32_t* experts, int32_t n,
                                         void* dst, void* compute_stream);
/* Prompt-tail seeding (ExpertCache._seed_from_batched_layer, expert_cache.py:1399-1430, with
 * hot_tail_experts, qwen_streaming_policy.py:23-45): routes [rows, k] int32 on the device
 * (written on compute_stream) are ranked on the device: over the last 128 rows, experts by
 * count, then latest position, then id; the first `limit` that are not resident are copied
 * from `layer` (the file's device copy) into free slots only, the most valuable first when
 * free slots run short (a prediction never evicts a demand-loaded expert). Synchronises
 * compute_stream to read the ranking. out_experts / out_slots (host, limit entries) receive
 * the seeded experts, least valuable first, and *out_count their number. E <= 1024. */
WM_EXPORT int wm_slot_cache_seed_tail(wm_slot_cache* cache, int32_t file, const int32_t* routes, int64_t rows,
                                      int32_t k, int32_t limit, const void* layer, int32_t* out_experts,
                                      int32_t* out_slots, int32_t* out_count, void* compute_stream);
/* out5 = (hits, misses, bytes copied, blobs filled, copies issued) since open. */
WM_EXPORT int wm_slot_cache_stats(const wm_slot_cache* cache, int64_t* out5);

/* ---- the slot cache's route-history policy (route mode with its own scores) --------
 * The reference's RouteCachePolicy (runtime/deepseek_v4_ssd/route_cache.py:12-120) as used
 * by ExpertCache (expert_cache.py:1088-1181), files = layers: two decayed decode routing
 * rates per (layer, expert) (half-lives 16 and 256 tokens of the layer), the prompt's
 * routes as a prior of weight 0.1 fading as 2^(-t/32) with the request's decode tokens,
 * a per-layer read cost relative to the median layer (clipped to [0.5, 2]), retention
 * score = (0.75 short + 0.25 long + prior) * cost, slot quotas per layer by marginal
 * value; rebalanced every 16 * layers decode tokens, when a prefill phase ends and on
 * request. In route mode the cache evicts by these scores and quotas (see set_route);
 * wm_slot_cache_acquire / acquire_ready / acquire_files observe the requested ids as
 * routes of the current phase. top_k 0 turns route mode off. */
WM_EXPORT int wm_slot_cache_route_policy(wm_slot_cache* cache, int32_t top_k);
/* Routes of `file` (token-major, top_k ids a token) that did not go through an acquire,
 * e.g. a batched prefill that reads whole files (observe_batched_routes). */
WM_EXPORT int wm_slot_cache_route_observe(wm_slot_cache* cache, int32_t file, const int32_t* experts, int64_t n,
                                          int32_t prefill);
/* The phase of the routes observed next: prefill (1) or decode (0); leaving a prefill
 * rebalances (ExpertCache.trace_routes). */
WM_EXPORT int wm_slot_cache_route_phase(wm_slot_cache* cache, int32_t prefill);
/* A new prompt: its routes become the prior (ExpertCache.begin_route_request). */
WM_EXPORT int wm_slot_cache_route_begin_request(wm_slot_cache* cache);
/* One expert read's duration for `file`, in seconds (nonpositive or non-finite ignored). */
WM_EXPORT int wm_slot_cache_route_record_read(wm_slot_cache* cache, int32_t file, double seconds);
WM_EXPORT int wm_slot_cache_route_rebalance(wm_slot_cache* cache);
/* The policy's state, every pointer nullable: scores [files * experts], quotas [files],
 * the short and long decayed rates [files * experts] at each file's current token count,
 * tokens [2 * files] (decode tokens, then prompt tokens, per file), read_cost [files],
 * counters [2] = (rebalances, slot capacity). */
WM_EXPORT int wm_slot_cache_route_state(wm_slot_cache* cache, double* scores, int32_t* quotas, double* short_rates,
                                        double* long_rates, int64_t* tokens, double* read_cost, int64_t* counters);

/* ---- MTP acceptance ----------------------------------------------------------
 * Verify n draft tokens (n <= 15) against n + 1 target rows [n + 1, vocab] fp32.
 * out: device int32[2] = (accepted drafts, next token).
 * Greedy: Sampler.verify at temperature 0 (runtime/deepseek_v4_ssd/native_qwen.py:395-400;
 * dspark._verify, dspark.py:862-873): argmax ties go to the lower index, a NaN wins.
 * Rejection (native_qwen.py:401-408; dspark.py:875-898): target_logp / draft_logp are
 * log-probabilities; uniforms[n + 1] are the caller's draws (u_0..u_{n-1} the accept
 * tests, u_n the sampling draw, inverse CDF as numpy Generator.choice). A draft id
 * outside [0, vocab) counts as rejected. workspace: wm_mtp_workspace_size bytes,
 * 16-byte aligned. */
WM_EXPORT size_t wm_mtp_workspace_size(int32_t drafts, int32_t vocab);
WM_EXPORT int wm_mtp_verify_greedy(const float* target_logits, const int32_t* drafts, int32_t n_drafts,
                                   int32_t vocab, int32_t* out, void* workspace, size_t workspace_bytes,
                                   void* stream);
WM_EXPORT int wm_mtp_verify_rejection(const float* target_logp, const float* draft_logp, const int32_t* drafts,
                                      int32_t n_drafts, int32_t vocab, const float* uniforms, int32_t* out,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* ---- the verify round's expert half -----------------------------------------
 * The MTP verify call (wq_verify, Native/QwenNative/capi.h:57; native_qwen.py:604-656) for
 * the part on the expert path: `rows` = the accepted token and its drafts (<= 16) through
 * `layers` FP8 MoE layers, each x_l = bf16(rmsnorm(r_l)), scored routing of
 * router_logits[l] (fp32 [layers, rows, experts]) with biases[l] (host array of device
 * pointers, nullable; nullable entries), r_{l+1} = r_l + MoE_l(x_l) (tables[l] and
 * shared[l]: host arrays of `layers` tables; shared nullable), then logits = x_L . head^T
 * (bf16 head [vocab, hidden] -> fp32 [rows, vocab]) and greedy acceptance of drafts[rows - 1]
 * into acceptance (device int32[2] = accepted drafts, next token; Sampler.verify,
 * native_qwen.py:389-408). residual (fp32 [rows, hidden]) is updated in place. Routing:
 * k, func (0 softmax, 1 sigmoid, 2 sqrt-softplus), route_scale, n_groups / topk_groups as
 * wm_route_scored with normalised weights. Every step is a library kernel on `stream`, with
 * no host synchronisation. The attention half, the KV state, wq_draft and wq_commit are not
 * on the expert path. workspace: wm_verify_step_fp8_workspace_size bytes, 256-byte aligned. */
WM_EXPORT size_t wm_verify_step_fp8_workspace_size(int32_t rows, int32_t k, int32_t vocab,
                                                   const wm_fp8_experts* experts);
WM_EXPORT int wm_verify_step_fp8(int32_t layers, const float* router_logits, float* residual, int32_t rows,
                                 const wm_fp8_experts* tables, const wm_fp8_experts* shared,
                                 const float* const* biases, int32_t k, int32_t func, float route_scale,
                                 int32_t n_groups, int32_t topk_groups, float eps, const void* head, int32_t vocab,
                                 const int32_t* drafts, float* logits, int32_t* acceptance, void* workspace,
                                 size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif
