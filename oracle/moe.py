"""MoE expert-path arithmetic restated in numpy (test oracle only; see oracle/__init__.py).

Pinning (tests/test_oracle_moe.py):

* ``route_softmax_topk`` — brute-force sort on tiny inputs; the reference's tie
  KAT (runtime/tests/test_runtime.py:2680-2683); softmax-over-kept equals
  renormalised full softmax (the two forms in qwen4_exp.py:1038-1042 and
  Native/QwenNative/engine.mm:2091-2096).
* ``route_scored`` (DeepSeek sqrt-softplus / sigmoid / softmax with bias-select)
  — closed form on hand-built rows; bias selects but does not weight. Its scores
  are the build's stated fp32 arithmetic (``exp_f32``, ``log1p_f32``,
  ``score_f32``, the device's reduction order for softmax sums), so device and
  oracle select identical experts; that arithmetic is pinned against float64
  math to a few ulp over the whole input range and at special values (exp 0 = 1,
  exp ln 2 = 2, sigmoid 0 = 1/2, softplus 0 = ln 2, under/overflow edges).
  Group-limited selection (n_groups > 1) has no reference implementation:
  PARITY UNPINNED against the reference; pinned only by brute force over all
  group subsets on tiny E.
* ``permute`` — invariants of Scripts/diagnose_qwen_grouped_experts.py:34-40
  (permutation, stable per-expert token order, inverse round trip) and the
  wave/pair tests of runtime/tests/portable/test_qwen_flash_portable.py:32-92.
* ``expert_ffn`` / ``moe_layer`` — constant-valued MXFP4 experts with a closed
  form (the reference's own test shape, runtime/tests/test_runtime.py:2507-2745),
  and a float64 per-pair loop on small shapes.
* ``verify_greedy`` / ``verify_rejection`` — the reference's distribution test
  (runtime/tests/test_native_qwen.py:71-87) and hand cases.
* ``SlotArena`` — state-machine cases read off Native/QwenNative/engine.mm:679-778.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .formats import dequant_mxfp4, dequant_fp8_blocks, dequant_fp8_e8m0, bf16_round_f32


# ----------------------------------------------------------------------------- routing

def topk_desc(scores: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest values per row, descending, ties -> lower index.

    The reference has no single rule: the Qwen native engine partial-sorts fp32
    logits (Native/QwenNative/engine.mm:2086-2090), MLX uses an unordered
    argpartition (qwen4_exp.py:1012), DeepSeek breaks ties toward the lower
    index (Native/DeepSeekNative/engine.mm:1881, model.py:590-602). This build
    fixes: value descending, ties to the lower index.
    """
    s = np.asarray(scores, np.float32)
    if np.isnan(s).any():
        raise ValueError("router scores contain NaN")
    order = np.argsort(-s, axis=-1, kind="stable")
    return order[..., :k].astype(np.int32)


def route_softmax_topk(logits: np.ndarray, k: int, norm_topk_prob: bool = True):
    """Qwen router: p = softmax(l); idx = topk(p, k); w = p[idx] (/ sum if norm).

    SparseMoE.route/_gates (qwen4_exp.py:1009-1046); the native engine's form
    exp(l_k - l_max) / sum_kept (Native/QwenNative/engine.mm:2091-2096) is the
    same quantity. Top-k is taken on the fp32 logits (monotone in p). Returns
    (indices int32 [T, k], weights float32 [T, k]); weights computed in float64.
    """
    l = np.asarray(logits, np.float32)
    idx = topk_desc(l, k)
    ld = l.astype(np.float64)
    top = ld.max(axis=-1, keepdims=True)
    e = np.exp(ld - top)
    kept = np.take_along_axis(e, idx, axis=-1)
    if norm_topk_prob:
        w = kept / kept.sum(axis=-1, keepdims=True)
    else:
        w = kept / e.sum(axis=-1, keepdims=True)
    return idx, w.astype(np.float32)


# The router's score arithmetic, stated in fp32 operations (each rounded to nearest even,
# no fused multiply-add) so that the device kernel (route_device.h) computes the same bits:
#   exp_f32(x):   n = rint(x log2e); r = (x - n ln2_hi) - n ln2_lo; p = degree-7 Taylor
#                 polynomial of e^r by Horner; e^x = p 2^n (0 when n < -125, +inf when n > 128);
#   log1p_f32(u): u in [0, 1]: m = 1 + u, halved when above sqrt 2 (k = 1); s = (m - 1)/(m + 1);
#                 ln m = k ln2 + 2 s (1 + z/3 + ... + z^5/11), z = s^2, plus the rounding
#                 correction (u - (m - 1)) / m;
#   sigmoid:      1 / (1 + exp_f32(-l));
#   sqrt-softplus: sqrt(max(l, 0) + log1p_f32(exp_f32(-|l|))), and exp_f32(l / 2) below l = -64;
#   softmax:      exp_f32(l - max) / sum, the sum in the device's wave order (softmax_sums_f32).
F32 = np.float32
LOG2E = F32(1.4426950408889634)
LN2_HI = F32(0.693145751953125)       # 0x3F317200: n * LN2_HI is exact for |n| <= 256
LN2_LO = F32(0.6931471805599453 - 0.693145751953125)
SQRT2 = F32(1.4142135623730951)
EXP_POLY = [F32(1.0 / f) for f in (1, 1, 2, 6, 24, 120, 720, 5040)]   # 1/j! for j = 0..7
ATANH_POLY = [F32(1.0 / j) for j in (1, 3, 5, 7, 9, 11)]


def exp_f32(x) -> np.ndarray:
    x = np.asarray(x, F32)
    with np.errstate(invalid="ignore", over="ignore"):
        n = np.rint(x * LOG2E)
        r = (x - n * LN2_HI) - n * LN2_LO
        p = EXP_POLY[7]
        for c in reversed(EXP_POLY[:7]):
            p = p * r + c
        ni = np.where(np.isfinite(n), n, 0).astype(np.int32)
        out = np.ldexp(p, ni).astype(F32)
    out = np.where(n > 128, F32(np.inf), out)
    out = np.where(n < -125, F32(0.0), out)
    return np.where(np.isnan(x), F32(np.nan), out).astype(F32)


def log1p_f32(u) -> np.ndarray:
    u = np.asarray(u, F32)
    m = F32(1.0) + u
    k = m > SQRT2
    m2 = np.where(k, m * F32(0.5), m)
    s = (m2 - F32(1.0)) / (m2 + F32(1.0))
    z = s * s
    p = ATANH_POLY[5]
    for c in reversed(ATANH_POLY[:5]):
        p = p * z + c
    lg = (s + s) * p
    corr = (u - (m - F32(1.0))) / m
    kf = k.astype(F32)
    return (kf * LN2_HI + (kf * LN2_LO + (lg + corr))).astype(F32)


def score_f32(logits: np.ndarray, func: str) -> np.ndarray:
    """The router's scores in the stated fp32 arithmetic (sigmoid, sqrt-softplus, softmax)."""
    l = np.asarray(logits, F32)
    if func == "sigmoid":
        return (F32(1.0) / (F32(1.0) + exp_f32(-l))).astype(F32)
    if func == "sqrtsoftplus":
        sp = np.maximum(l, F32(0.0)) + log1p_f32(exp_f32(-np.abs(l)))
        return np.where(l < F32(-64.0), exp_f32(F32(0.5) * l), np.sqrt(sp)).astype(F32)
    if func == "softmax":
        top = l.max(axis=-1, keepdims=True)
        e = exp_f32(l - top)
        return (e / softmax_sums_f32(e)[..., None]).astype(F32)
    raise ValueError(f"unknown score function {func!r}")


def softmax_sums_f32(e: np.ndarray) -> np.ndarray:
    """Row sums of e [.., E] in the router wave's order: lane j < 64 adds e[j], e[64 + j],
    ... in turn; then pairs of lanes (j, j ^ 1), quads (j ^ 2), eights (mirrored in each
    half row), sixteens (mirrored in each row), and the four rows as (r0 + r1) + (r2 + r3)."""
    e = np.asarray(e, F32)
    E = e.shape[-1]
    per = (E + 63) // 64
    pad = np.zeros(e.shape[:-1] + (per * 64,), F32)
    pad[..., :E] = e
    lanes = pad.reshape(e.shape[:-1] + (per, 64))
    v = lanes[..., 0, :].copy()
    for r in range(1, per):
        v = v + lanes[..., r, :]
    j = np.arange(64)
    for partner in (j ^ 1, j ^ 2, (j & ~7) | (7 - (j & 7)), (j & ~15) | (15 - (j & 15))):
        v = v + v[..., partner]
    return ((v[..., 0] + v[..., 16]) + (v[..., 32] + v[..., 48])).astype(F32)


def score_function(logits: np.ndarray, func: str) -> np.ndarray:
    """DeepSeek gate scores (deepseek_v41/moe.py:61-67; native sqrt-softplus at
    Native/DeepSeekNative/engine.mm:1875-1876), float64."""
    l = np.asarray(logits, np.float64)
    if func == "softmax":
        e = np.exp(l - l.max(axis=-1, keepdims=True))
        return e / e.sum(axis=-1, keepdims=True)
    if func == "sigmoid":
        return 1.0 / (1.0 + np.exp(-l))
    if func == "sqrtsoftplus":
        return np.sqrt(np.maximum(l, 0.0) + np.log1p(np.exp(-np.abs(l))))
    raise ValueError(f"unknown score function {func!r}")


def route_scored(logits: np.ndarray, bias: np.ndarray | None, k: int, func: str = "sigmoid",
                 route_scale: float = 1.0, norm_topk_prob: bool = True,
                 n_groups: int = 1, topk_groups: int = 1):
    """DeepSeek-style routing: the bias picks the experts but does not weight them.

    Gate.__call__ (deepseek_v41/moe.py:58-74): s = f(l) in the stated fp32 arithmetic
    (score_f32); selection on the fp32 s + bias; w = s[idx] / (sum + 1e-20) * route_scale
    (float64 sum). With n_groups > 1, the DeepSeek-V3
    group-limited rule (not in the reference): a group's score is the sum of
    its two largest biased scores, the topk_groups best groups are kept, and
    top-k runs over their experts. Ties go to the lower index (group or expert).
    """
    s = score_f32(logits, func)
    biased32 = (s + (F32(0.0) if bias is None else np.asarray(bias, F32))).astype(F32)
    T, E = biased32.shape
    if n_groups > 1:
        if E % n_groups:
            raise ValueError("experts must divide into groups")
        g = biased32.reshape(T, n_groups, E // n_groups)
        two = -np.sort(-g, axis=-1)[..., :2]
        group_scores = (two[..., 0].astype(np.float32) + two[..., 1].astype(np.float32)).astype(np.float32)
        keep = topk_desc(group_scores, topk_groups)
        mask = np.ones((T, n_groups), bool)
        np.put_along_axis(mask, keep, False, axis=-1)
        biased32 = np.where(np.repeat(mask, E // n_groups, axis=-1), np.float32(-np.inf), biased32)
    idx = topk_desc(biased32, k)
    w = np.take_along_axis(s, idx, axis=-1).astype(np.float64)
    if norm_topk_prob and k > 1:
        w = w / (w.sum(axis=-1, keepdims=True) + 1e-20)
    return idx, (w * route_scale).astype(np.float32)


# ----------------------------------------------------------------------------- permute

@dataclass
class Permutation:
    order: np.ndarray      # [P] pair index t*K+k at each permuted row
    inverse: np.ndarray    # [P] permuted row of each pair
    offsets: np.ndarray    # [E+1] first permuted row of each expert
    tiles: np.ndarray      # [n_tiles, 2] (expert, first permuted row) of each row tile


def permute(indices: np.ndarray, experts: int, tile_rows: int = 128) -> Permutation:
    """Stable sort of the flattened (token, k) pairs by expert.

    mlx-lm _gather_sort as restated at Scripts/diagnose_qwen_grouped_experts.py:34-40
    (order = argsort(flat), inverse = argsort(order)) with the stability of the
    native tile build (std::stable_sort, Native/QwenNative/engine.mm:2104-2126);
    per-expert row tiles of ``tile_rows`` as the native 16-row tiles
    (:2111-2122), described by (expert, first row) instead of padded row lists.
    """
    flat = np.asarray(indices).reshape(-1)
    if flat.size and (flat.min() < 0 or flat.max() >= experts):
        raise ValueError("expert ID is outside the model")
    order = np.argsort(flat, kind="stable").astype(np.int32)
    inverse = np.empty_like(order)
    inverse[order] = np.arange(order.size, dtype=np.int32)
    counts = np.bincount(flat, minlength=experts).astype(np.int32)
    offsets = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    tiles = [(e, offsets[e] + r) for e in range(experts) for r in range(0, counts[e], tile_rows)]
    return Permutation(order, inverse, offsets, np.array(tiles, np.int32).reshape(-1, 2))


# ----------------------------------------------------------------------------- expert FFN

def silu(x: np.ndarray) -> np.ndarray:
    return x / (1.0 + np.exp(-x))


@dataclass
class MXFP4Expert:
    """One expert in the reference's Qwen blob regions (manifest.py:37-42):
    gate_up [2I, H/8] u32 + [2I, H/32] u8 with gate rows 0..I-1 and up rows
    I..2I-1 (qwen4_exp.py:816-818), down [H, I/8] u32 + [H, I/32] u8."""
    gate_up: np.ndarray
    gate_up_scales: np.ndarray
    down: np.ndarray
    down_scales: np.ndarray


def expert_ffn(x: np.ndarray, e: MXFP4Expert, limit: float = 0.0, up_first: bool = False) -> np.ndarray:
    """fp32 dequant-then-matmul expert: silu(x Wg^T) * (x Wu^T) then @ Wd^T.

    StreamingExperts._one (qwen4_exp.py:815-818). With ``up_first`` the fused
    projection is DeepSeek's w13 = [w3 (up); w1 (gate)] (model.py:516-523,
    expert_layout.py:43-51). ``limit`` > 0 is the clamped SwiGLU
    (deepseek_v41/moe.py:30-43): up clamped to +-limit, gate clamped above.
    """
    wgu = dequant_mxfp4(e.gate_up, e.gate_up_scales)
    wd = dequant_mxfp4(e.down, e.down_scales)
    return ffn_dense(np.asarray(x, np.float32), wgu, wd, limit, up_first)


def ffn_dense(x: np.ndarray, wgu: np.ndarray, wd: np.ndarray, limit: float = 0.0,
              up_first: bool = False) -> np.ndarray:
    I = wgu.shape[0] // 2
    proj = x.astype(np.float32) @ wgu.T
    if up_first:
        up, gate = proj[..., :I], proj[..., I:]
    else:
        gate, up = proj[..., :I], proj[..., I:]
    if limit > 0:
        up = np.clip(up, -limit, limit)
        gate = np.minimum(gate, limit)
    return (silu(gate) * up).astype(np.float32) @ wd.T


def ffn_dense_bf16_steps(x: np.ndarray, wgu: np.ndarray, wd: np.ndarray, up_first: bool = False,
                         limit: float = 0.0, fp32_swiglu: bool = False, round_act: bool = True,
                         round_out: bool = True, rnd=bf16_round_f32) -> np.ndarray:
    """The reference's own arithmetic for one expert on bf16 activations, where every array op
    returns its inputs' dtype (MLX), so the fp32-accumulated projections come back as bf16:
    - Qwen (StreamingExperts._one, qwen4_exp.py:815-818, _qmm :774-783): the gate/up
      projection, sigmoid(gate), gate * sigmoid(gate) (nn.silu), its product with up and the
      down projection are each rounded to bf16;
    - DeepSeek V4.1 (``fp32_swiglu``, deepseek_v41/moe.py:36-44, :80-88): the bf16 gate/up
      projections are cast to fp32 and the clamped SwiGLU runs in fp32; the routed experts'
      down projection takes that fp32 input (``round_act``/``round_out`` False), the shared
      expert casts it back to bf16 first and returns bf16.
    Used to measure how far the reference itself sits from exact arithmetic; ``rnd`` is the
    rounding (identity gives ffn_dense)."""
    I = wgu.shape[0] // 2
    proj = rnd((x.astype(np.float32) @ wgu.T).astype(np.float32))
    gate, up = (proj[..., I:], proj[..., :I]) if up_first else (proj[..., :I], proj[..., I:])
    if limit > 0:
        up = np.clip(up, -limit, limit)
        gate = np.minimum(gate, limit)
    if fp32_swiglu:
        act = (silu(gate.astype(np.float64)) * up).astype(np.float32)
    else:
        sig = rnd((1.0 / (1.0 + np.exp(-gate.astype(np.float64)))).astype(np.float32))
        act = rnd(rnd((gate * sig).astype(np.float32)) * up)
    if round_act:
        act = rnd(act)
    out = (act.astype(np.float32) @ wd.T).astype(np.float32)
    return rnd(out) if round_out else out


def expert_ffn_bf16_steps(x: np.ndarray, e: MXFP4Expert, rnd=bf16_round_f32) -> np.ndarray:
    """expert_ffn with the reference's bf16 rounding points (ffn_dense_bf16_steps)."""
    return ffn_dense_bf16_steps(np.asarray(x, np.float32), dequant_mxfp4(e.gate_up, e.gate_up_scales),
                                dequant_mxfp4(e.down, e.down_scales), rnd=rnd)


def combine_bf16_steps(routed: np.ndarray, weights: np.ndarray, shared: np.ndarray | None = None,
                       shared_gate: np.ndarray | None = None, rnd=bf16_round_f32) -> np.ndarray:
    """combine with the reference's bf16 rounding points: the scores cast to the rows' dtype,
    each weighted row rounded, the sum over k accumulated in fp32 and rounded
    (SparseMoE._combine, qwen4_exp.py:1048-1051); sigmoid(gate logit) and its product with
    the shared row rounded, then the final add (_gates, :1045). ``routed``/``shared`` are the
    bf16 rows; ``rnd`` identity gives combine up to float32 rounding."""
    w = rnd(np.asarray(weights, np.float32))
    y = rnd((rnd(np.asarray(routed, np.float32) * w[..., None])).astype(np.float32).sum(axis=-2, dtype=np.float32))
    if shared is not None:
        s = np.asarray(shared, np.float32)
        if shared_gate is not None:
            g = rnd(np.asarray(shared_gate, np.float32).reshape(-1, 1))
            s = rnd(rnd((1.0 / (1.0 + np.exp(-g.astype(np.float64)))).astype(np.float32)) * s)
        y = rnd(y + s)
    return y.astype(np.float32)


@dataclass
class FP8Expert:
    """DeepSeek-style FP8 expert: w1 (gate) / w3 (up) [I, H] and w2 [H, I] E4M3 bytes with
    fp32 128x128 block scales (scale_format 0, mimo/weights.py:17-43) or E8M0 32x32 block
    scales (scale_format 1, the V4.1 release, deepseek_v41/dequant.py:45-50)."""
    w1: np.ndarray
    w1_scales: np.ndarray
    w3: np.ndarray
    w3_scales: np.ndarray
    w2: np.ndarray
    w2_scales: np.ndarray
    scale_format: int = 0


def fp8_expert_ffn(x: np.ndarray, e: FP8Expert, limit: float = 0.0) -> np.ndarray:
    """SharedExpert / routed expert of deepseek_v41/moe.py:77-93 in fp32."""
    deq = dequant_fp8_e8m0 if e.scale_format == 1 else dequant_fp8_blocks
    w1 = deq(e.w1, e.w1_scales)
    w3 = deq(e.w3, e.w3_scales)
    w2 = deq(e.w2, e.w2_scales)
    return ffn_dense(x, np.concatenate([w1, w3], axis=0), w2, limit, up_first=False)


def fp8_expert_ffn_bf16_steps(x: np.ndarray, e: FP8Expert, limit: float = 0.0, shared: bool = False,
                              rnd=bf16_round_f32) -> np.ndarray:
    """fp8_expert_ffn with the reference's rounding points (ffn_dense_bf16_steps, DeepSeek
    form): a routed expert returns fp32 rows, the shared expert bf16 (deepseek_v41/moe.py:80-88,
    :101-104)."""
    deq = dequant_fp8_e8m0 if e.scale_format == 1 else dequant_fp8_blocks
    wgu = np.concatenate([deq(e.w1, e.w1_scales), deq(e.w3, e.w3_scales)], axis=0)
    return ffn_dense_bf16_steps(np.asarray(x, np.float32), wgu, deq(e.w2, e.w2_scales), limit=limit,
                                fp32_swiglu=True, round_act=shared, round_out=shared, rnd=rnd)


def routed_outputs(x: np.ndarray, indices: np.ndarray, experts, ffn=expert_ffn, **kw) -> np.ndarray:
    """StreamingExperts.__call__ contract (qwen4_exp.py:853-904): per-pair expert
    outputs [T, K, H] in router order, grouped by expert for the math
    (the grouped/ungrouped equivalence of runtime/tests/test_qwen_grouped_experts.py:23-45)."""
    x = np.asarray(x, np.float32).reshape(-1, x.shape[-1])
    idx = np.asarray(indices).reshape(x.shape[0], -1)
    T, K = idx.shape
    flat = idx.reshape(-1)
    out = None
    for expert in np.unique(flat):
        positions = np.flatnonzero(flat == expert)
        y = ffn(x[positions // K], experts[int(expert)], **kw)
        if out is None:
            out = np.zeros((T * K, y.shape[-1]), np.float32)
        out[positions] = y
    if out is None:
        return np.zeros((T, K, x.shape[-1]), np.float32)
    return out.reshape(T, K, -1)


def combine(routed: np.ndarray, weights: np.ndarray, shared: np.ndarray | None = None,
            shared_gate: np.ndarray | None = None) -> np.ndarray:
    """y[t] = sum_k w[t,k] * routed[t,k] + sigmoid(g[t]) * shared[t].

    SparseMoE._combine (qwen4_exp.py:1048-1051) with the shared term of
    _gates (:1045); moe_combine (Native/QwenNative/kernels.metal:185-194).
    ``shared_gate`` None means an ungated shared expert (DeepSeek, model.py:540-541).
    Accumulated in float64, returned float32.
    """
    y = (np.asarray(routed, np.float64) * np.asarray(weights, np.float64)[..., None]).sum(axis=-2)
    if shared is not None:
        s = np.asarray(shared, np.float64)
        if shared_gate is not None:
            s = s / (1.0 + np.exp(-np.asarray(shared_gate, np.float64).reshape(-1, 1)))
        y = y + s
    return y.astype(np.float32)


def moe_layer(x: np.ndarray, logits: np.ndarray, experts, k: int, shared=None,
              shared_gate_weight: np.ndarray | None = None, norm_topk_prob: bool = True):
    """Whole Qwen-style MoE layer: route, routed experts, gated shared expert, combine.

    SparseMoE.__call__ (qwen4_exp.py:1015-1018). ``x`` is the bf16 input as
    float32 [T, H]; ``logits`` fp32 [T, E]; ``shared_gate_weight`` bf16 [H] as
    float32 (shared_expert_gate, :1003). Returns (y [T, H] f32, indices, weights).
    """
    idx, w = route_softmax_topk(logits, k, norm_topk_prob)
    routed = routed_outputs(x, idx, experts)
    sh = sg = None
    if shared is not None:
        sh = expert_ffn(np.asarray(x, np.float32), shared)
        if shared_gate_weight is not None:
            sg = np.asarray(x, np.float64) @ np.asarray(shared_gate_weight, np.float64)
    return combine(routed, w, sh, sg), idx, w


def rms_norm(r: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """Unit-weight RMSNorm, rounded to bf16: the pre-norm glue between MoE layers
    of the decode stack (a decoder layer's post-attention norm with the
    attention half removed)."""
    r = np.asarray(r, np.float64)
    inv = 1.0 / np.sqrt((r * r).mean(axis=-1, keepdims=True) + eps)
    return bf16_round_f32((r * inv).astype(np.float32))


def norm_router(r: np.ndarray, y: np.ndarray | None, router: np.ndarray, shared_gate: np.ndarray | None = None,
                norm_weight: np.ndarray | None = None, eps: float = 1e-6):
    """The step before the MoE: v = r + y (fp32 add), x = bf16(v / rms(v) * w_norm), router
    logits x @ router^T and the shared gate logit x @ g (float64 sums, returned float32).

    The norm is GroupRMSNorm's fp32 path (qwen4_exp.py:93-117, normalized * weight then
    cast) / kernels.metal rms_norm (Native/QwenNative/kernels.metal:73-91); the linears are
    SparseMoE.gate and shared_expert_gate (qwen4_exp.py:1000-1003), run by the native engine
    right before the expert step (Native/QwenNative/engine.mm:2074-2079). ``y``, ``router``,
    ``shared_gate`` and ``norm_weight`` are bf16 values as float32. Returns (v, x, logits,
    shared_logit or None)."""
    v = np.asarray(r, np.float32)
    if y is not None:
        v = (v + np.asarray(y, np.float32)).astype(np.float32)
    v64 = v.astype(np.float64)
    inv = 1.0 / np.sqrt((v64 * v64).mean(axis=-1, keepdims=True) + eps)
    z = v64 * inv
    if norm_weight is not None:
        z = z * np.asarray(norm_weight, np.float64)
    x = bf16_round_f32(z.astype(np.float32))
    x64 = x.astype(np.float64)
    logits = (x64 @ np.asarray(router, np.float64).T).astype(np.float32)
    shared = None if shared_gate is None else (x64 @ np.asarray(shared_gate, np.float64).reshape(-1)).astype(np.float32)
    return v, x, logits, shared


# ----------------------------------------------------------------------------- MTP acceptance

def verify_greedy(drafts: np.ndarray, target_logits: np.ndarray) -> tuple[int, int]:
    """Greedy acceptance (native_qwen.py:395-400, dspark.py:862-873): accept
    drafts while each equals the argmax of its target row; return (accepted,
    next token). argmax ties go to the lower index (np.argmax)."""
    t = np.asarray(target_logits, np.float32)
    for index, token in enumerate(np.asarray(drafts).reshape(-1)):
        target = int(np.argmax(t[index]))
        if int(token) != target:
            return index, target
    return len(drafts), int(np.argmax(t[len(drafts)]))


def verify_rejection(drafts, draft_logp: np.ndarray, target_logp: np.ndarray,
                     uniforms: np.ndarray, residual_pick) -> tuple[int, int]:
    """Rejection acceptance (native_qwen.py:401-408, dspark.py:875-898):
    accept draft i when u_i <= min(1, exp(t[tok] - d[tok])); on reject, sample
    from the residual max(p - q, 0) (``residual_pick(probs)`` draws). With all
    drafts accepted the bonus token comes from the last target row."""
    for index, token in enumerate(drafts):
        accept = min(1.0, float(np.exp(target_logp[index][token] - draft_logp[index][token])))
        if uniforms[index] > accept:
            residual = np.maximum(np.exp(target_logp[index]) - np.exp(draft_logp[index]), 0)
            total = residual.sum()
            if total > 0:
                return index, int(residual_pick(residual / total))
            return index, int(residual_pick(np.exp(target_logp[index])))
    return len(drafts), int(residual_pick(np.exp(target_logp[len(drafts)])))


# ----------------------------------------------------------------------------- slot cache policy

@dataclass
class SlotArena:
    """The native expert arena's replacement policy (Native/QwenNative/engine.mm:649-778).

    LFU: the victim is the least-used slot, oldest stamp among equals, never a
    slot handed out in the current plan (stamp == clock). Use counts halve
    (floor 1) every max(8 * slots, 64) touches. Free slots fill in order.
    """
    slots: int
    experts_per_layer: int
    owner: list = field(default_factory=list)
    stamp: list = field(default_factory=list)
    uses: list = field(default_factory=list)
    where: dict = field(default_factory=dict)
    used: int = 0
    clock: int = 0
    touches: int = 0
    hits: int = 0
    misses: int = 0

    def __post_init__(self):
        self.owner = [-1] * self.slots
        self.stamp = [0] * self.slots
        self.uses = [0] * self.slots

    def _victim(self) -> int:
        if self.used < self.slots:
            self.used += 1
            return self.used - 1
        best = -1
        for s in range(self.slots):
            if self.stamp[s] == self.clock:
                continue
            if (best < 0 or self.uses[s] < self.uses[best]
                    or (self.uses[s] == self.uses[best] and self.stamp[s] < self.stamp[best])):
                best = s
        if best < 0:
            raise RuntimeError("the expert cache is too small for one step")
        return best

    def _touch(self):
        self.touches += 1
        if self.touches < max(self.slots * 8, 64):
            return
        self.touches = 0
        self.uses = [max(1, u // 2) for u in self.uses]

    def plan(self, layer: int, experts: list[int]):
        """(slots, missing[(expert, slot)]) as ExpertArena::plan (:679-707)."""
        self.clock += 1
        slots, missing = [], []
        for expert in experts:
            key = layer * self.experts_per_layer + expert
            self._touch()
            if key in self.where:
                s = self.where[key]
                self.stamp[s] = self.clock
                self.uses[s] += 1
                self.hits += 1
                slots.append(s)
                continue
            s = self._victim()
            if self.owner[s] >= 0:
                del self.where[self.owner[s]]
            self.owner[s] = key
            self.where[key] = s
            self.stamp[s] = self.clock
            self.uses[s] = 1
            slots.append(s)
            missing.append((expert, s))
            self.misses += 1
        return slots, missing
