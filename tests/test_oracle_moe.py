"""Pins the MoE oracle (oracle/moe.py) — CPU only.

Sources of truth: the reference's own tests restated (tie KAT,
runtime/tests/test_runtime.py:2680-2683; pair/wave invariants,
runtime/tests/portable/test_qwen_flash_portable.py:32-92; constant-valued
experts, test_runtime.py:2507-2745; rejection sampling keeps the target
distribution, test_native_qwen.py:71-87) plus brute force and closed forms.
"""
import itertools

import numpy as np
import pytest

from oracle import formats as F
from oracle import moe as M
from oracle import c_oracle as C


# ----------------------------------------------------------------------------- routing

def test_topk_ties_resolve_to_lower_index():
    # _stable_topk_indices([[1, 1, 1, .5]], 2) == [[0, 1]] (test_runtime.py:2680-2683)
    assert M.topk_desc(np.array([[1.0, 1.0, 1.0, 0.5]], np.float32), 2).tolist() == [[0, 1]]


def test_topk_matches_brute_force_and_c():
    rng = np.random.default_rng(0)
    for E, k in ((8, 3), (64, 4), (512, 10), (37, 7)):
        s = rng.integers(-4, 4, size=(50, E)).astype(np.float32)  # many ties
        got = M.topk_desc(s, k)
        for t in range(50):
            brute = sorted(range(E), key=lambda e: (-s[t, e], e))[:k]
            assert got[t].tolist() == brute
        np.testing.assert_array_equal(got, C.topk(s, k))


def test_softmax_weights_equal_renormalised_full_softmax():
    rng = np.random.default_rng(1)
    logits = rng.standard_normal((20, 64)).astype(np.float32)
    idx, w = M.route_softmax_topk(logits, 4, True)
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    kept = np.take_along_axis(p, idx, -1)
    np.testing.assert_allclose(w, kept / kept.sum(-1, keepdims=True), rtol=1e-6)
    idx2, w2 = M.route_softmax_topk(logits, 4, False)
    np.testing.assert_array_equal(idx, idx2)
    np.testing.assert_allclose(w2, kept, rtol=1e-6)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)


def test_scored_routing_bias_selects_but_does_not_weight():
    logits = np.array([[0.0, 1.0, 2.0, 3.0]], np.float32)
    bias = np.array([10.0, 0.0, 0.0, 0.0], np.float32)
    idx, w = M.route_scored(logits, bias, 2, "sigmoid", route_scale=1.5)
    assert idx.tolist() == [[0, 3]]
    s = 1 / (1 + np.exp(-np.array([0.0, 3.0])))
    np.testing.assert_allclose(w[0], s / (s.sum() + 1e-20) * 1.5, rtol=1e-6)
    # sqrt-softplus closed form (Native/DeepSeekNative/engine.mm:1875-1876)
    idx, w = M.route_scored(logits, None, 1, "sqrtsoftplus", norm_topk_prob=False)
    assert idx.tolist() == [[3]]
    np.testing.assert_allclose(w[0, 0], np.sqrt(np.log1p(np.exp(3.0))), rtol=1e-6)


def test_group_limited_matches_brute_force_over_group_subsets():
    # No reference implementation exists (parity unpinned against the reference);
    # pinned against an exhaustive search of the DeepSeek-V3 rule on tiny shapes.
    rng = np.random.default_rng(2)
    E, G, TG, K = 16, 4, 2, 3
    for _ in range(200):
        logits = rng.standard_normal((1, E)).astype(np.float32)
        bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
        idx, _ = M.route_scored(logits, bias, K, "sigmoid", n_groups=G, topk_groups=TG)
        s = (M.score_f32(logits[0], "sigmoid") + bias).astype(np.float32)
        gscore = [np.float32(sum(sorted(s[g * 4:(g + 1) * 4])[-2:])) for g in range(G)]
        best = sorted(range(G), key=lambda g: (-gscore[g], g))[:TG]
        allowed = [e for e in range(E) if e // 4 in best]
        brute = sorted(allowed, key=lambda e: (-s[e], e))[:K]
        assert idx[0].tolist() == brute


# ----------------------------------------------------------------------------- permute

def test_permute_pair_coverage_order_and_inverse():
    # test_qwen_flash_portable.py:32-53 restated for the device permute's lists.
    rng = np.random.default_rng(20260921)
    for tokens in (1, 2, 17, 128, 1024):
        selected = rng.integers(0, 512, size=(tokens, 10), dtype=np.int32)
        p = M.permute(selected, 512, tile_rows=16)
        flat = selected.reshape(-1)
        np.testing.assert_array_equal(np.sort(p.order), np.arange(flat.size))
        assert np.all(np.diff(flat[p.order]) >= 0)
        for e in np.unique(flat):
            rows = p.order[p.offsets[e]:p.offsets[e + 1]]
            assert np.all(flat[rows] == e)
            assert np.all(np.diff(rows) > 0)           # stable: token order kept
        np.testing.assert_array_equal(flat[p.order][p.inverse], flat)
        np.testing.assert_array_equal(p.order[p.inverse], np.arange(flat.size))
        counts = np.bincount(flat, minlength=512)
        assert len(p.tiles) == int(np.sum(-(-counts // 16)))
        for e, start in p.tiles:
            assert p.offsets[e] <= start < p.offsets[e + 1]


def test_permute_rejects_ids_outside_the_model_and_handles_empty():
    with pytest.raises(ValueError):
        M.permute(np.array([[0, 512]]), 512)
    with pytest.raises(ValueError):
        M.permute(np.array([[-1]]), 512)
    p = M.permute(np.empty((0, 10), np.int32), 512)
    assert p.order.size == 0 and p.tiles.shape == (0, 2) and p.offsets[-1] == 0


def test_grouped_reduction_is_exact_against_per_expert_gemm():
    # test_qwen_flash_portable.py:55-80: grouping pairs by expert keeps every product
    rng = np.random.default_rng(7)
    source = rng.normal(size=(31, 8)).astype(np.float32)
    matrix = rng.normal(size=(13, 8, 8)).astype(np.float32)
    selected = rng.integers(0, 13, size=(31, 10))
    baseline = np.empty((selected.size, 8), np.float32)
    for expert in np.unique(selected):
        positions = np.flatnonzero(selected.reshape(-1) == expert)
        baseline[positions] = source[positions // 10] @ matrix[expert]
    p = M.permute(selected, 13)
    grouped = np.empty_like(baseline)
    for e in range(13):
        rows = p.order[p.offsets[e]:p.offsets[e + 1]]
        if rows.size:
            grouped[p.offsets[e]:p.offsets[e + 1]] = source[rows // 10] @ matrix[e]
    np.testing.assert_array_equal(grouped[p.inverse], baseline)


# ----------------------------------------------------------------------------- expert FFN

def _const_expert(value_gu_gate, value_gu_up, value_down, H, I):
    """An MXFP4 expert whose dequantized weights are constants (exact on the grid)."""
    def region(rows, cols, values):
        vals = np.repeat(np.asarray(values, np.float32)[:, None], cols, axis=1)
        w, s = F.quantize_mxfp4_bf16(F.bf16_round(vals), rows, cols)
        return np.ascontiguousarray(w).view(np.uint32), s
    gu, gus = region(2 * I, H, [value_gu_gate] * I + [value_gu_up] * I)
    d, ds = region(H, I, [value_down] * H)
    return M.MXFP4Expert(gu, gus, d, ds)


def test_constant_experts_closed_form():
    # Constant-valued 32x32 experts as in test_runtime.py:2507-2745 (0.125 ... 0.5).
    H = I = 32
    e = _const_expert(0.125, 0.25, 0.375, H, I)
    x = np.full((2, H), 0.5, np.float32)
    g = 0.5 * 0.125 * H
    u = 0.5 * 0.25 * H
    h = g / (1 + np.exp(-g)) * u
    want = np.full((2, H), h * 0.375 * I, np.float32)
    np.testing.assert_allclose(M.expert_ffn(x, e), want, rtol=1e-6)
    # DeepSeek w13 order: rows 0..I-1 are up.
    want_ds = np.full((2, H), (u / (1 + np.exp(-u)) * g) * 0.375 * I, np.float32)
    np.testing.assert_allclose(M.expert_ffn(x, e, up_first=True), want_ds, rtol=1e-6)
    # Clamped SwiGLU (deepseek_v41/moe.py:37-43): up to +-limit, gate clamped above.
    lim = 1.0
    want_cl = np.full((2, H), (min(g, lim) / (1 + np.exp(-min(g, lim))) * np.clip(u, -lim, lim)) * 0.375 * I,
                      np.float32)
    np.testing.assert_allclose(M.expert_ffn(x, e, limit=lim), want_cl, rtol=1e-6)


def test_expert_ffn_matches_float64_loop_and_c():
    rng = np.random.default_rng(11)
    H, I = 64, 32
    from whallm_amd.synthetic import mxfp4_experts_np
    a = mxfp4_experts_np(rng, 1, H, I)
    e = M.MXFP4Expert(a["gate_up"][0], a["gate_up_scales"][0], a["down"][0], a["down_scales"][0])
    x = rng.standard_normal((3, H)).astype(np.float32)
    wgu = F.dequant_mxfp4(e.gate_up, e.gate_up_scales).astype(np.float64)
    wd = F.dequant_mxfp4(e.down, e.down_scales).astype(np.float64)
    want = np.zeros((3, H))
    for t in range(3):
        for i in range(I):
            gsum = sum(x[t, h] * wgu[i, h] for h in range(H))
            usum = sum(x[t, h] * wgu[I + i, h] for h in range(H))
            hval = gsum / (1 + np.exp(-gsum)) * usum
            want[t] += hval * wd[:, i]
    got = M.expert_ffn(x, e)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) < 1e-5
    c = C.ffn(x, wgu.astype(np.float32), wd.astype(np.float32))
    assert np.linalg.norm(c - want) / np.linalg.norm(want) < 1e-5


def test_routed_outputs_keep_router_order_and_combine():
    # Router order preserved (test_runtime.py:2561-2609) and combine closed form.
    H = I = 32
    experts = [_const_expert(0.125, 0.25, 0.375, H, I), _const_expert(0.25, 0.5, 0.125, H, I)]
    x = np.ones((2, H), np.float32)
    idx = np.array([[1, 0], [0, 1]])
    out = M.routed_outputs(x, idx, experts)
    e0 = M.expert_ffn(x[:1], experts[0])[0]
    e1 = M.expert_ffn(x[:1], experts[1])[0]
    np.testing.assert_array_equal(out[0, 0], e1)
    np.testing.assert_array_equal(out[0, 1], e0)
    np.testing.assert_array_equal(out[1, 0], e0)
    w = np.array([[0.75, 0.25], [0.5, 0.5]], np.float32)
    shared = np.full((2, H), 2.0, np.float32)
    gate = np.array([0.0, 100.0])
    y = M.combine(out, w, shared, gate)
    np.testing.assert_allclose(y[0], 0.75 * e1 + 0.25 * e0 + 1.0, rtol=1e-6)
    np.testing.assert_allclose(y[1], 0.5 * e0 + 0.5 * e1 + 2.0, rtol=1e-6)


def test_bf16_steps_models_reduce_to_the_fp32_forms_and_round_at_each_step():
    """The models of the reference's own bf16 arithmetic: with the rounding taken out they are
    the fp32 forms; a one-value case worked by hand lands on the value each rounding forces."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64)).astype(np.float32)
    wgu = (rng.standard_normal((32, 64)) * 0.1).astype(np.float32)
    wd = (rng.standard_normal((64, 16)) * 0.1).astype(np.float32)
    ident = lambda v: np.asarray(v, np.float32)  # noqa: E731
    np.testing.assert_allclose(M.ffn_dense_bf16_steps(x, wgu, wd, rnd=ident), M.ffn_dense(x, wgu, wd), rtol=1e-5,
                               atol=1e-6)
    np.testing.assert_allclose(M.ffn_dense_bf16_steps(x, wgu, wd, limit=0.5, fp32_swiglu=True, rnd=ident),
                               M.ffn_dense(x, wgu, wd, limit=0.5), rtol=1e-5, atol=1e-6)
    rows = rng.standard_normal((4, 3, 64)).astype(np.float32)
    w = rng.random((4, 3)).astype(np.float32)
    sh = rng.standard_normal((4, 64)).astype(np.float32)
    g = rng.standard_normal(4)
    np.testing.assert_allclose(M.combine_bf16_steps(rows, w, sh, g, rnd=ident), M.combine(rows, w, sh, g),
                               rtol=1e-5, atol=1e-6)
    # Qwen rows and the shared V4.1 row come back in bf16, the routed V4.1 rows in fp32
    q = M.ffn_dense_bf16_steps(x, wgu, wd)
    np.testing.assert_array_equal(q, F.bf16_round_f32(q))
    ds = M.ffn_dense_bf16_steps(x, wgu, wd, fp32_swiglu=True, round_act=False, round_out=False)
    assert not np.array_equal(ds, F.bf16_round_f32(ds))
    # by hand: gate 1 + 2^-10 -> bf16 1; sigmoid(1) = 0.731059 -> bf16 187/256; 1 * 187/256 exact;
    # times up 3 = 2.19140625 -> bf16 (step 2^-6 in [2, 4)) 2.1875; times 1 exact
    one = M.ffn_dense_bf16_steps(np.ones((1, 1), np.float32), np.array([[1 + 2.0 ** -10], [3.0]], np.float32),
                                 np.ones((1, 1), np.float32))
    assert one[0, 0] == 2.1875
    # combine: w 0.3 -> bf16 0.30078125; times 1 exact; sum exact; sigmoid(0) = 0.5; 0.5 * 3 exact;
    # 0.30078125 + 1.5 = 1.80078125 -> bf16 (step 2^-7 in [1, 2)) 1.796875 (ties to even: 230.5 -> 230)
    y = M.combine_bf16_steps(np.ones((1, 1, 1), np.float32), np.array([[0.3]], np.float32),
                             np.array([[3.0]], np.float32), np.zeros(1))
    assert y[0, 0] == 1.796875


# ----------------------------------------------------------------------------- acceptance

def test_greedy_acceptance_cases():
    logits = np.zeros((4, 10), np.float32)
    logits[0, 3] = logits[1, 5] = logits[2, 7] = logits[3, 1] = 1.0
    assert M.verify_greedy([3, 5, 7], logits) == (3, 1)
    assert M.verify_greedy([3, 4, 7], logits) == (1, 5)
    assert M.verify_greedy([2, 5, 7], logits) == (0, 3)
    logits[0, 2] = 1.0  # tie: argmax is the lower index
    assert M.verify_greedy([3, 5, 7], logits) == (0, 2)


def test_rejection_sampling_keeps_the_target_distribution():
    # test_native_qwen.py:71-87: one draft position, 20k draws, atol 0.015.
    rng = np.random.default_rng(11)
    target = np.log(np.array([0.5, 0.2, 0.15, 0.1, 0.05]))
    draft = np.log(np.array([0.1, 0.1, 0.6, 0.1, 0.1]))
    counts = np.zeros(5)
    pick = lambda p: rng.choice(p.size, p=p)
    for _ in range(20_000):
        token = int(rng.choice(5, p=np.exp(draft)))
        accepted, following = M.verify_rejection([token], [draft], [target, target], [rng.uniform()], pick)
        counts[token if accepted else following] += 1
    np.testing.assert_allclose(counts / counts.sum(), np.exp(target), atol=0.015)


# ----------------------------------------------------------------------------- slot arena

def test_arena_lfu_protection_and_decay():
    # ExpertArena::plan / victim / touch (Native/QwenNative/engine.mm:679-778)
    a = M.SlotArena(slots=3, experts_per_layer=10)
    slots, missing = a.plan(0, [1, 2, 3])
    assert slots == [0, 1, 2] and missing == [(1, 0), (2, 1), (3, 2)]
    slots, missing = a.plan(0, [1, 2])          # hits raise uses of slots 0, 1
    assert missing == [] and a.hits == 2
    slots, missing = a.plan(0, [4])             # evicts the least used: expert 3 (slot 2)
    assert missing == [(4, 2)]
    with pytest.raises(RuntimeError):
        a.plan(0, [5, 6, 7, 8])                 # more new experts than slots in one step
    b = M.SlotArena(slots=1, experts_per_layer=10)
    for _ in range(70):
        b.plan(0, [1])
    assert b.uses[0] < 70                        # halved after max(8, 64) touches


def test_norm_router_oracle_against_closed_forms():
    """Pins oracle.norm_router: a constant row normalises to +-1 (times the norm weight),
    sum-instead-of-mean or a dropped sqrt would not; the norm weight scales exactly by
    powers of two; a zero row stays zero (eps); logits and the shared gate logit equal a
    brute-force dot product."""
    H = 8
    r = np.array([[2.0] * H, [-3.0] * H, [0.0] * H], np.float32)
    w = np.array([0.5, 2, 1, 1, -1, 4, 1, 0.25], np.float32)
    router = np.arange(3 * H, dtype=np.float32).reshape(3, H) / 8 - 1
    gate = np.linspace(-1, 1, H).astype(np.float32)
    v, x, logits, shared = M.norm_router(r, None, router, gate, w)
    np.testing.assert_array_equal(x, np.stack([w, -w, np.zeros(H, np.float32)]))
    for t in range(3):
        for e in range(3):
            assert logits[t, e] == pytest.approx(sum(float(x[t, h]) * float(router[e, h]) for h in range(H)))
        assert shared[t] == pytest.approx(sum(float(x[t, h]) * float(gate[h]) for h in range(H)))
    rng = np.random.default_rng(3)
    r2 = rng.standard_normal((5, 64)).astype(np.float32)
    y2 = rng.standard_normal((5, 64)).astype(np.float32)
    v2, x_unit, _, none = M.norm_router(r2, y2, np.zeros((1, 64), np.float32))
    assert none is None
    np.testing.assert_array_equal(v2, r2 + y2)
    np.testing.assert_array_equal(x_unit, M.rms_norm(v2))
    _, x_two, _, _ = M.norm_router(r2, y2, np.zeros((1, 64), np.float32), norm_weight=np.full(64, 2.0, np.float32))
    np.testing.assert_array_equal(x_two, 2 * x_unit)


# ----------------------------------------------------------------------------- router score arithmetic

def _ulps(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.abs(got - want) / np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)


def test_exp_f32_is_exp_to_about_one_ulp():
    # the stated fp32 exp against float64 exp over its whole normal range; a dropped
    # polynomial term, a wrong ln2 split or a wrong rounding of n breaks the bound
    x = np.linspace(-86.9, 88.7, 300001).astype(np.float32)   # below: flushed to 0 by definition
    assert _ulps(M.exp_f32(x), np.exp(x.astype(np.float64))).max() <= 1.5
    assert M.exp_f32(np.float32(0.0)) == 1.0
    assert M.exp_f32(np.float32(np.log(2.0))) == 2.0
    assert M.exp_f32(np.float32(-88.0)) == 0.0 and M.exp_f32(np.float32(89.0)) == np.inf
    assert np.isnan(M.exp_f32(np.float32(np.nan))) and M.exp_f32(np.float32(-np.inf)) == 0.0


def test_log1p_and_scores_are_the_functions_to_a_few_ulp():
    u = np.linspace(0.0, 1.0, 100001).astype(np.float32)[1:]
    assert _ulps(M.log1p_f32(u), np.log1p(u.astype(np.float64))).max() <= 4
    assert M.log1p_f32(np.float32(0.0)) == 0.0
    assert _ulps(M.log1p_f32(np.float32(1.0)), np.log(2.0)) <= 1
    z = np.linspace(-100.0, 100.0, 200001).astype(np.float32)
    zd = z.astype(np.float64)
    sig = 1.0 / (1.0 + np.exp(-zd))
    keep = sig > 1e-37
    assert _ulps(M.score_f32(z, "sigmoid")[keep], sig[keep]).max() <= 2.5
    ssp = np.sqrt(np.logaddexp(zd, 0.0))
    assert _ulps(M.score_f32(z, "sqrtsoftplus"), ssp).max() <= 2.5
    assert M.score_f32(np.float32(0.0), "sigmoid") == 0.5
    assert _ulps(M.score_f32(np.float32(0.0), "sqrtsoftplus"), np.sqrt(np.log(2.0))) <= 1
    # symmetric sigmoid, and the e^(l/2) branch joins the softplus branch at l = -64
    np.testing.assert_allclose(M.score_f32(z, "sigmoid") + M.score_f32(-z, "sigmoid"), 1.0, atol=1.2e-7)
    edge = np.float32([-64.0001, -63.9999])
    np.testing.assert_allclose(M.score_f32(edge, "sqrtsoftplus"), np.sqrt(np.logaddexp(edge.astype(np.float64), 0)),
                               rtol=3e-7)


def test_softmax_sums_follow_the_wave_tree():
    rng = np.random.default_rng(5)
    for E in (1, 7, 64, 200, 512, 1000):
        e = rng.random((9, E)).astype(np.float32)
        got = M.softmax_sums_f32(e)
        np.testing.assert_allclose(got, e.astype(np.float64).sum(-1), rtol=1e-6)
        # the tree itself: lane j sums e[j], e[64 + j], ... then the lanes combine pairwise
        lanes = np.zeros((9, 64), np.float32)
        for j in range(64):
            for col in range(j, E, 64):
                lanes[:, j] = lanes[:, j] + e[:, col]
        v = lanes
        for step in (1, 2):
            v = v + v[:, np.arange(64) ^ step]
        v = v + v[:, [(j & ~7) | (7 - (j & 7)) for j in range(64)]]
        v = v + v[:, [(j & ~15) | (15 - (j & 15)) for j in range(64)]]
        np.testing.assert_array_equal(got, (v[:, 0] + v[:, 16]) + (v[:, 32] + v[:, 48]))
    s = M.score_f32(rng.standard_normal((4, 300)).astype(np.float32), "softmax")
    np.testing.assert_allclose(s.astype(np.float64).sum(-1), 1.0, rtol=1e-6)
