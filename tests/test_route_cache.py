"""Route-aware slot retention (CPU): the route-history policy (whallm_amd/route_cache.py,
restating runtime/deepseek_v4_ssd/route_cache.py:12-120), the read-scheduling and
prompt-tail helpers (whallm_amd/streaming_policy.py, qwen_streaming_policy.py:7-45), and the
native cache's route-mode eviction against the oracle's heap-based restatement of
ExpertCache._evict_route_locked (expert_cache.py:1143-1181)."""
import numpy as np
import pytest

from oracle import route_cache as R
from whallm_amd.route_cache import RouteCachePolicy
from whallm_amd.slot_cache import SlotCache, SlotCacheError
from whallm_amd.streaming_policy import contiguous_batches, hot_tail_experts


def test_fresh_policy_spreads_slots_over_layers():
    # equal (zero) scores: ties go to the lower rank, then the lower layer
    pol = RouteCachePolicy(layers=3, experts=16, slots=8, top_k=2)
    assert pol.quotas.tolist() == [3, 3, 2]
    assert RouteCachePolicy(2, 4, 100, 1).capacity == 8


def test_decay_matches_closed_form():
    # one expert every token: the half-life-h rate after n tokens is 1 - 2^(-n / h),
    # whether the tokens arrive one at a time or as one batch (per-token ages)
    one, batch = RouteCachePolicy(1, 8, 4, 1), RouteCachePolicy(1, 8, 4, 1)
    n = 40
    for _ in range(n):
        one.observe(0, [3], "decode")
    batch.observe(0, [3] * n, "decode")
    for pol in (one, batch):
        assert pol.short[0, 3] == pytest.approx(1 - 2 ** (-n / 16), rel=1e-12)
        assert pol.long[0, 3] == pytest.approx(1 - 2 ** (-n / 256), rel=1e-12)
        assert pol.decode_tokens[0] == n
    # top_k = 2: a 3-token batch [a b | a c | a d] gives expert a weight 1 - 2^(-3/16)
    pol = RouteCachePolicy(1, 8, 4, 2)
    pol.observe(0, [1, 2, 1, 3, 1, 4], "decode")
    assert pol.short[0, 1] == pytest.approx(1 - 2 ** (-3 / 16), rel=1e-12)
    keep = 2 ** (-1 / 16)
    assert pol.short[0, 2] == pytest.approx((1 - keep) * keep ** 2, rel=1e-12)


def test_prefill_prior_and_read_cost():
    pol = RouteCachePolicy(2, 4, 4, 2)
    pol.begin_prefill()
    pol.observe(0, [0, 1, 0, 2], "prefill")       # 2 tokens
    pol.observe(1, [3, 3], "prefill")             # 1 token
    pol.record_read(0, 1.0)
    pol.record_read(0, 3.0)                        # running mean: 1 + 0.05 * 2
    pol.record_read(1, 8.0)
    assert pol.read_cost[0] == pytest.approx(1.1)
    pol.rebalance()
    median = (1.1 + 8.0) / 2
    cost = np.clip(np.array([1.1, 8.0]) / median, 0.5, 2.0)
    want0 = 0.1 * np.array([2, 1, 1, 0]) / 2 * cost[0]
    want1 = 0.1 * np.array([0, 0, 0, 2]) / 1 * cost[1]
    np.testing.assert_allclose(pol.scores[0], want0, rtol=1e-12)
    np.testing.assert_allclose(pol.scores[1], want1, rtol=1e-12)
    # the prior fades with the request's decode tokens: 2^(-t / 32) after t = 32 tokens
    pol.observe(0, [1] * 2 * 32, "decode")
    pol.rebalance()
    assert pol.scores[0, 2] == pytest.approx(0.1 * 1 / 2 * 0.5 * cost[0], rel=1e-12)
    assert pol.scores[1, 3] == pytest.approx(want1[3], rel=1e-12)


@pytest.mark.parametrize("seed", range(6))
def test_quotas_match_heap_allocation(seed):
    rng = np.random.default_rng(seed)
    layers, experts = int(rng.integers(1, 6)), int(rng.integers(2, 40))
    pol = RouteCachePolicy(layers, experts, int(rng.integers(1, layers * experts + 5)), int(rng.integers(1, 3)))
    for step in range(300):
        layer = int(rng.integers(layers))
        ids = rng.integers(0, min(experts, 1 + rng.integers(experts)), size=pol.top_k * int(rng.integers(1, 4)))
        phase = "prefill" if step % 50 < 10 else "decode"
        if step % 50 == 0:
            pol.begin_prefill()
        pol.observe(layer, ids, phase)
        if step % 37 == 0:
            pol.record_read(layer, float(rng.uniform(0.1, 3.0)))
            pol.rebalance()
        assert pol.quotas.sum() == pol.capacity
        np.testing.assert_array_equal(pol.quotas, R.route_quotas(pol.scores, pol.capacity))


def test_policy_rejects_bad_input():
    with pytest.raises(ValueError):
        RouteCachePolicy(2, 4, 4, 5)
    pol = RouteCachePolicy(2, 4, 4, 2)
    with pytest.raises(ValueError):
        pol.observe(2, [0], "decode")
    with pytest.raises(ValueError):
        pol.observe(0, [4], "decode")
    assert pol.observe(0, [], "decode") is False
    snap = pol.snapshot()
    assert [row["target_slots"] for row in snap["layers"]] == pol.quotas.tolist()


def test_contiguous_batches():
    assert list(contiguous_batches([1, 2, 3, 5, 6, 9], 2)) == [(1, 2), (3,), (5, 6), (9,)]
    assert list(contiguous_batches([], 4)) == []
    rng = np.random.default_rng(3)
    for _ in range(50):
        ids = sorted(set(int(i) for i in rng.integers(0, 60, size=int(rng.integers(0, 30)))))
        m = int(rng.integers(1, 33))
        runs = list(contiguous_batches(ids, m))
        assert [i for r in runs for i in r] == ids
        for r in runs:
            assert 1 <= len(r) <= m and all(b == a + 1 for a, b in zip(r, r[1:]))
        for a, b in zip(runs, runs[1:]):   # a run ends only at a gap or at the maximum
            assert b[0] != a[-1] + 1 or len(a) == m
    for bad in ((([2, 1]), 4), (([1, 1]), 4), (([-1]), 4), (([1]), 0), (([1]), 33), (([1]), 2.0)):
        with pytest.raises(ValueError):
            list(contiguous_batches(*bad))


def test_hot_tail_experts_against_brute_force():
    rng = np.random.default_rng(4)
    for _ in range(60):
        E, k = int(rng.integers(1, 30)), int(rng.integers(1, 5))
        T = int(rng.integers(1, 200))
        routes = rng.integers(0, E, size=(T, k))
        limit = int(rng.integers(0, E + 2))
        flat = routes[-128:].reshape(-1).tolist()   # the last 128 token positions
        stats = {e: (flat.count(e), max(i for i, v in enumerate(flat) if v == e)) for e in set(flat)}
        ranked = sorted(stats, key=lambda e: (-stats[e][0], -stats[e][1], e))[:limit]
        assert hot_tail_experts(routes, E, limit) == ranked[::-1]
    assert hot_tail_experts(np.zeros((3, 2, 2), np.int32), 4, 2) == [0]
    for args in ((np.zeros((2,), np.int32), 4, 1), (np.zeros((2, 2)), 4, 1), (np.full((2, 2), 4), 4, 1),
                 (np.zeros((2, 2), np.int32), 4, -1)):
        with pytest.raises(ValueError):
            hot_tail_experts(*args)


@pytest.mark.parametrize("slots,layers,experts,k", [(6, 2, 16, 2), (24, 4, 64, 4), (40, 3, 128, 8), (3, 3, 8, 1)])
def test_native_route_eviction_matches_oracle(slots, layers, experts, k):
    rng = np.random.default_rng(slots + 7 * experts)
    native = SlotCache(slots, 256, 128, layers, experts)
    pol = native.enable_route_policy(k)
    oracle = R.RouteArena(slots, layers, experts)
    oracle.set_route(pol.scores, pol.quotas)
    hot = rng.permutation(experts)
    for step in range(500):
        layer = int(rng.integers(layers))
        ids = [int(hot[min(experts - 1, rng.zipf(1.4) - 1)]) for _ in range(k)]
        before = pol.rebalances
        native.observe(layer, ids, "prefill" if step % 97 < 5 else "decode")
        if pol.rebalances != before:
            oracle.set_route(pol.scores, pol.quotas)
        try:
            want = oracle.plan(layer, ids)
        except RuntimeError:
            with pytest.raises(SlotCacheError, match="too small"):
                native.plan(layer, ids)
            return
        got_slots, filled = native.plan(layer, ids)
        assert got_slots == want[0], step
        assert [(e, s) for e, s, f in zip(ids, got_slots, filled) if f] == want[1], step
    native.disable_route_policy()
