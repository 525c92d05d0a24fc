"""Route-aware slot retention (CPU): the slot cache's native route-history policy
(whallm_amd/csrc/route_policy.h, the behaviour of runtime/deepseek_v4_ssd/route_cache.py:12-120)
against closed forms and the oracle's heap restatement of the quota split, and the native
cache's route-mode eviction against the oracle's heap-based restatement of
ExpertCache._evict_route_locked (expert_cache.py:1143-1181). A policy-only cache (no device
memory) runs all of it on the host."""
import numpy as np
import pytest

from oracle import route_cache as R
from whallm_amd.slot_cache import SlotCache, SlotCacheError


def policy(layers, experts, slots, top_k):
    cache = SlotCache(slots, 256, 128, layers, experts)
    cache.enable_route_policy(top_k)
    return cache


def test_fresh_policy_spreads_slots_over_layers():
    # equal (zero) scores: ties go to the lower rank, then the lower layer
    st = policy(3, 16, 8, 2).route_state()
    assert st["quotas"].tolist() == [3, 3, 2] and st["rebalances"] == 1
    assert policy(2, 4, 100, 1).route_state()["capacity"] == 8
    assert policy(2, 4, 100, 1).route_state()["quotas"].tolist() == [4, 4]


def test_decay_matches_closed_form():
    # one expert every token: the half-life-h rate after n tokens is 1 - 2^(-n / h),
    # whether the tokens arrive one at a time or as one batch (per-token ages)
    one, batch = policy(1, 8, 4, 1), policy(1, 8, 4, 1)
    n = 40
    for _ in range(n):
        one.observe(0, [3], "decode")
    batch.observe(0, [3] * n, "decode")
    for pol in (one, batch):
        st = pol.route_state()
        assert st["short"][0, 3] == pytest.approx(1 - 2 ** (-n / 16), rel=1e-12)
        assert st["long"][0, 3] == pytest.approx(1 - 2 ** (-n / 256), rel=1e-12)
        assert st["decode_tokens"][0] == n and st["short"][0, 2] == 0.0
    # top_k = 2: a 3-token batch [a b | a c | a d] gives expert a weight 1 - 2^(-3/16)
    pol = policy(1, 8, 4, 2)
    pol.observe(0, [1, 2, 1, 3, 1, 4], "decode")
    st = pol.route_state()
    assert st["short"][0, 1] == pytest.approx(1 - 2 ** (-3 / 16), rel=1e-12)
    keep = 2 ** (-1 / 16)
    assert st["short"][0, 2] == pytest.approx((1 - keep) * keep ** 2, rel=1e-12)
    assert st["short"][0, 4] == pytest.approx(1 - keep, rel=1e-12)


def test_decay_survives_a_long_history():
    # 20,000 tokens on one expert, then 48 on another: the lazily stored rates move their
    # time base forward and still equal the closed forms
    pol = policy(1, 4, 2, 1)
    pol.observe(0, [0] * 20000, "decode")
    pol.observe(0, [1] * 48, "decode")
    st = pol.route_state()
    assert st["short"][0, 0] == pytest.approx((1 - 2 ** (-20000 / 16)) * 2 ** (-48 / 16), rel=1e-9)
    assert st["long"][0, 0] == pytest.approx((1 - 2 ** (-20000 / 256)) * 2 ** (-48 / 256), rel=1e-9)
    assert st["short"][0, 1] == pytest.approx(1 - 2 ** (-48 / 16), rel=1e-9)


def test_prefill_prior_and_read_cost():
    pol = policy(2, 4, 4, 2)
    pol.begin_route_request()
    pol.observe(0, [0, 1, 0, 2], "prefill")       # 2 tokens
    pol.observe(1, [3, 3], "prefill")             # 1 token
    pol.record_read(0, 1.0)
    pol.record_read(0, 3.0)                        # running mean: 1 + 0.05 * 2
    pol.record_read(1, 8.0)
    pol.record_read(1, float("nan"))              # ignored
    pol.rebalance()
    st = pol.route_state()
    assert st["read_cost"][0] == pytest.approx(1.1) and st["prompt_tokens"].tolist() == [2, 1]
    median = (1.1 + 8.0) / 2
    cost = np.clip(np.array([1.1, 8.0]) / median, 0.5, 2.0)
    want0 = 0.1 * np.array([2, 1, 1, 0]) / 2 * cost[0]
    want1 = 0.1 * np.array([0, 0, 0, 2]) / 1 * cost[1]
    np.testing.assert_allclose(st["scores"][0], want0, rtol=1e-12)
    np.testing.assert_allclose(st["scores"][1], want1, rtol=1e-12)
    # the prior fades with the request's decode tokens: 2^(-t / 32) after t = 32 tokens
    pol.observe(0, [1] * 2 * 32, "decode")
    pol.rebalance()
    st = pol.route_state()
    assert st["scores"][0, 2] == pytest.approx(0.1 * 1 / 2 * 0.5 * cost[0], rel=1e-12)
    assert st["scores"][1, 3] == pytest.approx(want1[3], rel=1e-12)
    # a new request drops the prior but keeps the decode history
    pol.begin_route_request()
    pol.rebalance()
    st = pol.route_state()
    assert st["scores"][1, 3] == 0.0 and st["scores"][0, 1] > 0.0


def test_rebalance_every_16_tokens_per_layer_and_after_prefill():
    pol = policy(3, 8, 6, 1)
    start = pol.route_state()["rebalances"]
    for t in range(47):
        pol.observe(t % 3, [t % 8], "decode")
    assert pol.route_state()["rebalances"] == start
    pol.observe(0, [1], "decode")                   # the 48th decode token = 16 x 3 layers
    assert pol.route_state()["rebalances"] == start + 1
    pol.set_route_phase("prefill")
    pol.observe(1, [2, 2, 2], "prefill")
    assert pol.route_state()["rebalances"] == start + 1
    pol.set_route_phase("decode")                   # leaving the prefill rebalances
    assert pol.route_state()["rebalances"] == start + 2


@pytest.mark.parametrize("seed", range(6))
def test_quotas_match_heap_allocation(seed):
    rng = np.random.default_rng(seed)
    layers, experts = int(rng.integers(1, 6)), int(rng.integers(2, 40))
    top_k = int(rng.integers(1, 3))
    pol = policy(layers, experts, int(rng.integers(1, layers * experts + 5)), top_k)
    for step in range(300):
        layer = int(rng.integers(layers))
        ids = rng.integers(0, min(experts, 1 + rng.integers(experts)), size=top_k * int(rng.integers(1, 4)))
        phase = "prefill" if step % 50 < 10 else "decode"
        if step % 50 == 0:
            pol.begin_route_request()
        pol.observe(layer, ids, phase)
        if step % 37 == 0:
            pol.record_read(layer, float(rng.uniform(0.1, 3.0)))
            pol.rebalance()
        st = pol.route_state()
        assert st["quotas"].sum() == st["capacity"]
        np.testing.assert_array_equal(st["quotas"], R.route_quotas(st["scores"], st["capacity"]))


def test_policy_rejects_bad_input():
    cache = SlotCache(4, 256, 128, 2, 4)
    with pytest.raises(SlotCacheError, match="invalid dimensions"):
        cache.enable_route_policy(5)                # top_k above the expert count
    with pytest.raises(SlotCacheError, match="not enabled"):
        cache.observe(0, [0], "decode")
    cache.enable_route_policy(2)
    with pytest.raises(SlotCacheError, match="layer out of range"):
        cache.observe(2, [0], "decode")
    with pytest.raises(SlotCacheError, match="outside the model"):
        cache.observe(0, [4], "decode")
    cache.observe(0, [], "decode")
    with pytest.raises(ValueError):
        cache.set_route_phase("verify")
    cache.disable_route_policy()


@pytest.mark.parametrize("slots,layers,experts,k", [(6, 2, 16, 2), (24, 4, 64, 4), (40, 3, 128, 8), (3, 3, 8, 1)])
def test_native_route_eviction_matches_oracle(slots, layers, experts, k):
    rng = np.random.default_rng(slots + 7 * experts)
    native = SlotCache(slots, 256, 128, layers, experts)
    native.enable_route_policy(k)
    st = native.route_state()
    oracle = R.RouteArena(slots, layers, experts)
    oracle.set_route(st["scores"], st["quotas"])
    seen = st["rebalances"]
    hot = rng.permutation(experts)
    for step in range(500):
        layer = int(rng.integers(layers))
        ids = [int(hot[min(experts - 1, rng.zipf(1.4) - 1)]) for _ in range(k)]
        native.observe(layer, ids, "prefill" if step % 97 < 5 else "decode")
        st = native.route_state()
        if st["rebalances"] != seen:
            seen = st["rebalances"]
            oracle.set_route(st["scores"], st["quotas"])
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
