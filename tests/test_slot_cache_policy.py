"""The native slot-cache policy (wm_slot_cache_plan, policy-only handle) against the
oracle's ExpertArena restatement (oracle/moe.py SlotArena, engine.mm:649-778). CPU only."""
import numpy as np
import pytest

from oracle import moe as M
from whallm_amd.slot_cache import SlotCache, SlotCacheError


@pytest.mark.parametrize("slots,experts,files,k", [(3, 10, 1, 2), (11, 64, 4, 10), (40, 512, 3, 10), (1, 8, 2, 1)])
def test_plan_matches_oracle_arena(slots, experts, files, k):
    rng = np.random.default_rng(slots * 1000 + experts)
    native = SlotCache(slots, 256, 128, files, experts)
    oracle = M.SlotArena(slots=slots, experts_per_layer=experts)
    for step in range(400):
        file = int(rng.integers(files))
        # Zipf-skewed requests (repeats inside one plan are allowed, as in the reference)
        ids = [int(min(experts - 1, rng.zipf(1.3) - 1)) for _ in range(k)]
        want_error = None
        try:
            want_slots, want_missing = oracle.plan(file, ids)
        except RuntimeError as e:
            want_error = e
        if want_error is not None:
            with pytest.raises(SlotCacheError, match="too small"):
                native.plan(file, ids)
            return
        got_slots, filled = native.plan(file, ids)
        assert got_slots == want_slots, step
        assert [(e, s) for e, s, f in zip(ids, got_slots, filled) if f] == want_missing, step
    st = native.stats()
    assert (st["hits"], st["misses"]) == (oracle.hits, oracle.misses)


def test_plan_rejects_bad_ids_without_changing_state():
    c = SlotCache(4, 256, 128, 2, 8)
    with pytest.raises(SlotCacheError, match="out of range"):
        c.plan(0, [1, 8])
    with pytest.raises(SlotCacheError, match="out of range"):
        c.plan(2, [1])
    assert c.plan(0, [1]) == ([0], [1])     # nothing was planned by the failed calls
    with pytest.raises(SlotCacheError, match="policy-only"):
        c.acquire(0, [1])
