"""GPU tests of the HBM slot cache: fills from the pinned host pool land bit-exact in
their slots with the expert -> slot map refreshed, slots follow the oracle policy,
the MoE layer computed through the cache table matches the oracle, and a fill never
overwrites slots that work enqueued before it still reads."""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import moe as M
from whallm_amd import synthetic as S
from whallm_amd.slot_cache import SlotCache, SlotCacheError, qwen_blob_bytes

pytestmark = pytest.mark.gpu

H, I = 256, 128


def blob_of(a, e):
    return np.concatenate([a["gate_up"][e].view(np.uint8).reshape(-1), a["gate_up_scales"][e].reshape(-1),
                           a["down"][e].view(np.uint8).reshape(-1), a["down_scales"][e].reshape(-1)])


def make_pool(files, experts, seed):
    rng = np.random.default_rng(seed)
    arrays = [S.mxfp4_experts_np(rng, experts, H, I) for _ in range(files)]
    blob = qwen_blob_bytes(H, I)
    pool = torch.empty(files * experts * blob, dtype=torch.uint8).pin_memory()
    host = pool.numpy().reshape(files, experts, blob)
    for f in range(files):
        for e in range(experts):
            host[f, e] = blob_of(arrays[f], e)
    return arrays, pool


def test_fills_are_bit_exact_and_follow_the_policy(device):
    files, experts, slots = 3, 24, 12
    arrays, pool = make_pool(files, experts, 1)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    oracle = M.SlotArena(slots=slots, experts_per_layer=experts)
    rng = np.random.default_rng(2)
    blob = cache.blob
    for step in range(40):
        f = int(rng.integers(files))
        ids = [int(v) for v in rng.choice(experts, size=5, replace=False)]
        got = cache.acquire(f, ids)
        want, _ = oracle.plan(f, ids)
        assert got == want, step
        torch.cuda.current_stream(device).synchronize()
        mem = cache.slot_memory.view(slots, blob).cpu().numpy()
        row = cache.map[f].cpu().numpy()
        for e, s in zip(ids, got):
            assert np.array_equal(mem[s], blob_of(arrays[f], e)), (step, e, s)
            assert row[e] == s
    st = cache.stats()
    assert st["hits"] == oracle.hits and st["misses"] == oracle.misses and st["bytes"] == st["fills"] * blob


def test_moe_through_the_cache_matches_oracle(device):
    files, experts, slots, K, T = 2, 16, 16, 4, 8
    arrays, pool = make_pool(files, experts, 3)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    rng = np.random.default_rng(4)
    for f in range(files):
        logits = rng.standard_normal((T, experts)).astype(np.float32)
        idx, w = M.route_softmax_topk(logits, K)
        cache.acquire(f, sorted(set(int(v) for v in idx.reshape(-1))))   # every routed expert resident
        x = S.bf16_normal_np(rng, (T, H))
        xt = S.bf16_bits_to_tensor(x, device)
        y = wa.moe_mxfp4(xt, torch.from_numpy(idx.astype(np.int32)).to(device), torch.from_numpy(w.astype(np.float32)).to(device),
                         cache.table(f))
        ex = {e: M.MXFP4Expert(arrays[f]["gate_up"][e], arrays[f]["gate_up_scales"][e], arrays[f]["down"][e],
                               arrays[f]["down_scales"][e]) for e in range(experts)}
        want = M.moe_layer(S.bf16_bits_to_f32(x), logits, ex, K)[0]
        got = y.float().cpu().numpy()
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= 1e-2 and np.abs(got - want).max() <= 2e-2 * np.abs(want).max(), rel


def test_fill_waits_for_work_that_reads_the_evicted_slots(device):
    files, experts, slots, K, T = 2, 16, 8, 8, 4096
    arrays, pool = make_pool(files, experts, 5)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    ids0 = list(range(8))
    cache.acquire(0, ids0)
    rng = np.random.default_rng(6)
    idx = np.tile(np.arange(8, dtype=np.int32), (T, 1))
    w = np.full((T, K), 1.0 / K, np.float32)
    x = S.bf16_normal_np(rng, (T, H))
    y = wa.moe_mxfp4(S.bf16_bits_to_tensor(x, device), torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device),
                     cache.table(0))                                    # reads slots 0..7
    cache.acquire(1, list(range(8, 16)))                                 # evicts every one of them
    got = y.float().cpu().numpy()
    ex = {e: M.MXFP4Expert(arrays[0]["gate_up"][e], arrays[0]["gate_up_scales"][e], arrays[0]["down"][e],
                           arrays[0]["down_scales"][e]) for e in range(experts)}
    want = M.combine(M.routed_outputs(S.bf16_bits_to_f32(x[:64]), idx[:64], ex), w[:64])
    rel = np.linalg.norm(got[:64] - want) / np.linalg.norm(want)
    assert rel <= 1e-2, rel


def test_layer_reads_seeding_and_route_mode(device):
    """A whole file read into one of two layer buffers lands bit-exact, the layer computed
    from it matches the oracle, the prompt tail's hottest experts are seeded into free slots
    from that buffer (bytes and map), and route mode keeps serving fills."""
    files, experts, slots, K, T = 2, 16, 6, 4, 96
    arrays, pool = make_pool(files, experts, 7)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    bufs = [cache.layer_buffer(), cache.layer_buffer()]
    blob = cache.blob
    rng = np.random.default_rng(8)
    cache.read_layer(0, bufs[0])
    for f in range(files):
        cache.wait_layer(f)
        if f + 1 < files:
            cache.read_layer(f + 1, bufs[(f + 1) % 2])      # the next file streams in meanwhile
        buf = bufs[f % 2]
        logits = rng.standard_normal((T, experts)).astype(np.float32)
        idx, w = M.route_softmax_topk(logits, K)
        x = S.bf16_normal_np(rng, (T, H))
        it = torch.from_numpy(idx.astype(np.int32)).to(device)
        y = wa.moe_mxfp4(S.bf16_bits_to_tensor(x, device), it, torch.from_numpy(w.astype(np.float32)).to(device),
                         cache.layer_table(buf))
        ex = {e: M.MXFP4Expert(arrays[f]["gate_up"][e], arrays[f]["gate_up_scales"][e], arrays[f]["down"][e],
                               arrays[f]["down_scales"][e]) for e in range(experts)}
        want = M.moe_layer(S.bf16_bits_to_f32(x), logits, ex, K)[0]
        got = y.float().cpu().numpy()
        assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 1e-2, f
        host = buf.cpu().numpy().reshape(experts, blob)
        for e in range(experts):
            assert np.array_equal(host[e], blob_of(arrays[f], e)), (f, e)
        # keep this prompt's hottest experts resident (free slots only)
        keep, got_slots = cache.seed_tail(f, it, slots // files, buf)
        assert keep == tail_ranking(idx, experts, slots // files)
        torch.cuda.current_stream(device).synchronize()
        mem = cache.slot_memory.view(slots, blob).cpu().numpy()
        row = cache.map[f].cpu().numpy()
        for e, s in zip(keep, got_slots):
            assert np.array_equal(mem[s], blob_of(arrays[f], e)) and row[e] == s, (f, e, s)
    # route mode: a decode request for file 1 through the cache, its experts resident and exact
    cache.enable_route_policy(K)
    ids = [1, 5, 9, 13]
    got = cache.acquire(1, ids)
    torch.cuda.current_stream(device).synchronize()
    mem = cache.slot_memory.view(slots, blob).cpu().numpy()
    for e, s in zip(ids, got):
        assert np.array_equal(mem[s], blob_of(arrays[1], e))
    assert cache.route_state()["decode_tokens"][1] == 1     # the request counted as routes


def tail_ranking(routes, experts, limit):
    """Brute force of the prompt-tail ranking: the last 128 token rows, experts by count,
    then latest position, then id; the first `limit`, least valuable first."""
    flat = np.asarray(routes).reshape(-1, np.asarray(routes).shape[-1])[-128:].reshape(-1).tolist()
    stats = {e: (flat.count(e), max(i for i, v in enumerate(flat) if v == e)) for e in set(flat) if 0 <= e < experts}
    return sorted(stats, key=lambda e: (-stats[e][0], -stats[e][1], e))[:limit][::-1]


def test_tail_seeding_ranks_like_brute_force_and_uses_free_slots_only(device):
    experts, slots = 40, 30
    _, pool = make_pool(1, experts, 30)
    rng = np.random.default_rng(31)
    for trial in range(12):
        cache = SlotCache(slots, H, I, 1, experts, pool, device)
        buf = cache.layer_buffer()
        cache.read_layer(0, buf)
        cache.wait_layer(0)
        pre = sorted(set(int(v) for v in rng.choice(experts, size=int(rng.integers(0, 20)), replace=False)))
        if pre:
            cache.acquire(0, pre)
        T, k = int(rng.integers(1, 300)), int(rng.integers(1, 5))
        routes = rng.integers(0, experts, size=(T, k)).astype(np.int32)
        limit = int(rng.integers(0, experts + 3))
        got, got_slots = cache.seed_tail(0, torch.from_numpy(routes).to(device), limit, buf)
        ranked = [e for e in tail_ranking(routes, experts, limit) if e not in pre]
        free = slots - len(pre)
        want = ranked[-free:] if free and len(ranked) > free else (ranked if free else [])
        assert got == want, trial
        assert sorted(got_slots) == list(range(len(pre), len(pre) + len(got)))  # free slots, in order


def test_partial_layer_reads_batch_consecutive_experts(device):
    experts = 64
    arrays, pool = make_pool(1, experts, 32)
    cache = SlotCache(4, H, I, 1, experts, pool, device)
    buf = cache.layer_buffer()
    buf.fill_(0xAB)
    ids = [0, 1, 2, 3, 7, 9, 10] + list(range(20, 60))       # runs: 4, 1, 2, 32, 8
    before = cache.stats()
    cache.read_layer(0, buf, ids)
    cache.wait_layer(0)
    after = cache.stats()
    assert after["copies"] - before["copies"] == 5
    assert after["bytes"] - before["bytes"] == len(ids) * cache.blob
    host = buf.cpu().numpy().reshape(experts, cache.blob)
    for e in range(experts):
        if e in ids:
            assert np.array_equal(host[e], blob_of(arrays[0], e)), e
        else:
            assert (host[e] == 0xAB).all(), e
    with pytest.raises(SlotCacheError, match="sorted"):
        cache.read_layer(0, buf, [3, 2])


def test_acquire_files_keeps_every_layer_resident(device):
    files, experts, slots = 4, 16, 12
    arrays, pool = make_pool(files, experts, 33)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    rng = np.random.default_rng(34)
    for step in range(20):
        req = {f: sorted(int(v) for v in rng.choice(experts, 3, replace=False)) for f in range(files)}
        got = cache.acquire_files(req)
        torch.cuda.current_stream(device).synchronize()
        mem = cache.slot_memory.view(slots, cache.blob).cpu().numpy()
        m = cache.map.cpu().numpy()
        for f, ids in req.items():
            for e, s in zip(ids, got[f]):
                assert m[f, e] == s and np.array_equal(mem[s], blob_of(arrays[f], e)), (step, f, e)
    with pytest.raises(SlotCacheError, match="too small"):
        cache.acquire_files({f: list(range(4)) for f in range(files)})   # 16 experts, 12 slots


@pytest.mark.parametrize("kind,limit", [("qwen", 0.0), ("deepseek", 1.5)])
def test_installed_files_feed_the_cache(device, tmp_path, kind, limit):
    """Expert files in the reference's on-disk format read into the pinned pool (DeepSeek
    rewritten to the fused slot order) and served through the slot cache: the layer matches
    the oracle built gate-first from the files' source regions."""
    from install_files import write_install
    from whallm_amd.blob_loader import ExpertFiles
    layers, experts, slots, K, T = 2, 16, 16, 4, 24
    src = write_install(tmp_path, kind, layers, experts, H, I, seed=9)
    files = ExpertFiles(tmp_path)
    pool = files.read()
    cache = files.slot_cache(slots, pool, device, swiglu_limit=limit)
    assert cache.up_first == (kind == "deepseek")
    rng = np.random.default_rng(10)
    for f in range(layers):
        s = src[f]
        if kind == "qwen":
            gu = lambda e: (s["gate_up.weight"][e], s["gate_up.scale"][e])
        else:   # gate = w1 then up = w3: the oracle's gate-first expert
            gu = lambda e: (np.concatenate([s["w1.weight"][e], s["w3.weight"][e]]),
                            np.concatenate([s["w1.scale"][e], s["w3.scale"][e]]))
        dn = "down" if kind == "qwen" else "w2"
        ex = {e: M.MXFP4Expert(gu(e)[0].view(np.uint32).reshape(2 * I, H // 8), gu(e)[1].reshape(2 * I, H // 32),
                               s[f"{dn}.weight"][e].view(np.uint32).reshape(H, I // 8),
                               s[f"{dn}.scale"][e].reshape(H, I // 32)) for e in range(experts)}
        logits = rng.standard_normal((T, experts)).astype(np.float32)
        idx, w = M.route_softmax_topk(logits, K)
        cache.acquire(f, sorted(set(int(v) for v in idx.reshape(-1))))   # every routed expert resident
        x = S.bf16_normal_np(rng, (T, H))
        y = wa.moe_mxfp4(S.bf16_bits_to_tensor(x, device), torch.from_numpy(idx.astype(np.int32)).to(device),
                         torch.from_numpy(w.astype(np.float32)).to(device), cache.table(f))
        want = M.combine(M.routed_outputs(S.bf16_bits_to_f32(x), idx, ex, limit=limit), w)
        got = y.float().cpu().numpy()
        rel = np.linalg.norm(got - want) / np.linalg.norm(want)
        assert rel <= 1e-2 and np.abs(got - want).max() <= 2e-2 * np.abs(want).max(), (f, rel)
