"""GPU tests of expert residency, masked pairs and the cached-first order.

- The slot cache's device map always equals the oracle arena's placement: an expert that
  lost its slot to another file reads -1 in its own file's row.
- A pair whose expert is not resident contributes nothing (zero per-pair row, no share of
  the combine), on the decode GEMV and the grouped-GEMM paths, MXFP4 and FP8.
- A pair with a negative id leaves its per-pair row as it was, so two calls over
  complementary masks give the one-call result bit for bit.
- The cached-first acquire (ready experts computed while the missing ones are copied in)
  gives the all-resident result bit for bit, at a small shape and at the C2 expert shape;
  hits on slots whose fills are still pending are not ready, and acquire waits for them.
- The per-pair combine and the bf16 shared-expert MLP match the oracle's float64 closed
  forms (relative L2 <= 1e-2, max |err| <= 2e-2 max |ref|).
"""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import moe as M
from whallm_amd import synthetic as S
from whallm_amd.slot_cache import SlotCache, qwen_blob_bytes

pytestmark = pytest.mark.gpu

H, I = 256, 128


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    mx = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"


def blob_of(a, e):
    return np.concatenate([a["gate_up"][e].view(np.uint8).reshape(-1), a["gate_up_scales"][e].reshape(-1),
                           a["down"][e].view(np.uint8).reshape(-1), a["down_scales"][e].reshape(-1)])


def make_pool(files, experts, seed, hidden=H, inter=I):
    rng = np.random.default_rng(seed)
    arrays = [S.mxfp4_experts_np(rng, experts, hidden, inter) for _ in range(files)]
    blob = qwen_blob_bytes(hidden, inter)
    pool = torch.empty(files * experts * blob, dtype=torch.uint8).pin_memory()
    host = pool.numpy().reshape(files, experts, blob)
    for f in range(files):
        for e in range(experts):
            host[f, e] = blob_of(arrays[f], e)
    return arrays, pool


def test_device_map_tracks_evictions(device):
    files, experts, slots = 3, 24, 12
    _, pool = make_pool(files, experts, 11)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    oracle = M.SlotArena(slots=slots, experts_per_layer=experts)
    rng = np.random.default_rng(12)
    for step in range(30):
        f = int(rng.integers(files))
        ids = [int(v) for v in rng.choice(experts, size=5, replace=False)]
        cache.acquire(f, ids)
        oracle.plan(f, ids)
        torch.cuda.current_stream(device).synchronize()
        want = np.full((files, experts), -1, np.int32)
        for key, s in oracle.where.items():
            want[key // experts, key % experts] = s
        np.testing.assert_array_equal(cache.map.cpu().numpy(), want, err_msg=f"step {step}")


@pytest.mark.parametrize("tokens", [4, 200])   # decode GEMV (T*K <= 256) and grouped GEMM
def test_evicted_experts_contribute_nothing(device, tokens):
    files, experts, slots, K = 2, 8, 8, 4
    arrays, pool = make_pool(files, experts, 13)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    cache.acquire(0, list(range(8)))
    cache.acquire(1, [0, 1, 2])          # takes three of file 0's slots (LFU: the oldest)
    torch.cuda.current_stream(device).synchronize()
    row = cache.map[0].cpu().numpy()
    gone = [e for e in range(experts) if row[e] < 0]
    assert len(gone) == 3, row
    rng = np.random.default_rng(14)
    idx = np.stack([rng.choice(experts, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    w = rng.random((tokens, K)).astype(np.float32)
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, H)), device)
    it, wt = torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device)
    dense = S.experts_to_device(arrays[0], device)
    got = wa.experts_mxfp4(x, it, cache.table(0)).cpu()
    want = wa.experts_mxfp4(x, it, dense).cpu()
    dead = torch.from_numpy(np.isin(idx, gone))
    assert bool((got[dead] == 0).all())
    assert torch.equal(got[~dead], want[~dead])
    # the layer: evicted pairs drop out of the combine (their weight counts as 0)
    y = wa.moe_mxfp4(x, it, wt, cache.table(0)).float().cpu().numpy()
    w0 = np.where(np.isin(idx, gone), 0.0, w).astype(np.float32)
    y0 = wa.moe_mxfp4(x, it, torch.from_numpy(w0).to(device), dense).float().cpu().numpy()
    np.testing.assert_allclose(y, y0, rtol=1e-2, atol=1e-6 * np.abs(y0).max())


@pytest.mark.parametrize("tokens", [4, 200])
def test_fp8_non_resident_slots_contribute_nothing(device, tokens):
    E, Hf, If, K = 6, 256, 256, 2
    rng = np.random.default_rng(15)
    arrays = S.fp8_experts_np(rng, E, Hf, If)
    dense = S.fp8_experts_to_device(arrays, device)
    slots = torch.tensor([0, -1, 2, 3, -1, 5], dtype=torch.int32, device=device)
    table = S.fp8_experts_to_device(arrays, device, slots=slots, experts=E)
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, Hf)), device)
    it = torch.from_numpy(idx).to(device)
    got = wa.experts_fp8(x, it, table).cpu()
    want = wa.experts_fp8(x, it, dense).cpu()
    dead = torch.from_numpy(np.isin(idx, [1, 4]))
    assert bool((got[dead] == 0).all())
    assert torch.equal(got[~dead], want[~dead])


@pytest.mark.parametrize("kind,tokens", [("mxfp4", 6), ("mxfp4", 300), ("fp8", 6), ("fp8", 300)])
def test_complementary_masks_equal_one_call(device, kind, tokens):
    E, K = 16, 4
    rng = np.random.default_rng(16 + tokens)
    if kind == "mxfp4":
        table = S.experts_to_device(S.mxfp4_experts_np(rng, E, H, I), device)
        run, hid = wa.experts_mxfp4, H
    else:
        table = S.fp8_experts_to_device(S.fp8_experts_np(rng, E, 256, 256), device)
        run, hid = wa.experts_fp8, 256
    idx = np.stack([rng.choice(E, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    mask = rng.random(idx.shape) < 0.5
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, hid)), device)
    full = run(x, torch.from_numpy(idx).to(device), table)
    out = torch.full((tokens, K, hid), 7.0, dtype=torch.bfloat16, device=device)
    run(x, torch.from_numpy(np.where(mask, idx, -1)).to(device), table, out=out)
    held = out.cpu()
    m = torch.from_numpy(mask)
    assert bool((held[~m] == 7.0).all()), "a masked pair's row was written"
    run(x, torch.from_numpy(np.where(mask, -1, idx)).to(device), table, out=out)
    assert torch.equal(out.cpu(), full.cpu())


@pytest.mark.parametrize("tokens", [1, 40])
def test_cached_first_acquire_equals_all_resident(device, tokens):
    files, experts, slots, K = 2, 32, 28, 6
    arrays, pool = make_pool(files, experts, 17)
    cache = SlotCache(slots, H, I, files, experts, pool, device)
    rng = np.random.default_rng(18)
    cache.acquire(0, list(range(0, 12)))                     # half of what the step routes to
    idx = np.stack([rng.choice(24, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, H)), device)
    it = torch.from_numpy(idx).to(device)
    unique = sorted(set(idx.reshape(-1).tolist()))
    got = cache.experts_ready_first(0, x, it)
    want = wa.experts_mxfp4(x, it, S.experts_to_device(arrays[0], device))
    assert torch.equal(got.cpu(), want.cpu())
    _, ready = cache.acquire_ready(0, unique)                # now every one is resident
    assert all(ready)
    cache.wait_fills()


def test_cached_first_at_decode_shape(device):
    # The C2 expert shape (H 2048, I 512; 1.6 MB blobs). After a warm-up call, 20 of the
    # step's experts are copied in from pinned host memory while the pairs of the resident
    # ones run (the rocprofv3 trace of this test shows those kernels inside the copy's span).
    # Three fresh caches in a row, so the last round runs with every code path warm.
    files, experts, slots, K, tokens = 1, 48, 40, 10, 16
    arrays, pool = make_pool(files, experts, 21, hidden=2048, inter=512)
    table = S.experts_to_device(arrays[0], device)
    rng = np.random.default_rng(22)
    for _ in range(3):
        cache = SlotCache(slots, 2048, 512, files, experts, pool, device)
        cache.acquire(0, list(range(12)))
        for lo, hi in ((12, 18), (18, 38)):    # 6 missing experts, then 20
            idx = np.stack([np.concatenate([rng.choice(12, 4, replace=False),
                                            rng.choice(np.arange(lo, hi), K - 4, replace=False)])
                            for _ in range(tokens)]).astype(np.int32)
            x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, 2048)), device)
            it = torch.from_numpy(idx).to(device)
            got = cache.experts_ready_first(0, x, it)
            want = wa.experts_mxfp4(x, it, table)
            assert torch.equal(got.cpu(), want.cpu())
        assert cache.stats()["copies"] > 0


def test_hits_on_slots_still_filling_wait_for_their_fills(device):
    """acquire_ready fills 20 missing experts (33 MB at the C2 expert shape) without making the
    stream wait. A second request for them before any wait_fills finds hits whose copies may
    still be in flight: acquire_ready and acquire_split report them not ready, and acquire
    (every expert a hit) still makes the stream wait for those fills, so the kernel enqueued
    right after it reads the filled weights (the output equals the all-resident table's bit
    for bit and matches the oracle)."""
    files, experts, slots, K, tokens = 1, 48, 40, 10, 4
    arrays, pool = make_pool(files, experts, 31, hidden=2048, inter=512)
    cache = SlotCache(slots, 2048, 512, files, experts, pool, device)
    table = S.experts_to_device(arrays[0], device)
    missing = list(range(4, 24))
    _, ready = cache.acquire_ready(0, missing)
    assert not any(ready)
    _, ready = cache.acquire_ready(0, missing[:3])          # hits, but their fills are pending
    assert not any(ready)
    rng = np.random.default_rng(32)
    idx = np.stack([rng.choice(missing, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    it = torch.from_numpy(idx).to(device)
    ready_idx, late_idx, any_late = cache.acquire_split(0, it)
    assert any_late and bool((ready_idx == -1).all()) and torch.equal(late_idx, it)
    cache.acquire(0, missing)                               # every expert a hit
    x_bits = S.bf16_normal_np(rng, (tokens, 2048))
    x = S.bf16_bits_to_tensor(x_bits, device)
    got = wa.experts_mxfp4(x, it, cache.table(0))
    want = wa.experts_mxfp4(x, it, table)
    assert torch.equal(got.cpu(), want.cpu())
    ex = {e: M.MXFP4Expert(arrays[0]["gate_up"][e], arrays[0]["gate_up_scales"][e], arrays[0]["down"][e],
                           arrays[0]["down_scales"][e]) for e in set(idx.reshape(-1).tolist())}
    close(got.float().cpu().numpy(), M.routed_outputs(S.bf16_bits_to_f32(x_bits), idx, ex), "after the hits")
    _, ready = cache.acquire_ready(0, missing)              # acquire waited: resident now
    assert all(ready)
    ready_idx, late_idx, any_late = cache.acquire_split(0, it)
    assert not any_late and torch.equal(ready_idx, it) and bool((late_idx == -1).all())


def test_held_fills_start_on_the_next_cache_call(device):
    """acquire_split holds its copies back until start_fills; a caller that goes on to another
    cache call (here acquire, or wait_fills) without start_fills still gets them: the kernel
    after that call reads the filled weights (equal to the all-resident table bit for bit)."""
    files, experts, slots, K, tokens = 1, 48, 40, 10, 4
    arrays, pool = make_pool(files, experts, 33, hidden=2048, inter=512)
    table = S.experts_to_device(arrays[0], device)
    rng = np.random.default_rng(34)
    idx = np.stack([rng.choice(experts, K, replace=False) for _ in range(tokens)]).astype(np.int32)
    it = torch.from_numpy(idx).to(device)
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, 2048)), device)
    want = wa.experts_mxfp4(x, it, table)
    for follow in ("acquire", "wait_fills"):
        cache = SlotCache(slots, 2048, 512, files, experts, pool, device)
        _, _, any_late = cache.acquire_split(0, it)
        assert any_late
        if follow == "acquire":
            cache.acquire(0, sorted(set(idx.reshape(-1).tolist())))   # every expert a hit of the held plan
        else:
            cache.wait_fills()
        got = wa.experts_mxfp4(x, it, cache.table(0))
        assert torch.equal(got.cpu(), want.cpu()), follow


def test_combine_pairs_matches_oracle(device):
    rng = np.random.default_rng(19)
    T, K, Hc = 37, 10, 2048
    rows = S.bf16_normal_np(rng, (T, K, Hc))
    w = rng.random((T, K)).astype(np.float32)
    add = S.bf16_normal_np(rng, (T, Hc))
    y = wa.combine_pairs(S.bf16_bits_to_tensor(rows, device), torch.from_numpy(w).to(device),
                         S.bf16_bits_to_tensor(add, device))
    want = M.combine(S.bf16_bits_to_f32(rows), w) + S.bf16_bits_to_f32(add)
    close(y.float().cpu().numpy(), want, "combine_pairs")


@pytest.mark.parametrize("tokens,gated,added", [(1, True, True), (16, False, False), (130, True, True)])
def test_mlp_bf16_matches_oracle(device, tokens, gated, added):
    rng = np.random.default_rng(20 + tokens)
    Hm, Im = 2048, 512
    x = S.bf16_normal_np(rng, (tokens, Hm))
    g, u = S.bf16_normal_np(rng, (Im, Hm), 0.02), S.bf16_normal_np(rng, (Im, Hm), 0.02)
    d = S.bf16_normal_np(rng, (Hm, Im), 0.02)
    gv = S.bf16_normal_np(rng, (Hm,), 0.02) if gated else None
    add = S.bf16_normal_np(rng, (tokens, Hm), 0.1) if added else None
    t = lambda a: None if a is None else S.bf16_bits_to_tensor(a, device)  # noqa: E731
    y = wa.mlp_bf16(t(x), t(g), t(u), t(d), t(gv), t(add))
    xf, gf, uf, df = (S.bf16_bits_to_f32(a).astype(np.float64) for a in (x, g, u, d))
    want = (M.silu(xf @ gf.T) * (xf @ uf.T)) @ df.T
    if gated:
        want = want / (1.0 + np.exp(-(xf @ S.bf16_bits_to_f32(gv).astype(np.float64))))[:, None]
    if added:
        want = want + S.bf16_bits_to_f32(add)
    close(y.float().cpu().numpy(), want, f"mlp_bf16 T={tokens}")
