"""GPU parity of the FP8-E4M3 (128x128 block-scale) expert FFN against the oracle's fp32
dequant-then-matmul (oracle/moe.py fp8_expert_ffn, restating deepseek_v41/moe.py:77-93
and mimo/weights.py:17-43). Tolerance: relative L2 <= 1e-2 and max |err| <= 2e-2 * max |ref|.
Covers the fused GEMV (T*K <= 256) and the grouped GEMM, DeepSeek routing (sigmoid,
group-limited), the ungated shared expert, the clamped SwiGLU, the up-first w13 order and
router-order outputs, at the C4 hidden / intermediate sizes and at small ones."""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import formats as F
from oracle import moe as M
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu


def oracle_experts(a, n, up_first=False):
    I = a["w13"].shape[1] // 2
    fmt = 1 if a["w13_scales"].dtype == np.uint8 else 0   # E8M0 32x32 or fp32 128x128 blocks
    b = I // (32 if fmt else 128)
    out = {}
    for e in range(n):
        w13, s13 = a["w13"][e], a["w13_scales"][e]
        g, sg = (w13[I:], s13[b:]) if up_first else (w13[:I], s13[:b])
        u, su = (w13[:I], s13[:b]) if up_first else (w13[I:], s13[b:])
        out[e] = M.FP8Expert(g, sg, u, su, a["w2"][e], a["w2_scales"][e], scale_format=fmt)
    return out


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    mx = np.abs(got - want).max() / np.abs(want).max()
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"


CASES = {  # name: (H, I, E, K, T)
    "decode-small": (1024, 1024, 16, 4, 2),
    "prefill-small": (1024, 1024, 16, 4, 300),
    "prefill-odd": (640, 384, 8, 2, 70),   # multiples of 128 only: GEMM path even at small T
    "prefill-tiny-k": (256, 128, 8, 2, 150),  # 2 and 1 K steps per tile: the rings' short paths
    "c4-decode": (7168, 2048, 8, 4, 1),
}


@pytest.mark.parametrize("fmt", [0, 1], ids=["fp32-128", "e8m0-32"])
@pytest.mark.parametrize("case", sorted(CASES))
def test_moe_fp8_matches_oracle(device, case, fmt):
    H, I, E, K, T = CASES[case]
    rng = np.random.default_rng(H + I + T)
    a = S.fp8_experts_np(rng, E, H, I, scale_format=fmt)
    sh = S.fp8_experts_np(rng, 1, H, I, scale_format=fmt)
    x = S.bf16_normal_np(rng, (T, H))
    logits = rng.standard_normal((T, E)).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32)
    groups = 4 if E % 4 == 0 and E // 4 >= 2 else 1
    idx_t, w_t = wa.route_scored(torch.from_numpy(logits).to(device), torch.from_numpy(bias).to(device), K,
                                 func="sigmoid", route_scale=2.5, n_groups=groups, topk_groups=min(2, groups))
    y = wa.moe_fp8(S.bf16_bits_to_tensor(x, device), idx_t, w_t, S.fp8_experts_to_device(a, device),
                   S.fp8_experts_to_device(sh, device), None)
    idx, w = M.route_scored(logits, bias, K, func="sigmoid", route_scale=2.5, n_groups=groups,
                            topk_groups=min(2, groups))
    np.testing.assert_array_equal(idx_t.cpu().numpy(), idx)
    xf = S.bf16_bits_to_f32(x)
    ex = oracle_experts(a, E)
    routed = M.routed_outputs(xf, idx, ex, ffn=M.fp8_expert_ffn)
    shared = M.fp8_expert_ffn(xf, oracle_experts(sh, 1)[0])
    want = M.combine(routed, w, shared, None)
    close(y.float().cpu().numpy(), want, case)


@pytest.mark.parametrize("T", [3, 120])
def test_router_order_clamp_and_up_first(device, T):
    H, I, E, K = 1024, 1024, 8, 3
    rng = np.random.default_rng(T)
    a = S.fp8_experts_np(rng, E, H, I, scale_low=2.0 ** -4, scale_high=2.0 ** -3)  # large enough to clamp
    x = S.bf16_normal_np(rng, (T, H))
    idx = rng.integers(0, E, size=(T, K)).astype(np.int32)
    table = S.fp8_experts_to_device(a, device, up_first=True, swiglu_limit=10.0)
    out = wa.experts_fp8(S.bf16_bits_to_tensor(x, device), torch.from_numpy(idx).to(device), table)
    ex = oracle_experts(a, E, up_first=True)
    want = M.routed_outputs(S.bf16_bits_to_f32(x), idx, ex, ffn=M.fp8_expert_ffn, limit=10.0)
    close(out.float().cpu().numpy(), want, f"router order T={T}")


def _fp8_tile_layout_np(w):
    """[R, K] FP8 rows -> the prefill tile layout [K/128][R/16][8][16 rows][16 bytes], flattened
    back to [R, K] (the row layout's region size)."""
    R, K = w.shape
    return np.ascontiguousarray(w.reshape(R // 16, 16, K // 128, 8, 16).transpose(2, 0, 3, 1, 4)).reshape(R, K)


def test_fp8_prefill_layout_bytes(device):
    H, I, E, pool = 384, 256, 3, 5
    rng = np.random.default_rng(11)
    a = S.fp8_experts_np(rng, pool, H, I)
    slots = np.array([4, 0, 2], np.int32)
    table = S.fp8_experts_to_device(a, device, slots=torch.from_numpy(slots).to(device), experts=E)
    tiled = wa.prefill_layout(table)
    torch.cuda.synchronize()
    assert tiled.tiled and tiled.slots is None and tiled.count == E
    for e, s in enumerate(slots):
        np.testing.assert_array_equal(tiled.w13[e].cpu().numpy(), _fp8_tile_layout_np(a["w13"][s]))
        np.testing.assert_array_equal(tiled.w2[e].cpu().numpy(), _fp8_tile_layout_np(a["w2"][s]))
        np.testing.assert_array_equal(tiled.w13_scales[e].cpu().numpy(), a["w13_scales"][s])
        np.testing.assert_array_equal(tiled.w2_scales[e].cpu().numpy(), a["w2_scales"][s])


@pytest.mark.parametrize("case", ["decode-small", "prefill-small", "prefill-odd", "prefill-tiny-k"])
def test_fp8_prefill_layout_matches_oracle_and_row_layout(device, case):
    """Tables in the prefill tile layout take the grouped GEMM at every batch size; the GEMM
    reads the same bytes in the same order, so its output equals the row layout's bit for bit
    (where the row layout also takes the GEMM) and the oracle within the FP8 tolerance."""
    H, I, E, K, T = CASES[case]
    rng = np.random.default_rng(H + 7 * T)
    a = S.fp8_experts_np(rng, E, H, I)
    sh = S.fp8_experts_np(rng, 1, H, I)
    x = S.bf16_normal_np(rng, (T, H))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, size=(T, K)).astype(np.float32)
    rows, rows_sh = S.fp8_experts_to_device(a, device), S.fp8_experts_to_device(sh, device)
    tiled, tiled_sh = wa.prefill_layout(rows), wa.prefill_layout(rows_sh)
    xt = S.bf16_bits_to_tensor(x, device)
    it, wt = torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device)
    y = wa.moe_fp8(xt, it, wt, tiled, tiled_sh, None)
    xf = S.bf16_bits_to_f32(x)
    want = M.combine(M.routed_outputs(xf, idx, oracle_experts(a, E), ffn=M.fp8_expert_ffn), w,
                     M.fp8_expert_ffn(xf, oracle_experts(sh, 1)[0]), None)
    close(y.float().cpu().numpy(), want, f"tiled {case}")
    y_rows = wa.moe_fp8(xt, it, wt, rows, rows_sh, None)
    if T * K > 256:   # the row layout takes the grouped GEMM as well (else the fused GEMV)
        assert torch.equal(y, y_rows), case
    else:
        close(y_rows.float().cpu().numpy(), want, f"row layout {case}")


def test_fp8_edges_empty_k1_slots_and_invalid_ids(device):
    """Edges of both paths: empty batches in both layouts, K = 1, experts resolved through a
    slot pool, and an out-of-range expert id."""
    H, I, E, pool = 256, 128, 6, 9
    rng = np.random.default_rng(41)
    a = S.fp8_experts_np(rng, pool, H, I)
    slots = np.array([7, 2, 0, 5, 8, 3], np.int32)
    table = S.fp8_experts_to_device(a, device, slots=torch.from_numpy(slots).to(device), experts=E)
    tiled = wa.prefill_layout(table)
    # empty batches
    x0 = torch.empty(0, H, dtype=torch.bfloat16, device=device)
    i0 = torch.empty(0, 2, dtype=torch.int32, device=device)
    w0 = torch.empty(0, 2, dtype=torch.float32, device=device)
    for tab in (table, tiled):
        assert wa.moe_fp8(x0, i0, w0, tab).shape == (0, H)
        assert wa.experts_fp8(x0, i0, tab).shape == (0, 2, H)
    # K = 1 and the slot map (pool entry slots[e] holds expert e)
    T = 200
    x = S.bf16_normal_np(rng, (T, H))
    idx = rng.integers(0, E, size=(T, 1)).astype(np.int32)
    w = rng.uniform(0.2, 1.0, size=(T, 1)).astype(np.float32)
    xt, it, wt = S.bf16_bits_to_tensor(x, device), torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device)
    pool_ex = oracle_experts(a, pool)
    ex = {e: pool_ex[int(slots[e])] for e in range(E)}
    xf = S.bf16_bits_to_f32(x)
    want = M.combine(M.routed_outputs(xf, idx, ex, ffn=M.fp8_expert_ffn), w, None, None)
    for tab, what in ((table, "slots"), (tiled, "slots tiled")):
        y = wa.moe_fp8(xt, it, wt, tab)
        close(y.float().cpu().numpy(), want, what)
    # an out-of-range id: rejected when validated; otherwise its pair contributes nothing
    bad = it.clone()
    bad[0, 0] = E
    with pytest.raises(ValueError):
        wa.moe_fp8(xt, bad, wt, table, validate=True)
    out = wa.experts_fp8(xt, bad, table)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0, 0]).item() == 0
    close(out[1:, 0].float().cpu().numpy(), M.routed_outputs(xf, idx, ex, ffn=M.fp8_expert_ffn)[1:, 0], "valid pairs")


# ----------------------------------------------------------------------------- V4.1 FP8 (E8M0 32x32 blocks)

def test_dequant_fp8_e8m0_bit_exact(device):
    """wm_dequant_fp8_e8m0 against the oracle (dequant_fp8, deepseek_v41/dequant.py:45-50) for
    every E4M3 code under scale bytes 10..245 (the products stay normal fp32 numbers), on a
    ragged shape whose last 32 x 32 blocks are cropped; the NaN codes give NaN."""
    rng = np.random.default_rng(5)
    rows, cols = 70, 8 * 256 + 24
    w = np.tile(np.arange(256, dtype=np.uint8), (rows, cols // 256 + 1))[:, :cols].copy()
    rng.shuffle(w, axis=1)
    s = rng.integers(10, 246, size=(-(-rows // 32), -(-cols // 32)), dtype=np.uint8)
    got = wa.dequant_fp8_e8m0(torch.from_numpy(w).to(device), torch.from_numpy(s).to(device)).cpu().numpy()
    nan = (w & 127) == 127
    want = F.dequant_fp8_e8m0(np.where(nan, 0, w).astype(np.uint8), s)
    assert np.all(np.isnan(got[nan]))
    np.testing.assert_array_equal(got[~nan], want[~nan])


V41 = (5120, 2304)   # hidden, moe_inter_dim of the V4.1 release (deepseek_v41/config.py:31-33)


@pytest.mark.parametrize("T", [1, 4, 300])
def test_v41_fp8_shared_expert_and_routed(device, T):
    """The V4.1 shared expert's format (E4M3 with E8M0 32x32 blocks, deepseek_v41/moe.py:77-93)
    at its hidden 5120 / intermediate 2304: T = 1 and 4 take the fused GEMV (2304 is not a
    multiple of 1024, so the last chunk of each down row is partial), T = 300 the grouped GEMM
    with the E8M0 bytes as MFMA scales; the prefill tile layout gives the row layout's output
    bit for bit. Routed experts of the same format, clamped SwiGLU (limit 10)."""
    H, I = V41
    E, K = 6, 2
    rng = np.random.default_rng(T + 91)
    a = S.fp8_experts_np(rng, E, H, I, scale_format=1)
    sh = S.fp8_experts_np(rng, 1, H, I, scale_format=1)
    x = S.bf16_normal_np(rng, (T, H))
    idx = np.stack([rng.permutation(E)[:K] for _ in range(T)]).astype(np.int32)
    w = rng.uniform(0.1, 1.0, size=(T, K)).astype(np.float32)
    rows = S.fp8_experts_to_device(a, device, swiglu_limit=10.0)
    rows_sh = S.fp8_experts_to_device(sh, device, swiglu_limit=10.0)
    assert rows.scale_format == 1
    xt, it, wt = S.bf16_bits_to_tensor(x, device), torch.from_numpy(idx).to(device), torch.from_numpy(w).to(device)
    y = wa.moe_fp8(xt, it, wt, rows, rows_sh, None)
    out = wa.experts_fp8(xt, it, rows)
    torch.cuda.synchronize()
    xf = S.bf16_bits_to_f32(x)
    check = np.arange(T) if T <= 4 else np.linspace(0, T - 1, 16).astype(np.int64)
    ex = oracle_experts(a, E)
    routed = M.routed_outputs(xf[check], idx[check], ex, ffn=M.fp8_expert_ffn, limit=10.0)
    shared = M.fp8_expert_ffn(xf[check], oracle_experts(sh, 1)[0], limit=10.0)
    close(y.float().cpu().numpy()[check], M.combine(routed, w[check], shared, None), f"V4.1 FP8 layer T={T}")
    close(out.float().cpu().numpy()[check], routed, f"V4.1 FP8 router order T={T}")
    if T == 300:
        tiled, tiled_sh = wa.prefill_layout(rows), wa.prefill_layout(rows_sh)
        assert torch.equal(wa.moe_fp8(xt, it, wt, tiled, tiled_sh, None), y)
