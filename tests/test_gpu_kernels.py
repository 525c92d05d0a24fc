"""GPU parity of the format, routing and permute kernels against the oracle.

Bar: bit-exact for dequantised weights, top-k indices and permutation lists;
routing weights (fp32 transcendental math) within 2e-6 relative.
"""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import formats as F
from oracle import moe as M
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy()


# ----------------------------------------------------------------------------- formats

@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
def test_dequant_mxfp4_every_code_and_scale_bit_exact(device, out_dtype):
    # 256 rows (one per scale byte) x 64 values: every code appears at every scale.
    rng = np.random.default_rng(0)
    codes = np.tile(np.arange(16, dtype=np.uint8), 4)
    packed = np.stack([F.pack_mxfp4_codes(rng.permutation(codes)) for _ in range(256)])   # [256, 8] u32
    scales = np.repeat(np.arange(256, dtype=np.uint8)[:, None], 2, axis=1)               # [256, 2]
    want = F.dequant_mxfp4(packed, scales)
    got = wa.dequant_mxfp4(torch.from_numpy(packed.view(np.int32)).to(device), torch.from_numpy(scales).to(device),
                           out_dtype)
    got = _np(got.float())
    if out_dtype == torch.bfloat16:
        want = F.bf16_round_f32(want)  # exact: every decoded value is a bf16
        want = np.where(np.isnan(F.dequant_mxfp4(packed, scales)), np.nan, want)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(want))
    np.testing.assert_array_equal(got[~np.isnan(got)], want[~np.isnan(want)])


def test_dequant_mxfp4_baseline_distribution(device):
    rng = np.random.default_rng(1)
    a = S.mxfp4_experts_np(rng, 2, 2048, 512)
    for name, sname in (("gate_up", "gate_up_scales"), ("down", "down_scales")):
        p, s = a[name].reshape(-1, a[name].shape[-1]), a[sname].reshape(-1, a[sname].shape[-1])
        got = wa.dequant_mxfp4(torch.from_numpy(p.view(np.int32)).to(device), torch.from_numpy(s).to(device))
        np.testing.assert_array_equal(_np(got), F.dequant_mxfp4(p, s))


def test_dequant_fp8_blocks_bit_exact_with_ragged_edges(device):
    rng = np.random.default_rng(2)
    w = rng.integers(0, 256, size=(300, 200)).astype(np.uint8)
    w = np.where((w & 0x7F) == 0x7F, w ^ 1, w).astype(np.uint8)
    s = (rng.random((3, 2)) * 2).astype(np.float32)
    got = wa.dequant_fp8_blocks(torch.from_numpy(w).to(device), torch.from_numpy(s).to(device))
    np.testing.assert_array_equal(_np(got), F.dequant_fp8_blocks(w, s))


# ----------------------------------------------------------------------------- routing

@pytest.mark.parametrize("tokens,experts,k", [(16, 64, 4), (1, 512, 10), (333, 512, 10), (64, 1000, 32), (5, 7, 7)])
def test_route_softmax_topk_indices_exact(device, tokens, experts, k):
    rng = np.random.default_rng(tokens + experts)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    logits[:, ::5] = np.round(logits[:, ::5])            # plant exact ties
    for norm in (True, False):
        idx, w, probs = wa.route_softmax_topk(torch.from_numpy(logits).to(device), k, norm, probabilities=True)
        want_idx, want_w = M.route_softmax_topk(logits, k, norm)
        np.testing.assert_array_equal(_np(idx), want_idx)
        np.testing.assert_allclose(_np(w), want_w, rtol=2e-6, atol=1e-7)
        p = np.exp(logits.astype(np.float64) - logits.max(-1, keepdims=True))
        np.testing.assert_allclose(_np(probs), p / p.sum(-1, keepdims=True), rtol=2e-6, atol=1e-8)


@pytest.mark.parametrize("experts,k", [(512, 10), (100, 4), (64, 8)])
def test_route_softmax_topk_signed_zero_and_masked_logits(device, experts, k):
    """Ties between +0 and -0 (equal values: the lower index wins), masked experts (-inf
    logits) and rows whose top k must include masked experts (ties among -inf, again to the
    lower index): indices equal the oracle's, weights match (masked ones are 0)."""
    rng = np.random.default_rng(experts + k)
    logits = rng.standard_normal((6, experts)).astype(np.float32)
    logits[0] = 0.0
    logits[0, rng.choice(experts, experts // 2, replace=False)] = -0.0
    logits[1, rng.choice(experts, experts // 2, replace=False)] = -np.inf
    logits[2] = -np.inf
    logits[2, rng.choice(experts, k - 2, replace=False)] = rng.standard_normal(k - 2)
    logits[3] = np.where(rng.random(experts) < 0.5, np.float32(0.0), np.float32(-0.0))
    logits[3, ::7] = 0.5
    logits[4] = np.round(logits[4])
    logits[4, ::3] = -0.0
    logits[5, ::2] = -np.inf
    for norm in (True, False):
        idx, w = wa.route_softmax_topk(torch.from_numpy(logits).to(device), k, norm)
        want_idx, want_w = M.route_softmax_topk(logits, k, norm)
        np.testing.assert_array_equal(_np(idx), want_idx)
        np.testing.assert_allclose(_np(w), want_w, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("experts,k", [(512, 10), (1000, 16), (128, 4)])
def test_route_topk_candidate_set_edges(device, experts, k):
    """Rows around the top-k's prefilter (the candidates are the keys at or above the k-th
    largest per-lane maximum, ranked among themselves when at most 64, else a full radix
    walk): exactly 64 and 65 copies of the maximum, 100 copies, the k-th value tied 20 times
    after k - 1 distinct larger ones, and copies placed in one lane (ids 64 apart)."""
    rng = np.random.default_rng(experts * 7 + k)
    logits = rng.standard_normal((7, experts)).astype(np.float32)
    for row, copies in ((0, 64), (1, 65), (2, 100)):
        logits[row, rng.choice(experts, copies, replace=False)] = 5.0
    logits[3, :] = rng.standard_normal(experts).astype(np.float32) - 3.0
    logits[3, :k - 1] = np.arange(k - 1, 0, -1, dtype=np.float32) + 10.0
    logits[3, rng.choice(np.arange(k, experts), 20, replace=False)] = 5.0
    logits[4, ::64] = 7.0                    # the maxima share one lane
    logits[5, 1::64] = logits[5, 1::64] + 9.0
    logits[6, :] = np.float32(0.5)           # every key equal
    for norm in (True, False):
        idx, w = wa.route_softmax_topk(torch.from_numpy(logits).to(device), k, norm)
        want_idx, want_w = M.route_softmax_topk(logits, k, norm)
        np.testing.assert_array_equal(_np(idx), want_idx)
        np.testing.assert_allclose(_np(w), want_w, rtol=2e-6, atol=1e-7)


def test_route_softmax_c1_router_linear(device):
    # C1: router weight bf16 N(0, 0.02) [64, 1024], x bf16 N(0, 1) [16, 1024], seed 0.
    rng = np.random.default_rng(0)
    x_bits = S.bf16_normal_np(rng, (16, 1024))
    wr_bits = S.bf16_normal_np(rng, (64, 1024), 0.02)
    x = S.bf16_bits_to_tensor(x_bits, device)
    wr = S.bf16_bits_to_tensor(wr_bits, device)
    logits = wa.linear_bf16(x, wr)
    want = S.bf16_bits_to_f32(x_bits).astype(np.float64) @ S.bf16_bits_to_f32(wr_bits).astype(np.float64).T
    np.testing.assert_allclose(_np(logits), want, rtol=1e-5, atol=1e-5)
    idx, w = wa.route_softmax_topk(logits, 4)
    want_idx, want_w = M.route_softmax_topk(_np(logits), 4)
    np.testing.assert_array_equal(_np(idx), want_idx)
    np.testing.assert_allclose(_np(w), want_w, rtol=2e-6)


def _scored_case(rng, tokens, experts, func, groups, topk_groups, k):
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    bias = (rng.standard_normal(experts) * 0.05).astype(np.float32)
    # planted ties: tokens whose logits repeat one value, or repeat blocks of experts, so
    # that biased scores (bias 0 there) and group scores tie exactly and the lower index wins
    bias[: experts // 4] = 0.0
    logits[0] = 0.25
    logits[1, : experts // 4] = np.tile(logits[1, :4], experts // 16)
    logits[2, :] = np.round(logits[2, :] * 4) / 4
    return logits, bias


@pytest.mark.parametrize("func,groups,topk_groups,k,experts",
                         [("sigmoid", 8, 4, 8, 256), ("sigmoid", 1, 1, 8, 256), ("sqrtsoftplus", 1, 1, 6, 384),
                          ("softmax", 1, 1, 6, 64), ("softmax", 1, 1, 10, 512), ("sigmoid", 4, 2, 3, 16),
                          ("sqrtsoftplus", 8, 4, 8, 256), ("sigmoid", 16, 4, 8, 512)])
def test_route_scored_matches_oracle(device, func, groups, topk_groups, k, experts):
    """Indices bit-exact: the device evaluates the scores in the stated fp32 arithmetic that
    the oracle restates op for op (route_device.h, oracle/moe.py score_f32)."""
    rng = np.random.default_rng(experts + k)
    logits, bias = _scored_case(rng, 512, experts, func, groups, topk_groups, k)
    logits[3] = logits[3] * 60.0                          # saturated scores: exp under/overflow
    idx, w = wa.route_scored(torch.from_numpy(logits).to(device), torch.from_numpy(bias).to(device), k, func,
                             route_scale=2.5, n_groups=groups, topk_groups=topk_groups)
    want_idx, want_w = M.route_scored(logits, bias, k, func, 2.5, True, groups, topk_groups)
    np.testing.assert_array_equal(_np(idx), want_idx)
    np.testing.assert_allclose(_np(w), want_w, rtol=2e-6, atol=1e-30)


# ----------------------------------------------------------------------------- permute

@pytest.mark.parametrize("tokens,k,experts,skew", [(1, 10, 512, False), (16, 4, 64, False), (1000, 10, 512, True),
                                                    (16384, 10, 512, True), (7, 3, 1, False)])
def test_permute_exact(device, tokens, k, experts, skew):
    rng = np.random.default_rng(tokens)
    logits = rng.standard_normal((tokens, experts)).astype(np.float32)
    if skew:
        logits += S.zipf_bias(experts, 1.1, rng)
    idx = M.topk_desc(logits, k) if k <= experts else rng.integers(0, experts, (tokens, k))
    if experts == 1:
        idx = np.zeros((tokens, k), np.int32)
    p = wa.permute(torch.from_numpy(idx.astype(np.int32)).to(device), experts, 128)
    want = M.permute(idx, experts, 128)
    np.testing.assert_array_equal(_np(p.order), want.order)
    np.testing.assert_array_equal(_np(p.inverse), want.inverse)
    np.testing.assert_array_equal(_np(p.offsets), want.offsets)
    n = int(_np(p.tile_count)[0])
    assert n == len(want.tiles)
    np.testing.assert_array_equal(_np(p.tiles)[:n], want.tiles)


def test_permute_skips_invalid_ids(device):
    idx = np.array([[0, 5], [9, 1], [-1, 0]], np.int32)
    p = wa.permute(torch.from_numpy(idx).to(device), 8, 4)
    inv = _np(p.inverse)
    assert inv[2] == -1 and inv[4] == -1
    assert _np(p.offsets)[-1] == 4
    np.testing.assert_array_equal(_np(p.order)[:4], [0, 5, 3, 1])


def test_permute_empty(device):
    p = wa.permute(torch.empty(0, 10, dtype=torch.int32, device=device), 512)
    assert int(_np(p.tile_count)[0]) == 0 and int(_np(p.offsets)[-1]) == 0


@pytest.mark.parametrize("H", [256, 640, 2048])
def test_split_rows_e2m3_bit_exact(device, H):
    # the prefill GEMMs' activation terms (wm_split_rows_e2m3) against the restatement, byte
    # for byte (padding bytes 200-207 of each step excepted), on N(0,1) rows and on rows built
    # to reach the edges: zero blocks, blocks many binades apart, tiny negatives that round to
    # -0 beside a large value, exact E2M3 ties, and maxima that saturate (7.9 x 2^k).
    rng = np.random.default_rng(H)
    R = 24
    x = rng.standard_normal((R, H)).astype(np.float32)
    x[1] = 0.0
    x[2] *= np.exp2(rng.integers(-40, 40, H // 32)).repeat(32).astype(np.float32)
    x[3, ::32] = 50.0
    x[3, 1::32] = -1e-3
    x[4] = np.float32(2.0 ** -5) * np.tile(F.E2M3_MAGNITUDES[16:] + np.float32(0.125), H // 16)[:H]
    x[5, ::32] = np.float32(7.9 * 2.0 ** 6)
    x[6, :] = -x[6, :]
    bits = F.bf16_round(x)
    got = wa.split_rows_e2m3(S.bf16_bits_to_tensor(bits, device)).cpu().numpy()
    want = F.split_rows_e2m3(F.bf16_bits_to_f32(bits))
    np.testing.assert_array_equal(got[..., :200], want[..., :200])


@pytest.mark.parametrize("H", [128, 2048, 7168])
def test_split_rows_e4m3_bit_exact(device, H):
    # the bf16-exact activation terms (wm_split_rows_e4m3) against the restatement, byte for
    # byte (terms and scale dwords), on N(0,1) rows and on rows built to reach the edges: zero
    # blocks, blocks many binades apart, tiny negatives that round to -0 beside a large value,
    # E4M3 ties in the hi and the lo term, block maxima at a binade's top, and rows of one sign
    rng = np.random.default_rng(H + 1)
    R = 24
    x = rng.standard_normal((R, H)).astype(np.float32)
    x[1] = 0.0
    x[2] *= np.exp2(rng.integers(-40, 40, H // 32)).repeat(32).astype(np.float32)
    x[3, ::32] = 50.0
    x[3, 1::32] = -1e-5
    x[4] = np.tile(np.float32(128.0) + np.arange(32, dtype=np.float32) * 8 + 4, H // 32)[:H]   # hi ties
    x[5] = np.tile(np.float32(200.0) + np.arange(32, dtype=np.float32) * 0.75, H // 32)[:H]   # lo ties
    x[6, ::32] = np.float32(255.9 * 2.0 ** 9)
    x[7, :] = -np.abs(x[7, :])
    bits = F.bf16_round(x)
    terms, scales = wa.split_rows_e4m3(S.bf16_bits_to_tensor(bits, device))
    want_t, want_s = F.split_rows_e4m3(F.bf16_bits_to_f32(bits))
    np.testing.assert_array_equal(terms.cpu().numpy(), want_t)
    np.testing.assert_array_equal(scales.cpu().numpy().view(np.uint32), want_s)
    # and the terms reproduce every bf16 value at or above 2^-13 of its block's maximum
    xf = F.bf16_bits_to_f32(bits).astype(np.float64)
    back = F.split_rows_e4m3_value(want_t, want_s)
    blk = np.abs(xf).reshape(R, -1, 32).max(-1, keepdims=True)
    keep = (np.abs(xf).reshape(R, -1, 32) >= blk * 2.0 ** -13).reshape(R, H)
    np.testing.assert_array_equal(back[keep], xf[keep])
