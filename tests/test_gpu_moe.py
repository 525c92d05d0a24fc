"""GPU parity of the MXFP4 MoE layer against the fp32 dequant-then-matmul oracle.

Tolerance (BASELINE correctness bar, written here): relative L2 error <= 1e-2 and
max |error| <= 2e-2 * max |reference| (outputs are O(100-1000) at the benchmark
distributions, so the max-abs bar is stated relative to the output scale).
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import moe as M
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
MAX_ABS = 2e-2


def assert_close(got: np.ndarray, want: np.ndarray, what: str):
    got = got.astype(np.float64)
    want = want.astype(np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    mx = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
    assert rel <= REL_L2 and mx <= MAX_ABS, f"{what}: rel L2 {rel:.3e}, max-abs/max {mx:.3e}"
    return rel, mx


def _experts_np(a, E):
    return [M.MXFP4Expert(a["gate_up"][e], a["gate_up_scales"][e], a["down"][e], a["down_scales"][e])
            for e in range(E)]


class Layer:
    """One synthetic MXFP4 MoE layer on host (numpy) and device."""

    def __init__(self, device, seed, tokens, experts, hidden, inter, k, shared=True, up_first=False, limit=0.0,
                 skew=False):
        rng = np.random.default_rng(seed)
        self.k = k
        self.arrays = S.mxfp4_experts_np(rng, experts, hidden, inter)
        self.shared_arrays = S.mxfp4_experts_np(rng, 1, hidden, inter) if shared else None
        self.x_bits = S.bf16_normal_np(rng, (tokens, hidden))
        self.gate_bits = S.bf16_normal_np(rng, (hidden,), 0.02) if shared else None
        self.logits = rng.standard_normal((tokens, experts)).astype(np.float32)
        if skew:
            self.logits += S.zipf_bias(experts, 1.1, rng)
        self.idx, self.w = M.route_softmax_topk(self.logits, k)
        self.dev = S.experts_to_device(self.arrays, device, up_first=up_first, swiglu_limit=limit)
        self.dev_shared = (S.experts_to_device({n: v for n, v in self.shared_arrays.items()}, device,
                                               up_first=up_first, swiglu_limit=limit) if shared else None)
        self.x = S.bf16_bits_to_tensor(self.x_bits, device)
        self.gate = S.bf16_bits_to_tensor(self.gate_bits, device) if shared else None
        self.idx_d = torch.from_numpy(self.idx).to(device)
        self.w_d = torch.from_numpy(self.w).to(device)
        self.up_first, self.limit = up_first, limit

    def oracle_routed(self):
        xf = S.bf16_bits_to_f32(self.x_bits)
        return M.routed_outputs(xf, self.idx, _experts_np(self.arrays, self.arrays["gate_up"].shape[0]),
                                limit=self.limit, up_first=self.up_first)

    def oracle_layer(self):
        xf = S.bf16_bits_to_f32(self.x_bits)
        routed = self.oracle_routed()
        sh = sg = None
        if self.shared_arrays is not None:
            e = _experts_np(self.shared_arrays, 1)[0]
            sh = M.expert_ffn(xf, e, limit=self.limit, up_first=self.up_first)
            sg = xf.astype(np.float64) @ S.bf16_bits_to_f32(self.gate_bits).astype(np.float64)
        return M.combine(routed, self.w, sh, sg)

    def run(self, act_terms="e4m3"):
        dev = replace(self.dev, act_terms=act_terms)
        sh = None if self.dev_shared is None else replace(self.dev_shared, act_terms=act_terms)
        return wa.moe_mxfp4(self.x, self.idx_d, self.w_d, dev, sh, self.gate)


# T*K <= 256 takes the decode (GEMV) path, larger calls the grouped-GEMM path.
CASES = [
    # name, tokens, experts, hidden, inter, k
    ("c1-decode", 16, 64, 1024, 512, 4),          # BASELINE C1 (seed 0)
    ("c2-decode", 1, 512, 2048, 512, 10),         # one C2 layer at T=1
    ("mtp-rows", 4, 512, 2048, 512, 10),          # M=4 verify rows
    ("prefill-small", 100, 64, 1024, 512, 4),     # 400 pairs: grouped GEMM
    ("prefill-c3-shape", 512, 512, 2048, 512, 10),
    ("tiny", 3, 8, 128, 64, 2),
]


@pytest.mark.parametrize("act_terms", ["e4m3", "e2m3"])
@pytest.mark.parametrize("name,tokens,experts,hidden,inter,k", CASES, ids=[c[0] for c in CASES])
def test_moe_layer_matches_oracle(device, name, tokens, experts, hidden, inter, k, act_terms):
    # act_terms picks the grouped GEMM's activation terms (decode-sized calls take the GEMV)
    layer = Layer(device, 0, tokens, experts, hidden, inter, k)
    y = layer.run(act_terms)
    torch.cuda.synchronize()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), f"{name} {act_terms}")


@pytest.mark.parametrize("name,tokens,experts,hidden,inter,k", CASES, ids=[c[0] for c in CASES])
def test_expert_outputs_router_order(device, name, tokens, experts, hidden, inter, k):
    layer = Layer(device, 1, tokens, experts, hidden, inter, k, shared=False)
    out = wa.experts_mxfp4(layer.x, layer.idx_d, layer.dev)
    torch.cuda.synchronize()
    assert out.shape == (tokens, k, hidden)
    assert_close(out.float().cpu().numpy(), layer.oracle_routed(), name)


@pytest.mark.parametrize("tokens", [2, 200])
def test_no_shared_and_ungated_shared(device, tokens):
    layer = Layer(device, 2, tokens, 32, 256, 128, 3, shared=False)
    y = wa.moe_mxfp4(layer.x, layer.idx_d, layer.w_d, layer.dev)
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), "no shared")
    layer = Layer(device, 3, tokens, 32, 256, 128, 3, shared=True)
    y = wa.moe_mxfp4(layer.x, layer.idx_d, layer.w_d, layer.dev, layer.dev_shared, None)
    xf = S.bf16_bits_to_f32(layer.x_bits)
    sh = M.expert_ffn(xf, _experts_np(layer.shared_arrays, 1)[0])
    assert_close(y.float().cpu().numpy(), M.combine(layer.oracle_routed(), layer.w, sh, None), "ungated shared")


@pytest.mark.parametrize("tokens", [2, 150])
def test_deepseek_w13_order_and_clamped_swiglu(device, tokens):
    layer = Layer(device, 4, tokens, 16, 256, 128, 4, shared=True, up_first=True, limit=10.0)
    y = layer.run()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), "deepseek")


def test_zipf_skewed_prefill(device):
    layer = Layer(device, 5, 2048, 512, 2048, 512, 10, skew=True)
    y = layer.run()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), "zipf prefill")


def test_decode_and_prefill_paths_agree(device):
    # The same pairs through both paths: 25 tokens x 10 = 250 pairs (decode) vs 26 x 10 (prefill).
    layer = Layer(device, 6, 26, 64, 1024, 512, 10)
    y_all = layer.run()
    y_25 = wa.moe_mxfp4(layer.x[:25], layer.idx_d[:25], layer.w_d[:25], layer.dev, layer.dev_shared, layer.gate)
    torch.cuda.synchronize()
    assert_close(y_25.float().cpu().numpy(), y_all[:25].float().cpu().numpy(), "paths")


def test_edges_empty_k1_and_invalid_ids(device):
    layer = Layer(device, 7, 4, 8, 128, 64, 1)
    y = layer.run()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), "k=1")
    empty = wa.moe_mxfp4(layer.x[:0], layer.idx_d[:0], layer.w_d[:0], layer.dev, layer.dev_shared, layer.gate)
    assert empty.shape == (0, 128)
    bad = layer.idx_d.clone()
    bad[0, 0] = 8
    with pytest.raises(ValueError):
        wa.moe_mxfp4(layer.x, bad, layer.w_d, layer.dev, validate=True)
    # Unvalidated: the bad pair contributes nothing (its expert output is zero).
    out = wa.experts_mxfp4(layer.x, bad, layer.dev)
    torch.cuda.synchronize()
    assert torch.count_nonzero(out[0, 0]).item() == 0


# ----------------------------------------------------------------------------- prefill tile layout

def _tile_layout_np(region: np.ndarray, rows: int, k: int) -> np.ndarray:
    """The tile layout of one expert's weight region as a numpy reindexing (the layout the
    header states): bytes [k/128 steps][rows/16 groups][4 pieces][16 rows][16 bytes]."""
    b = np.ascontiguousarray(region).view(np.uint8).reshape(rows // 16, 16, k // 128, 4, 16)
    return b.transpose(2, 0, 3, 1, 4).reshape(-1)


def _tile_scales_np(region: np.ndarray, rows: int, k: int) -> np.ndarray:
    """[k/128 steps][rows][4 bytes] from [rows][k/32]."""
    return np.ascontiguousarray(region).reshape(rows, k // 128, 4).transpose(1, 0, 2).reshape(-1)


def test_prefill_layout_bytes(device):
    E, H, I = 3, 256, 384
    arrays = S.mxfp4_experts_np(np.random.default_rng(11), E, H, I)
    dev = S.experts_to_device(arrays, device)
    tiled = wa.prefill_layout(dev)
    torch.cuda.synchronize()
    assert tiled.tiled and tiled.gate_up.shape == dev.gate_up.shape
    for e in range(E):
        got = tiled.gate_up[e].cpu().numpy().view(np.uint8).reshape(-1)
        assert np.array_equal(got, _tile_layout_np(arrays["gate_up"][e], 2 * I, H)), f"gate_up {e}"
        got = tiled.gate_up_scales[e].cpu().numpy().reshape(-1)
        assert np.array_equal(got, _tile_scales_np(arrays["gate_up_scales"][e], 2 * I, H)), f"gate_up scales {e}"
        got = tiled.down[e].cpu().numpy().view(np.uint8).reshape(-1)
        assert np.array_equal(got, _tile_layout_np(arrays["down"][e], H, I)), f"down {e}"
        got = tiled.down_scales[e].cpu().numpy().reshape(-1)
        assert np.array_equal(got, _tile_scales_np(arrays["down_scales"][e], H, I)), f"down scales {e}"


@pytest.mark.parametrize("name,tokens,experts,hidden,inter,k", [
    ("decode-sized", 4, 64, 1024, 512, 4),       # T*K <= 256: a tiled table still takes the GEMM path
    ("prefill-small", 100, 64, 1024, 512, 4),
    ("prefill-c3-shape", 512, 512, 2048, 512, 10),
    ("odd-tiles", 200, 32, 256, 384, 3),           # a partial intermediate tile (384 = 256 + 128)
])
def test_prefill_layout_matches_oracle(device, name, tokens, experts, hidden, inter, k):
    layer = Layer(device, 21, tokens, experts, hidden, inter, k)
    tiled, tiled_shared = wa.prefill_layout(layer.dev), wa.prefill_layout(layer.dev_shared)
    y = wa.moe_mxfp4(layer.x, layer.idx_d, layer.w_d, tiled, tiled_shared, layer.gate)
    torch.cuda.synchronize()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), name)
    out = wa.experts_mxfp4(layer.x, layer.idx_d, tiled)
    torch.cuda.synchronize()
    assert_close(out.float().cpu().numpy(), layer.oracle_routed(), name + " router order")


def test_prefill_layout_deepseek_form(device):
    layer = Layer(device, 22, 150, 16, 256, 128, 4, shared=True, up_first=True, limit=10.0)
    y = wa.moe_mxfp4(layer.x, layer.idx_d, layer.w_d, wa.prefill_layout(layer.dev),
                     wa.prefill_layout(layer.dev_shared), layer.gate)
    torch.cuda.synchronize()
    assert_close(y.float().cpu().numpy(), layer.oracle_layer(), "deepseek tiled")


def test_prefill_layout_zipf_agrees_with_row_layout(device):
    layer = Layer(device, 23, 2048, 512, 2048, 512, 10, skew=True)
    y_rows = layer.run()
    y_tiled = wa.moe_mxfp4(layer.x, layer.idx_d, layer.w_d, wa.prefill_layout(layer.dev),
                           wa.prefill_layout(layer.dev_shared), layer.gate)
    torch.cuda.synchronize()
    # the two layouts feed the same bytes to the same MFMAs: identical results
    assert torch.equal(y_rows, y_tiled)
    assert_close(y_tiled.float().cpu().numpy(), layer.oracle_layer(), "zipf tiled")
