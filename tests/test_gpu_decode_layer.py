"""GPU parity of the one-launch MoE decode layer (wm_moe_layer_decode, whallm_amd.ops.DecodeLayer).

One token through a decoder layer's MoE half: x = bf16(rmsnorm(r) * w_norm), logits = x . Wr^T,
softmax top-k, y = sum_k w_k FFN_k(x) + sigmoid(x . g) FFN_shared(x), r' = r + bf16(y)
(qwen4_exp.py:1146, :1036-1051; Native/QwenNative/engine.mm:2073-2236). Checked against the
oracle from the call's own x and logits (the norm's and the router GEMV's fp32 sums may round
differently from the oracle's float64 ones):
- x within one bf16 step of the oracle's bf16(rmsnorm(r) * w) on at most 0.1% of its values;
- logits within 1e-5 of the float64 dot of the call's x with the router rows;
- indices equal the oracle's top-k of the call's logits, weights within 2e-6;
- y within relative L2 1e-2 and max |err| 2e-2 max |ref| of the oracle's fp32 dequant-then-matmul
  layer on the call's x and routes;
- r' = r + bf16(y) exactly.
The fused shapes (2048 / 512, 1024 / 512) and an unfused one (2560 / 640, the per-layer
kernels) run the same checks over successive calls (the fused launch's epochs advance) and
graph replays; a NaN residual (no valid route) ends the fused call with status 4 and leaves
the residual unchanged; a non-resident expert contributes nothing.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import moe as M
from whallm_amd import synthetic as S
from whallm_amd.ops import DecodeLayer, DecodeStackError

pytestmark = pytest.mark.gpu

SHAPES = {  # hidden, intermediate, experts, k
    "c2": (2048, 512, 512, 10),
    "c1": (1024, 512, 64, 4),
    "qwen-unfused": (2560, 640, 512, 10),
}


def close(got, want, what, rel_l2=1e-2, max_abs=2e-2):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    mx = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
    assert rel <= rel_l2 and mx <= max_abs, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"


def host_expert(tab, e):
    g = lambda t: t[e].cpu().numpy()  # noqa: E731
    return M.MXFP4Expert(g(tab.gate_up).view(np.uint32), g(tab.gate_up_scales), g(tab.down).view(np.uint32),
                         g(tab.down_scales))


class Case:
    def __init__(self, device, name, seed, slots=None, norm_weight=True):
        H, I, E, K = SHAPES[name]
        self.H, self.I, self.E, self.K = H, I, E, K
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.experts = S.mxfp4_experts_device(E, H, I, device, g)
        if slots is not None:
            self.experts = replace(self.experts, slots=slots, experts=E)
        self.shared = S.mxfp4_experts_device(1, H, I, device, g)
        self.router = (torch.randn(E, H, device=device, generator=g) * 0.05).to(torch.bfloat16)
        self.gate = (torch.randn(H, device=device, generator=g) * 0.02).to(torch.bfloat16)
        self.norm_w = (1.0 + 0.1 * torch.randn(H, device=device, generator=g)).to(torch.bfloat16) if norm_weight else None
        self.layer = DecodeLayer(self.experts, self.router, self.shared, self.gate, k=K, norm_weight=self.norm_w)
        self.g = g
        self.device = device

    def outputs(self):
        d = self.device
        return dict(y=torch.empty(self.H, dtype=torch.bfloat16, device=d),
                    x_out=torch.empty(self.H, dtype=torch.bfloat16, device=d),
                    logits_out=torch.empty(self.E, dtype=torch.float32, device=d),
                    indices_out=torch.empty(self.K, dtype=torch.int32, device=d),
                    weights_out=torch.empty(self.K, dtype=torch.float32, device=d))

    def check(self, r, r_out, out, what, skip=()):
        r = r.cpu().numpy().astype(np.float64)
        x = out["x_out"].float().cpu().numpy()
        nw = None if self.norm_w is None else self.norm_w.float().cpu().numpy()
        # GroupRMSNorm's fp32 path: normalized * weight, then one rounding to bf16
        _, want_x, _, _ = M.norm_router(r.astype(np.float32)[None], None, self.router.float().cpu().numpy(),
                                        None, nw)
        want_x = want_x[0]
        step = np.abs(want_x).astype(np.float64) * 2.0 ** -7
        diff = np.abs(x.astype(np.float64) - want_x)
        assert np.all(diff <= step + 1e-30) and np.count_nonzero(diff) <= max(2, x.size // 1000), f"{what}: x"
        logits = out["logits_out"].cpu().numpy()
        want_l = self.router.float().cpu().numpy().astype(np.float64) @ x.astype(np.float64)
        np.testing.assert_allclose(logits, want_l, rtol=1e-5, atol=1e-5)
        idx, w = M.route_softmax_topk(logits[None], self.K)
        np.testing.assert_array_equal(out["indices_out"].cpu().numpy(), idx[0])
        np.testing.assert_allclose(out["weights_out"].cpu().numpy(), w[0], rtol=2e-6, atol=1e-7)
        ex = {int(e): host_expert(self.experts, int(e)) for e in idx[0] if int(e) not in skip}
        keep = np.array([[int(e) not in skip for e in idx[0]]])
        routed = M.routed_outputs(x[None], np.where(keep, idx, idx[0, np.argmax(keep[0])]), ex)
        routed = np.where(keep[..., None], routed, 0.0)
        sh = M.expert_ffn(x[None], host_expert(self.shared, 0))
        sg = x.astype(np.float64) @ self.gate.float().cpu().numpy().astype(np.float64)
        want_y = M.combine(routed, w, sh, np.array([sg]))[0]
        y = out["y"].float().cpu().numpy()
        close(y, want_y, f"{what}: y")
        np.testing.assert_array_equal(r_out.cpu().numpy(), (r + y.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("name", list(SHAPES))
def test_decode_layer_matches_oracle(device, name):
    case = Case(device, name, seed=41)
    for call in range(3):   # successive calls: the fused launch's epochs advance
        r = torch.randn(case.H, device=device, generator=case.g)
        r_out = torch.empty_like(r)
        out = case.outputs()
        case.layer(r, r_out, **out)
        torch.cuda.synchronize()
        assert case.layer.status() == 0
        case.check(r, r_out, out, f"{name} call {call}")


def test_decode_layer_in_place_and_graph_replay(device):
    """The residual updated in place, and the call captured in a graph and replayed with eager
    work between replays: every replay equals an eager call on the same input, bit for bit."""
    case = Case(device, "c2", seed=42)
    r0 = torch.randn(case.H, device=device, generator=case.g)
    want = r0.clone()
    case.layer(want)
    torch.cuda.synchronize()
    r = r0.clone()
    stream = torch.cuda.Stream(device)
    stream.wait_stream(torch.cuda.current_stream(device))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            case.layer(r)
    torch.cuda.synchronize()
    for rep in range(3):
        r.copy_(r0)
        torch.randn(1000, device=device).sum()      # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        assert case.layer.status() == 0
        assert torch.equal(r, want), f"replay {rep}"


def test_decode_layer_no_valid_route(device):
    case = Case(device, "c2", seed=43)
    r = torch.full((case.H,), float("nan"), device=device)
    r_out = torch.zeros(case.H, device=device)
    case.layer(r, r_out)
    with pytest.raises(DecodeStackError, match="no valid route"):
        case.layer.raise_for_status()
    assert torch.count_nonzero(r_out).item() == 0
    r = torch.randn(case.H, device=device, generator=case.g)   # the state was reset: the next call runs
    out = case.outputs()
    case.layer(r, r_out, **out)
    torch.cuda.synchronize()
    assert case.layer.status() == 0
    case.check(r, r_out, out, "after a call with no valid route")


def test_decode_layer_non_resident_expert(device):
    """A slot map whose entry for some routed expert is -1: that expert contributes nothing."""
    H, I, E, K = SHAPES["c2"]
    slots = torch.arange(E, dtype=torch.int32, device=device)
    case = Case(device, "c2", seed=44, slots=slots)
    r = torch.randn(case.H, device=device, generator=case.g)
    out = case.outputs()
    case.layer(r.clone(), **out)
    torch.cuda.synchronize()
    gone = int(out["indices_out"][3].item())
    slots[gone] = -1
    r_out = torch.empty_like(r)
    out = case.outputs()
    case.layer(r, r_out, **out)
    torch.cuda.synchronize()
    assert case.layer.status() == 0
    assert gone in out["indices_out"].cpu().numpy().tolist()
    case.check(r, r_out, out, "non-resident expert", skip=(gone,))
