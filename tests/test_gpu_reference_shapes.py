"""GPU parity of the MXFP4 expert path at the reference's own model shapes.

- Qwen: hidden 2560, intermediate 640, 512 experts, top-10, shared expert of 640
  (runtime/deepseek_v4_ssd/qwen4_exp.py:31-46; expert blob regions manifest.py:37-42);
- DeepSeek V4.1: hidden 5120, intermediate 2304, 384 experts, top-6, w13 = [up; gate],
  clamped SwiGLU (limit 10) (deepseek_v41/config.py:31-48, manifest.py:29-36,
  deepseek_v41/moe.py:30-43);
- a square-ish shape, hidden 4096 / intermediate 2048.

The reference's decode GEMV takes any width that is a multiple of 32
(Native/QwenNative/kernels.metal:1190-1220); so must this path. Each shape runs at T = 1 and 4
(the fused dequant-GEMV) and T = 300 (the grouped GEMM), through wm_moe_mxfp4,
wm_experts_mxfp4 and the operator mirrors. Tolerance (written here, the BASELINE bar):
relative L2 <= 1e-2 and max |err| <= 2e-2 * max |ref| against the oracle's fp32
dequant-then-matmul.

The weights are generated on the device (the V4.1 layer is 7 GB). For the oracle's sake the
checked tokens route into a small set of experts (their other logits are pushed to -30) while
the rest of the 300 tokens route freely; at T <= 4 every token is checked.
"""
from dataclasses import replace
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import moe as M
from whallm_amd import operators as O
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu

SHAPES = {
    # name: hidden, inter, experts, k, DeepSeek form (up first, limit 10)
    "qwen": (2560, 640, 512, 10, False),
    "v41": (5120, 2304, 384, 6, True),
    "h4096": (4096, 2048, 128, 8, False),
}
SEEDS = {"qwen": 31, "v41": 32, "h4096": 33}
CHECKED = 12        # checked tokens at T = 300
FEW_EXPERTS = 16    # experts the checked tokens route into


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    rel = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    mx = np.abs(got - want).max() / max(np.abs(want).max(), 1e-30)
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"
    print(f"{what}: rel L2 {rel:.2e} max {mx:.2e}", flush=True)


def host_expert(tab, e):
    g = lambda t: t[e].cpu().numpy()  # noqa: E731
    return M.MXFP4Expert(g(tab.gate_up).view(np.uint32), g(tab.gate_up_scales), g(tab.down).view(np.uint32),
                         g(tab.down_scales))


_LAYERS = {}


def layer(device, name):
    """Device experts of one shape, built once per session (the V4.1 layer is 7 GB)."""
    if name not in _LAYERS:
        _LAYERS.clear()
        torch.cuda.empty_cache()
        H, I, E, K, ds = SHAPES[name]
        g = torch.Generator(device=device)
        g.manual_seed(SEEDS[name])
        experts = S.mxfp4_experts_device(E, H, I, device, g)
        shared = S.mxfp4_experts_device(1, H, I, device, g)
        if ds:
            experts = replace(experts, up_first=True, swiglu_limit=10.0)
            shared = replace(shared, up_first=True, swiglu_limit=10.0)
        gate = None if ds else (torch.randn(H, device=device, generator=g) * 0.02).to(torch.bfloat16)
        _LAYERS[name] = (experts, shared, gate, g)
    return _LAYERS[name]


def routes(device, name, tokens, g):
    """Top-k routes of `tokens` tokens; the checked ones use FEW_EXPERTS experts only."""
    H, I, E, K, ds = SHAPES[name]
    logits = torch.randn(tokens, E, device=device, generator=g)
    checked = np.arange(tokens) if tokens <= 4 else np.linspace(0, tokens - 1, CHECKED).astype(np.int64)
    keep = torch.zeros(E, dtype=torch.bool, device=device)
    keep[torch.randperm(E, device=device, generator=g)[:FEW_EXPERTS]] = True
    rows = torch.from_numpy(checked).to(device)
    logits[rows] = torch.where(keep, logits[rows], torch.full_like(logits[rows], -30.0))
    idx, w = wa.route_softmax_topk(logits, K)
    return idx, w, checked


def oracle(xs, ids, ws, experts, shared, gate, ds):
    lim = 10.0 if ds else 0.0
    ex = {int(e): host_expert(experts, int(e)) for e in np.unique(ids)}
    routed = M.routed_outputs(xs, ids, ex, limit=lim, up_first=ds)
    sh = M.expert_ffn(xs, host_expert(shared, 0), limit=lim, up_first=ds)
    sg = None if gate is None else xs.astype(np.float64) @ gate.float().cpu().numpy().astype(np.float64)
    return routed, M.combine(routed, ws, sh, sg)


@pytest.mark.parametrize("tokens", [1, 4, 300])
@pytest.mark.parametrize("name", list(SHAPES))
def test_layer_and_router_order_at_reference_shapes(device, name, tokens):
    H, I, E, K, ds = SHAPES[name]
    experts, shared, gate, g = layer(device, name)
    x = torch.randn(tokens, H, device=device, generator=g).to(torch.bfloat16)
    idx, w, checked = routes(device, name, tokens, g)
    y = wa.moe_mxfp4(x, idx, w, experts, shared, gate)
    out = wa.experts_mxfp4(x, idx, experts)
    torch.cuda.synchronize()
    xs = x.float().cpu().numpy()[checked]
    ids, ws = idx.cpu().numpy()[checked], w.cpu().numpy()[checked]
    routed, want = oracle(xs, ids, ws, experts, shared, gate, ds)
    close(y.float().cpu().numpy()[checked], want, f"{name} T={tokens} layer")
    close(out.float().cpu().numpy()[checked], routed, f"{name} T={tokens} router order")
    if tokens == 300:
        # every token, through a size-independent property: the per-pair rows combined on the
        # host equal the layer output within the bf16 rounding of the rows
        rows = out.float().cpu().numpy().astype(np.float64)
        sh = wa.experts_mxfp4(x, torch.zeros(tokens, 1, dtype=torch.int32, device=device), shared)
        sgv = (None if gate is None else
               x.float().cpu().numpy().astype(np.float64) @ gate.float().cpu().numpy().astype(np.float64))
        host = M.combine(rows, w.cpu().numpy(), sh.float().cpu().numpy()[:, 0], sgv)
        close(y.float().cpu().numpy(), host, f"{name} T={tokens} all tokens vs per-pair rows")


@pytest.mark.parametrize("tokens", [1, 4, 300])
def test_sparse_moe_at_qwen_shape(device, tokens):
    # SparseMoE (qwen4_exp.py:997-1051) with the reference's bf16 shared MLP (640) and its gate
    H, I, E, K, ds = SHAPES["qwen"]
    experts, _, _, g = layer(device, "qwen")
    args = SimpleNamespace(hidden_size=H, num_experts=E, shared_expert_intermediate_size=I, num_experts_per_tok=K,
                           norm_topk_prob=True)
    cache = SimpleNamespace(current_batched=lambda _l: experts, record_gather_qmm=lambda n: None)
    moe = O.SparseMoE(args, 0, cache, device=device)
    moe.gate.weight = (torch.randn(E, H, device=device, generator=g) * 0.02).to(torch.bfloat16)
    moe.shared_expert_gate.weight = (torch.randn(1, H, device=device, generator=g) * 0.02).to(torch.bfloat16)
    mats = [(torch.randn(*shape, device=device, generator=g) * 0.03).to(torch.bfloat16)
            for shape in ((I, H), (I, H), (H, I))]
    for lin, m in zip((moe.shared_expert.gate_proj, moe.shared_expert.up_proj, moe.shared_expert.down_proj), mats):
        lin.weight = m
    x = torch.randn(1, tokens, H, device=device, generator=g).to(torch.bfloat16)
    probabilities, indices = moe.route(x)
    y = moe(x, (probabilities, indices))
    torch.cuda.synchronize()
    checked = np.arange(tokens) if tokens <= 4 else np.linspace(0, tokens - 1, 4).astype(np.int64)
    xf = x.float().cpu().numpy().reshape(tokens, H)[checked]
    logits = wa.linear_bf16(x.reshape(tokens, H), moe.gate.weight).cpu().numpy()[checked]
    ids, ws = M.route_softmax_topk(logits, K)
    assert np.array_equal(indices.cpu().numpy().reshape(tokens, K)[checked], ids)
    ex = {int(e): host_expert(experts, int(e)) for e in np.unique(ids)}
    routed = M.routed_outputs(xf, ids, ex)
    gm, um, dm = (m.float().cpu().numpy().astype(np.float64) for m in mats)
    x64 = xf.astype(np.float64)
    shared = (M.silu(x64 @ gm.T) * (x64 @ um.T)) @ dm.T
    sg = x64 @ moe.shared_expert_gate.weight.float().cpu().numpy().reshape(-1).astype(np.float64)
    want = M.combine(routed, ws, shared, sg)
    close(y.float().cpu().numpy().reshape(tokens, H)[checked], want, f"SparseMoE qwen T={tokens}")


@pytest.mark.parametrize("tokens", [1, 4, 300])
def test_switchglu_at_v41_shape(device, tokens):
    # _StreamingSwitchGLU (model.py:318-385) over the V4.1 experts with ClampedSwiGLU(10)
    H, I, E, K, ds = SHAPES["v41"]
    experts, _, _, g = layer(device, "v41")
    cache = SimpleNamespace(current_batched=lambda _l: experts, record_gather_qmm=lambda n: None)
    switch = O._StreamingSwitchGLU(0, cache, O.ClampedSwiGLU(10.0))
    x = torch.randn(tokens, H, device=device, generator=g).to(torch.bfloat16)
    idx, _, checked = routes(device, "v41", tokens, g)
    out = switch(x, idx)
    torch.cuda.synchronize()
    assert out.shape == (tokens, K, H)
    xs = x.float().cpu().numpy()[checked]
    ids = idx.cpu().numpy()[checked]
    ex = {int(e): host_expert(experts, int(e)) for e in np.unique(ids)}
    close(out.float().cpu().numpy()[checked], M.routed_outputs(xs, ids, ex, limit=10.0, up_first=True),
          f"SwitchGLU v41 T={tokens}")
