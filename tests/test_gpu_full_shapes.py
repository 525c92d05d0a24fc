"""GPU parity at the full shapes the benchmark times (C4 prefill and decode, C5).

The oracle cannot afford every token at these sizes, so each test checks a seeded sample
of tokens against the oracle's fp32 dequant-then-matmul (relative L2 <= 1e-2, max |err|
<= 2e-2 max |ref|) and the whole output through size-independent properties:
- the prefill tile layout gives the row layout's output bit for bit;
- two calls over complementary pair masks give the one-call per-pair output bit for bit.
C4 routes the sampled tokens into a few experts (their other logits at -10) so the oracle
dequantizes 17 experts instead of all 257, while the rest of the 4,096 tokens route freely
(sigmoid, bias select, 8 groups / top 4). C5 checks every layer of the verify step from
its own inputs (teacher forcing), the LM head, and acceptance.
"""
from dataclasses import replace

import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import formats as F
from oracle import moe as M
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    mx = np.abs(got - want).max() / np.abs(want).max()
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"
    print(f"{what}: rel L2 {rel:.2e} max {mx:.2e}", flush=True)
    return rel


def mx_expert(tab, e):
    g = lambda t: t[e].cpu().numpy()  # noqa: E731
    return M.MXFP4Expert(g(tab.gate_up).view(np.uint32), g(tab.gate_up_scales), g(tab.down).view(np.uint32),
                         g(tab.down_scales))


def fp8_expert(tab, e):
    I = tab.inter
    w13, s13 = tab.w13[e].cpu().numpy(), tab.w13_scales[e].cpu().numpy()
    return M.FP8Expert(w13[:I], s13[:I // 128], w13[I:], s13[I // 128:], tab.w2[e].cpu().numpy(),
                       tab.w2_scales[e].cpu().numpy())


def test_c3_prefill_full_size(device):
    T, H, E, I, K = 16384, 2048, 512, 512, 10
    g = torch.Generator(device=device)
    g.manual_seed(11)
    experts = S.mxfp4_experts_device(E, H, I, device, g)
    shared = S.mxfp4_experts_device(1, H, I, device, g)
    gate = (torch.randn(H, device=device, generator=g) * 0.02).to(torch.bfloat16)
    rng = np.random.default_rng(11)
    logits = torch.randn(T, E, device=device, generator=g) + torch.from_numpy(S.zipf_bias(E, 1.1, rng)).to(device)
    x = torch.randn(T, H, device=device, generator=g).to(torch.bfloat16)
    idx, w = wa.route_softmax_topk(logits, K)
    tiled, tiled_shared = wa.prefill_layout(experts), wa.prefill_layout(shared)
    y = wa.moe_mxfp4(x, idx, w, tiled, tiled_shared, gate)
    y_rows = wa.moe_mxfp4(x, idx, w, experts, shared, gate)
    assert torch.equal(y, y_rows), "tile layout differs from the row layout"
    # sampled tokens against the oracle
    sample = np.sort(rng.choice(T, 256, replace=False))
    ids, ws = idx.cpu().numpy()[sample], w.cpu().numpy()[sample]
    xs = x[torch.from_numpy(sample).to(device)].float().cpu().numpy()
    ex = {int(e): mx_expert(experts, int(e)) for e in np.unique(ids)}
    print(f"C3 sample: {len(ex)} distinct experts", flush=True)
    routed = M.routed_outputs(xs, ids, ex)
    sh = M.expert_ffn(xs, mx_expert(shared, 0))
    want = M.combine(routed, ws, sh, xs.astype(np.float64) @ gate.float().cpu().numpy().astype(np.float64))
    rel = close(y.float().cpu().numpy()[sample], want, "C3 sampled tokens, E4M3 activation terms")
    # the faster E2M3 terms (about 7 significant bits of each block's maximum) on the same call
    y6 = wa.moe_mxfp4(x, idx, w, replace(tiled, act_terms="e2m3"), replace(tiled_shared, act_terms="e2m3"), gate)
    rel6 = close(y6.float().cpu().numpy()[sample], want, "C3 sampled tokens, E2M3 activation terms")
    assert rel < rel6, "the bf16-exact terms should be the closer ones"
    # reference precision: the reference's own bf16 arithmetic (projections, SwiGLU steps, rows,
    # weighted rows, sum and shared term each rounded to bf16) sits this far from the same fp32
    # oracle; the bf16-exact path (rows and output rounded to bf16 once each) sits no farther
    gl = xs.astype(np.float64) @ gate.float().cpu().numpy().astype(np.float64)
    ref = M.combine_bf16_steps(M.routed_outputs(xs, ids, ex, ffn=M.expert_ffn_bf16_steps), ws,
                               M.expert_ffn_bf16_steps(xs, mx_expert(shared, 0)), gl)
    rel_ref = float(np.linalg.norm(ref - want) / np.linalg.norm(want))
    print(f"C3 the reference's bf16 arithmetic against the fp32 oracle: rel L2 {rel_ref:.2e}", flush=True)
    assert rel <= rel_ref
    # what is left is mostly the bf16 rounding of the per-pair rows (the StreamingExperts
    # contract returns them as bf16, qwen4_exp.py:853-904) and of the output
    want_rows = M.combine(F.bf16_round_f32(routed), ws, F.bf16_round_f32(sh), gl)
    got = y.float().cpu().numpy()[sample].astype(np.float64)
    rel_rows = float(np.linalg.norm(got - want_rows) / np.linalg.norm(want_rows))
    print(f"C3 E4M3 against the oracle with bf16 rows: rel L2 {rel_rows:.2e}", flush=True)
    assert rel_rows <= 2.5e-3
    # per-pair outputs: complementary masks give the one-call rows bit for bit
    full = wa.experts_mxfp4(x, idx, tiled)
    mask = torch.from_numpy(rng.random((T, K)) < 0.5).to(device)
    out = torch.empty_like(full)
    none = torch.full_like(idx, -1)
    wa.experts_mxfp4(x, torch.where(mask, idx, none), tiled, out=out)
    wa.experts_mxfp4(x, torch.where(mask, none, idx), tiled, out=out)
    assert torch.equal(out, full)


def test_c3_prefill_all_tokens_on_ten_experts(device):
    """The most skewed routing top-10 allows: 8,192 tokens all on the same 10 experts (64 row
    tiles each, so one expert's tiles span several XCDs' shares of the tile list), against
    the oracle on a sample and the row layout bit for bit."""
    T, H, E, I, K = 8192, 2048, 512, 512, 10
    g = torch.Generator(device=device)
    g.manual_seed(13)
    experts = S.mxfp4_experts_device(E, H, I, device, g)
    shared = S.mxfp4_experts_device(1, H, I, device, g)
    gate = (torch.randn(H, device=device, generator=g) * 0.02).to(torch.bfloat16)
    hot = torch.tensor([3, 17, 64, 100, 200, 256, 300, 400, 450, 511], device=device)
    logits = torch.randn(T, E, device=device, generator=g)
    logits[:, hot] += 20.0
    x = torch.randn(T, H, device=device, generator=g).to(torch.bfloat16)
    idx, w = wa.route_softmax_topk(logits, K)
    assert set(np.unique(idx.cpu().numpy()).tolist()) == set(hot.cpu().numpy().tolist())
    tiled, tiled_shared = wa.prefill_layout(experts), wa.prefill_layout(shared)
    y = wa.moe_mxfp4(x, idx, w, tiled, tiled_shared, gate)
    y_rows = wa.moe_mxfp4(x, idx, w, experts, shared, gate)
    assert torch.equal(y, y_rows), "tile layout differs from the row layout"
    rng = np.random.default_rng(13)
    sample = np.sort(rng.choice(T, 64, replace=False))
    ids, ws = idx.cpu().numpy()[sample], w.cpu().numpy()[sample]
    xs = x[torch.from_numpy(sample).to(device)].float().cpu().numpy()
    ex = {int(e): mx_expert(experts, int(e)) for e in np.unique(ids)}
    routed = M.routed_outputs(xs, ids, ex)
    sh = M.expert_ffn(xs, mx_expert(shared, 0))
    want = M.combine(routed, ws, sh, xs.astype(np.float64) @ gate.float().cpu().numpy().astype(np.float64))
    close(y.float().cpu().numpy()[sample], want, "hot experts, sampled tokens")


def test_c4_prefill_full_size(device):
    T, H, E, I, K = 4096, 7168, 256, 2048, 8
    g = torch.Generator(device=device)
    g.manual_seed(12)
    experts = S.fp8_experts_device(E, H, I, device, g)
    shared = S.fp8_experts_device(1, H, I, device, g)
    bias = torch.randn(E, device=device, generator=g) * 0.1
    rng = np.random.default_rng(12)
    logits = torch.randn(T, E, device=device, generator=g)
    sample = np.sort(rng.choice(T, 64, replace=False))
    chosen = np.concatenate([np.arange(4) + 32 * grp for grp in (0, 2, 4, 6)])  # 16 experts over 4 groups
    hot = torch.full((len(sample), E), -10.0, device=device)
    hot[:, torch.from_numpy(chosen).to(device)] = torch.randn(len(sample), len(chosen), device=device,
                                                              generator=g) + 3.0
    logits[torch.from_numpy(sample).to(device)] = hot
    x = torch.randn(T, H, device=device, generator=g).to(torch.bfloat16)
    idx, w = wa.route_scored(logits, bias, K, "sigmoid", 2.5, True, 8, 4)
    want_idx, want_w = M.route_scored(logits.cpu().numpy(), bias.cpu().numpy(), K, "sigmoid", 2.5, True, 8, 4)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    y_rows = wa.moe_fp8(x, idx, w, experts, shared, None)
    tiled, tiled_shared = wa.prefill_layout(experts), wa.prefill_layout(shared)
    y = wa.moe_fp8(x, idx, w, tiled, tiled_shared, None)
    assert torch.equal(y, y_rows), "tile layout differs from the row layout"
    ids, ws = want_idx[sample], w.cpu().numpy()[sample]
    assert set(np.unique(ids).tolist()) <= set(chosen.tolist())
    xs = x[torch.from_numpy(sample).to(device)].float().cpu().numpy()
    ex = {int(e): fp8_expert(experts, int(e)) for e in np.unique(ids)}
    routed = M.routed_outputs(xs, ids, ex, ffn=M.fp8_expert_ffn)
    want = M.combine(routed, ws, M.fp8_expert_ffn(xs, fp8_expert(shared, 0)), None)
    rel = close(y.float().cpu().numpy()[sample], want, "C4 sampled tokens, E4M3 activation terms")
    y6 = wa.moe_fp8(x, idx, w, replace(tiled, act_terms="e2m3"), replace(tiled_shared, act_terms="e2m3"), None)
    rel6 = close(y6.float().cpu().numpy()[sample], want, "C4 sampled tokens, E2M3 activation terms")
    assert rel < rel6, "the bf16-exact terms should be the closer ones"
    # reference precision: the V4.1 reference's arithmetic (bf16 projections, fp32 SwiGLU, fp32
    # routed rows, bf16 shared row and output) against the same fp32 oracle
    ref = F.bf16_round_f32(M.combine(M.routed_outputs(xs, ids, ex, ffn=M.fp8_expert_ffn_bf16_steps), ws,
                                     M.fp8_expert_ffn_bf16_steps(xs, fp8_expert(shared, 0), shared=True), None))
    rel_ref = float(np.linalg.norm(ref - want) / np.linalg.norm(want))
    print(f"C4 the reference's arithmetic against the fp32 oracle: rel L2 {rel_ref:.2e}", flush=True)
    assert rel <= rel_ref
    want_rows = M.combine(F.bf16_round_f32(routed), ws, F.bf16_round_f32(M.fp8_expert_ffn(xs, fp8_expert(shared, 0))),
                          None)
    got = y.float().cpu().numpy()[sample].astype(np.float64)
    rel_rows = float(np.linalg.norm(got - want_rows) / np.linalg.norm(want_rows))
    print(f"C4 E4M3 against the oracle with bf16 rows: rel L2 {rel_rows:.2e}", flush=True)
    assert rel_rows <= 2.5e-3


def fp8_expert_any(tab, e):
    """One FP8 expert of a device table as the oracle's FP8Expert, either scale format."""
    I, fmt = tab.inter, tab.scale_format
    b = I // (32 if fmt else 128)
    w13, s13 = tab.w13[e].cpu().numpy(), tab.w13_scales[e].cpu().numpy()
    return M.FP8Expert(w13[:I], s13[:b], w13[I:], s13[b:], tab.w2[e].cpu().numpy(), tab.w2_scales[e].cpu().numpy(),
                       scale_format=fmt)


@pytest.mark.parametrize("fmt", [0, 1], ids=["fp32-128", "e8m0-32"])
def test_c4_decode_full_size(device, fmt):
    """The C4 decode layer at its full shape (H 7168, I 2048, 256 experts, top-8 over 8 groups /
    top 4, sigmoid scores with bias, the ungated shared expert), one token a call through the
    fused GEMV path, as the bench runs it: routes bit-exact and every output element against
    the oracle (each token's 8 experts and the shared one dequantized), for two tokens."""
    H, E, I, K = 7168, 256, 2048, 8
    g = torch.Generator(device=device)
    g.manual_seed(13 + fmt)
    experts = S.fp8_experts_device(E, H, I, device, g, scale_format=fmt)
    shared = S.fp8_experts_device(1, H, I, device, g, scale_format=fmt)
    bias = torch.randn(E, device=device, generator=g) * 0.1
    sh = fp8_expert_any(shared, 0)
    for t in range(2):
        logits = torch.randn(1, E, device=device, generator=g)
        x = torch.randn(1, H, device=device, generator=g).to(torch.bfloat16)
        idx, w = wa.route_scored(logits, bias, K, "sigmoid", 2.5, True, 8, 4)
        want_idx, want_w = M.route_scored(logits.cpu().numpy(), bias.cpu().numpy(), K, "sigmoid", 2.5, True, 8, 4)
        np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
        y = wa.moe_fp8(x, idx, w, experts, shared, None)
        xs = x.float().cpu().numpy()
        ex = {int(e): fp8_expert_any(experts, int(e)) for e in np.unique(want_idx)}
        want = M.combine(M.routed_outputs(xs, want_idx, ex, ffn=M.fp8_expert_ffn), w.cpu().numpy(),
                         M.fp8_expert_ffn(xs, sh), None)
        close(y.float().cpu().numpy(), want, f"C4 decode token {t}, scale format {fmt}")


def test_c5_verify_step(device):
    from whallm_amd.verify import VerifyStep
    L, T, H, E, I, K, V = 4, 4, 7168, 256, 2048, 8, 129280
    g = torch.Generator(device=device)
    g.manual_seed(13)
    layers = [S.fp8_experts_device(E, H, I, device, g) for _ in range(L)]
    shared = [S.fp8_experts_device(1, H, I, device, g) for _ in range(L)]
    biases = [torch.randn(E, device=device, generator=g) * 0.1 for _ in range(L)]
    head = (torch.randn(V, H, device=device, generator=g) * H ** -0.5).to(torch.bfloat16)
    step = VerifyStep(layers, shared, biases, head, k=K)
    # every layer routes the 4 rows within 12 experts spread over 4 groups (a bounded oracle)
    rng = np.random.default_rng(13)
    router = torch.full((L, T, E), -10.0, device=device)
    for l in range(L):
        chosen = torch.from_numpy(np.concatenate([rng.choice(32, 3, replace=False) + 64 * grp
                                                  for grp in range(4)])).to(device)
        router[l][:, chosen] = torch.randn(T, len(chosen), device=device, generator=g) + 3.0
    r0 = torch.randn(T, H, device=device, generator=g)
    drafts = torch.zeros(T - 1, dtype=torch.int32, device=device)
    _, logits = step(router, r0.clone(), drafts)
    top = logits.argmax(dim=-1).to(torch.int32)
    drafts = torch.stack([top[0], top[1], (top[2] + 7) % V]).to(torch.int32)   # two accepted, then a miss
    trace = []
    residual = r0.clone()
    accept, logits = step(router, residual, drafts, trace=trace)
    assert accept.cpu().tolist() == [2, int(top[2])]
    assert accept.cpu().tolist() == list(M.verify_greedy(drafts.cpu().numpy(), logits.cpu().numpy()))
    prev = r0.cpu().numpy()
    for l, (x_l, r_l) in enumerate(trace):
        idx, w = M.route_scored(router[l].cpu().numpy(), biases[l].cpu().numpy(), K, "sigmoid", 2.5, True, 8, 4)
        xs = x_l.float().cpu().numpy()
        ex = {int(e): fp8_expert(layers[l], int(e)) for e in np.unique(idx)}
        routed = M.routed_outputs(xs, idx, ex, ffn=M.fp8_expert_ffn)
        y = M.combine(routed, w, M.fp8_expert_ffn(xs, fp8_expert(shared[l], 0)), None)
        now = r_l.cpu().numpy()
        close(now.astype(np.float64) - prev, y, f"C5 layer {l}")
        prev = now
    # the LM head on 8,192 sampled vocabulary rows plus each row's arg-max
    x_last = M.rms_norm(prev.astype(np.float64)).astype(np.float64)
    rows = np.unique(np.concatenate([rng.choice(V, 8192, replace=False), top.cpu().numpy()]))
    want = x_last @ head[torch.from_numpy(rows).to(device)].float().cpu().numpy().astype(np.float64).T
    close(logits.cpu().numpy()[:, rows], want, "C5 LM head logits")
    # the library's one C entry for the same step (wm_verify_step_fp8) equals the composition bit for bit
    residual_n = r0.clone()
    accept_n, logits_n = step.native(router, residual_n, drafts)
    assert torch.equal(accept_n, accept) and torch.equal(logits_n, logits) and torch.equal(residual_n, residual)
