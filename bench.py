#!/usr/bin/env python3
"""Benchmark of the MI355X MoE expert path (one JSON line on stdout).

Default workload ("c2-decode"): a Qwen3-Next-style
48-layer stack of MXFP4 MoE layers (H 2048, 512 experts, I 512, top-10 + one
always-on MXFP4 shared expert), one token per step, router logits N(0, 1), all
weights resident in HBM (41 GB). A step = one token through the 48 layers,
replayed from one HIP graph. The same run then times the metric's other half, one
layer at a 16,384-token prefill with Zipf(1.1)-skewed routing (
"c3-prefill"), and reports it under "prefill" in the same line (``--no-prefill`` leaves
it out; ``--config c3-prefill`` runs it alone).

Synthetic data (random-init weights of the configured shapes; no checkpoints).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E
BF16_PEAK_TFLOPS = 2500.0      # dense bf16 MFMA
FP8_PEAK_TFLOPS = 5000.0       # dense fp8 MFMA
FP4_PEAK_TFLOPS = 10100.0      # dense MXFP4 MFMA
METRIC = "MoE-layer tok/s (decode, 16K prefill) + % of HBM / MFMA roofline"
HERE = os.path.dirname(os.path.abspath(__file__))


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo), for the CPU baseline's record."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def capture_steps(device, body, n: int):
    """One graph per step input: body(j) runs the workload on step j's inputs where they lie
    in HBM, so a timed step replays graph j and stages nothing. The graphs share one memory
    pool (replays are stream-ordered); an eager run on a side stream comes first."""
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        body(0)
    torch.cuda.current_stream(device).wait_stream(side)
    torch.cuda.synchronize(device)
    graphs, pool = [], None
    for j in range(n):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, pool=pool):
            body(j)
        pool = g.pool()
        graphs.append(g)
    torch.cuda.synchronize(device)
    return graphs


# ----------------------------------------------------------------------------- workloads

class DecodeStack:
    """C2: 48-layer MXFP4 MoE decode, 1 token per step."""
    name = "c2-decode"
    # MXFP4 weights straight into scaled MFMAs against E4M3 terms of the bf16 activations,
    # fp32 accumulation
    dtype = "mxfp4"
    data = "synthetic (random-init MXFP4 weights, N(0,1) router logits and residual inputs)"

    def __init__(self, device, layers=48, hidden=2048, experts=512, inter=512, k=10, tokens=1, seed=0,
                 impl="persistent"):
        import whallm_amd as wa
        from whallm_amd import synthetic as S
        from whallm_amd.ops import MoEStack, PersistentDecodeStack
        self.L, self.H, self.E, self.I, self.K, self.T = layers, hidden, experts, inter, k, tokens
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        log(f"[bench] generating {layers} layers x {experts} MXFP4 experts on device")
        self.layers = [S.mxfp4_experts_device(experts, hidden, inter, device, g) for _ in range(layers)]
        self.shared = [S.mxfp4_experts_device(1, hidden, inter, device, g) for _ in range(layers)]
        self.gates = [(torch.randn(hidden, device=device, generator=g) * 0.02).to(torch.bfloat16)
                      for _ in range(layers)]
        self.impl = impl
        if impl == "persistent":
            self.stack = PersistentDecodeStack(self.layers, self.shared, self.gates, k=k)
        else:
            self.stack = MoEStack(self.layers, self.shared, self.gates, k=k)
        self.logits = torch.empty(layers, tokens, experts, dtype=torch.float32, device=device)
        self.residual = torch.empty(tokens, hidden, dtype=torch.float32, device=device)
        self.x_out = torch.empty(tokens, hidden, dtype=torch.bfloat16, device=device)
        self.gen = g
        self.graphs = None

    # Bytes every step must move: 11 expert blobs per layer-token (10 routed + shared)
    # plus the logits row (fp32) and the token's input and output rows (bf16).
    def expert_bytes(self):
        return 2 * self.I * self.H // 2 + 2 * self.I * self.H // 32 + self.H * self.I // 2 + self.H * self.I // 32

    def algorithmic_bytes(self):
        per_layer_token = (self.K + 1) * self.expert_bytes() + self.E * 4 + 2 * self.H * 2
        return per_layer_token * self.L * self.T

    def flops(self):
        return 2 * 3 * self.H * self.I * (self.K + 1) * self.L * self.T

    def tokens_per_step(self):
        return self.T

    def prepare_inputs(self, steps):
        self.step_logits = torch.randn(steps, self.L, self.T, self.E, device=self.device, generator=self.gen)
        self.step_embed = torch.randn(steps, self.T, self.H, device=self.device, generator=self.gen)

    def _body(self):
        if self.impl == "persistent":
            self.stack(self.logits, self.residual.view(-1), self.x_out.view(-1), check=False)
        else:
            self.stack(self.logits, self.residual, self.x_out)

    def check(self):
        if self.impl == "persistent":
            self.stack.raise_for_status()

    def _body_at(self, j):
        if self.impl == "persistent":
            self.stack(self.step_logits[j], self.step_embed[j].view(-1), self.x_out.view(-1), check=False)
        else:
            self.stack(self.step_logits[j], self.step_embed[j], self.x_out)

    def capture(self):
        self.graphs = capture_steps(self.device, self._body_at, len(self.step_logits))

    def step(self, i):
        self.graphs[i].replay()

    def config(self):
        return {"workload": "c2-decode: Qwen3-Next-style MXFP4 MoE decode, 48-layer stack, 1 token/step",
                "hidden": self.H, "experts": self.E, "moe_intermediate": self.I, "top_k": self.K,
                "shared_experts": 1, "shared_intermediate": self.I, "layers": self.L, "tokens_per_step": self.T,
                "weights": "MXFP4 E2M1 + E8M0/32, codes uniform, scale exponents uniform [-8,-2]",
                "router_logits": "N(0,1) per layer per step", "activations": "bf16",
                "hbm_resident_weight_gb": round(self.L * (self.E + 1) * self.expert_bytes() / 1e9, 2)}

    # -- CPU baseline: the numpy oracle on a bounded sample (one token, `layers` layers)
    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        from oracle import formats as F
        from whallm_amd import synthetic as S
        threads = len(os.sched_getaffinity(0))
        logits = self.step_logits[0].cpu().numpy()       # [L, T, E]
        x = F.bf16_round_f32(self.step_embed[0].cpu().numpy())
        r = x.astype(np.float64)

        def fetch(t: torch.Tensor, e):
            a = t[e].cpu().numpy()
            return a.view(np.uint32) if a.dtype == np.int32 else a

        done = 0
        elapsed = 0.0
        with ThreadPoolExecutor(threads) as pool:
            for l in range(self.L):
                ids = [int(e) for e in M.topk_desc(logits[l], self.K)[0]]
                ex = {e: M.MXFP4Expert(fetch(self.layers[l].gate_up, e), fetch(self.layers[l].gate_up_scales, e),
                                       fetch(self.layers[l].down, e), fetch(self.layers[l].down_scales, e))
                      for e in ids}
                sh = M.MXFP4Expert(fetch(self.shared[l].gate_up, 0), fetch(self.shared[l].gate_up_scales, 0),
                                   fetch(self.shared[l].down, 0), fetch(self.shared[l].down_scales, 0))
                g = S.bf16_bits_to_f32(self.gates[l].view(torch.int16).cpu().numpy().view(np.uint16))
                t0 = time.perf_counter()   # compute only: routing, 11 expert FFNs, combine, residual
                xin = M.rms_norm(r)
                idx, w = M.route_softmax_topk(logits[l], self.K)
                outs = list(pool.map(lambda e: M.expert_ffn(xin, ex[e]), [int(e) for e in idx[0]]))
                shared_out = M.expert_ffn(xin, sh)
                gate = xin.astype(np.float64) @ g.astype(np.float64)
                y = M.combine(np.stack(outs, axis=1), w, shared_out, gate)
                r = r + F.bf16_round_f32(y)
                elapsed += time.perf_counter() - t0
                done += 1
                if elapsed > budget_s:
                    break
        # The sample is `done` layer-tokens of the 48-layer stack (expert bytes fetched beforehand).
        per_token_s = elapsed / done * self.L
        return {"value": round(1.0 / per_token_s, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"1 token through {done} of {self.L} layers (numpy fp32 dequant-then-matmul oracle, "
                          f"{threads} threads over experts), scaled to the 48-layer stack"}


class LayerCalls(DecodeStack):
    """The C2 stack driven one layer call at a time (wm_moe_layer_decode, whallm_amd.ops.DecodeLayer):
    each layer's call takes the residual and that layer's router weights (bf16 [512, 2048]) and
    runs the pre-norm, the router GEMV and top-k, the 10 routed + 1 shared experts and the
    residual add in one launch, as a runtime calls the MoE between attention blocks
    (qwen4_exp.py:1146). A step = one token through the 48 layers = 48 calls, replayed from one
    graph; the line reports the time per layer call."""
    name = "layer-c2"
    data = "synthetic (random-init MXFP4 weights, bf16 N(0, 0.05) router rows, N(0,1) residual inputs)"

    def __init__(self, device, layers=48, hidden=2048, experts=512, inter=512, k=10, seed=0):
        from whallm_amd.ops import DecodeLayer
        super().__init__(device, layers, hidden, experts, inter, k, 1, seed, impl="layers")
        g = self.gen
        self.routers = [(torch.randn(experts, hidden, device=device, generator=g) * 0.05).to(torch.bfloat16)
                        for _ in range(layers)]
        self.calls = [DecodeLayer(self.layers[l], self.routers[l], self.shared[l], self.gates[l], k=k)
                      for l in range(layers)]

    def algorithmic_bytes(self):
        # per layer: the router rows, 11 expert blobs, r in and out (fp32) and y (bf16)
        per_layer = self.E * self.H * 2 + (self.K + 1) * self.expert_bytes() + 2 * self.H * 4 + self.H * 2
        return per_layer * self.L

    def prepare_inputs(self, steps):
        self.step_embed = torch.randn(steps, self.H, device=self.device, generator=self.gen)

    def _body_at(self, j):
        r = self.step_embed[j]
        for call in self.calls:
            call(r)

    def capture(self):
        self.graphs = capture_steps(self.device, self._body_at, len(self.step_embed))

    def cpu_baseline(self, budget_s: float):
        """The numpy oracle on a bounded sample: one token through as many of the layers as the
        budget allows (pre-norm, router GEMV, top-k, 11 expert FFNs, combine, residual add)."""
        from oracle import moe as M
        from oracle import formats as F
        from whallm_amd import synthetic as S
        threads = len(os.sched_getaffinity(0))
        r = self.step_embed[0].cpu().numpy().astype(np.float64)

        def fetch(t: torch.Tensor, e):
            a = t[e].cpu().numpy()
            return a.view(np.uint32) if a.dtype == np.int32 else a

        done, elapsed = 0, 0.0
        with ThreadPoolExecutor(threads) as pool:
            for l in range(self.L):
                router = self.routers[l].float().cpu().numpy()
                g = S.bf16_bits_to_f32(self.gates[l].view(torch.int16).cpu().numpy().view(np.uint16))
                sh = M.MXFP4Expert(fetch(self.shared[l].gate_up, 0), fetch(self.shared[l].gate_up_scales, 0),
                                   fetch(self.shared[l].down, 0), fetch(self.shared[l].down_scales, 0))
                t0 = time.perf_counter()
                x = F.bf16_round_f32(M.rms_norm(r[None]).astype(np.float32))
                logits = (router @ x[0])[None].astype(np.float32)
                idx, w = M.route_softmax_topk(logits, self.K)
                elapsed += time.perf_counter() - t0
                ex = {int(e): M.MXFP4Expert(fetch(self.layers[l].gate_up, e), fetch(self.layers[l].gate_up_scales, e),
                                            fetch(self.layers[l].down, e), fetch(self.layers[l].down_scales, e))
                      for e in idx[0]}
                t0 = time.perf_counter()   # compute only: the experts' bytes were fetched above
                outs = list(pool.map(lambda e: M.expert_ffn(x, ex[e]), [int(e) for e in idx[0]]))
                shared_out = M.expert_ffn(x, sh)
                gate = x.astype(np.float64) @ g.astype(np.float64)
                y = M.combine(np.stack(outs, axis=1), w, shared_out, gate)
                r = r + F.bf16_round_f32(y[0])
                elapsed += time.perf_counter() - t0
                done += 1
                if elapsed > budget_s:
                    break
        per_call_s = elapsed / done
        return {"value": round(1.0 / (per_call_s * self.L), 4), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"1 token through {done} of {self.L} layer calls (numpy oracle: norm, router GEMV, top-k, "
                          f"fp32 dequant-then-matmul experts, {threads} threads over experts), "
                          f"{per_call_s * 1e3:.2f} ms per layer call, scaled to the 48-layer stack"}

    def check(self):
        for call in self.calls:
            call.raise_for_status()

    def config(self):
        c = super().config()
        c.update(workload="layer-c2: the C2 stack as 48 one-launch layer calls (pre-norm, router GEMV, top-k, "
                          "experts, residual add), 1 token/step", router="bf16 [512, 2048] per layer")
        return c


class Prefill:
    """C3: one MXFP4 MoE layer at a 16,384-token prefill, Zipf(1.1)-skewed routing.

    act_terms "e4m3": the activations enter the scaled MFMAs as two E4M3 terms per 32 values
    (bf16-exact above 2^-13 of each block's maximum, the reference's activation precision;
    fp4 x fp8 at the FP8 rate); "e2m3": two E2M3 terms (~7 significant bits of the block
    maximum; fp4 x fp6 at the FP4 rate)."""
    name = "c3-prefill"
    # MXFP4 weights (E2M1 + E8M0 per 32) straight into scaled MFMAs against two terms (hi, lo)
    # of the bf16 activations, fp32 accumulation
    dtype = "mxfp4"
    data = "synthetic (random-init MXFP4 weights, N(0,1) bf16 tokens, N(0,1) + Zipf(1.1) bias router logits)"

    def __init__(self, device, hidden=2048, experts=512, inter=512, k=10, tokens=16384, seed=0, act_terms="e4m3"):
        from whallm_amd import synthetic as S
        self.H, self.E, self.I, self.K, self.T = hidden, experts, inter, k, tokens
        self.act_terms = act_terms
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.experts = S.mxfp4_experts_device(experts, hidden, inter, device, g)
        self.shared = S.mxfp4_experts_device(1, hidden, inter, device, g)
        # the layer's weights are repacked once into the prefill tile layout (set-up, untimed);
        # the row-layout copies stay for the CPU baseline
        import dataclasses
        import whallm_amd as wa
        self.tiled = dataclasses.replace(wa.prefill_layout(self.experts), act_terms=act_terms)
        self.tiled_shared = dataclasses.replace(wa.prefill_layout(self.shared), act_terms=act_terms)
        self.gate = (torch.randn(hidden, device=device, generator=g) * 0.02).to(torch.bfloat16)
        rng = np.random.default_rng(seed)
        bias = torch.from_numpy(S.zipf_bias(experts, 1.1, rng)).to(device)
        self.logits = torch.randn(tokens, experts, device=device, generator=g) + bias
        self.x = torch.randn(tokens, hidden, device=device, generator=g).to(torch.bfloat16)
        self.graph = None

    def flops(self):
        return 2 * 3 * self.H * self.I * (self.K + 1) * self.T

    def algorithmic_bytes(self):
        blob = 3 * self.H * self.I // 2 + 3 * self.H * self.I // 32
        return (self.E + 1) * blob + self.T * self.H * 2 * 2 + self.T * self.E * 4

    def tokens_per_step(self):
        return self.T

    def gate_up_flops(self):
        """Algorithmic FLOPs of one gate_up launch: every routed pair and shared row times 2I x H."""
        return 2 * (self.K + 1) * self.T * self.H * 2 * self.I

    def prepare_inputs(self, steps):
        pass

    def _body(self):
        import whallm_amd as wa
        idx, w = wa.route_softmax_topk(self.logits, self.K)
        self.y = wa.moe_mxfp4(self.x, idx, w, self.tiled, self.tiled_shared, self.gate)

    def kernel_ms(self, launches: int):
        """Average (gate_up, down) duration over `launches` layer calls, from the library's
        HIP events recorded on the call's stream around each grouped GEMM."""
        import ctypes
        from whallm_amd import _lib
        lib = _lib.load()
        lib.wm_set_kernel_timing(1)
        out = (ctypes.c_float * 2)()
        sums = [0.0, 0.0]
        try:
            for _ in range(launches):
                self._body()
                _lib.call("wm_kernel_timing_ms", out)
                sums[0] += out[0]
                sums[1] += out[1]
        finally:
            lib.wm_set_kernel_timing(0)
        return sums[0] / launches, sums[1] / launches

    def capture(self):
        side = torch.cuda.Stream(self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):
            self._body()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._body()
        torch.cuda.synchronize(self.device)

    def step(self, i):
        self.graph.replay()

    def config(self):
        terms = ("two E4M3 terms per 32 values (bf16-exact above 2^-13 of the block maximum), fp4 x fp8"
                 if self.act_terms == "e4m3" else
                 "two E2M3 terms per 32 values (~7 significant bits of the block maximum), fp4 x fp6")
        return {"workload": "c3-prefill: Qwen3-Next-style MXFP4 MoE layer, 16384-token prefill, Zipf(1.1) routing",
                "hidden": self.H, "experts": self.E, "moe_intermediate": self.I, "top_k": self.K,
                "shared_experts": 1, "tokens": self.T, "activations": "bf16", "activation_terms": terms,
                "compute": "v_mfma_scale_f32_32x32x64_f8f6f4: MXFP4 weights (prefill tile layout) x the "
                           "activation terms"}

    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        from whallm_amd import synthetic as S
        threads = len(os.sched_getaffinity(0))
        # Sample: the first tokens of the prompt, one expert group at a time, within the budget.
        sample = 64
        logits = self.logits[:sample].cpu().numpy()
        x = self.x[:sample].float().cpu().numpy()
        idx, w = M.route_softmax_topk(logits, self.K)

        def fetch(t, e):
            a = t[e].cpu().numpy()
            return a.view(np.uint32) if a.dtype == np.int32 else a

        experts = {int(e): M.MXFP4Expert(fetch(self.experts.gate_up, e), fetch(self.experts.gate_up_scales, e),
                                         fetch(self.experts.down, e), fetch(self.experts.down_scales, e))
                   for e in np.unique(idx)}
        started = time.perf_counter()
        with ThreadPoolExecutor(threads) as pool:
            flat = idx.reshape(-1)
            groups = [(e, np.flatnonzero(flat == e)) for e in np.unique(flat)]
            list(pool.map(lambda g: M.expert_ffn(x[g[1] // self.K], experts[int(g[0])]), groups))
        elapsed = time.perf_counter() - started
        return {"value": round(sample / elapsed, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"{sample} prompt tokens x top-{self.K} routed experts (numpy fp32 dequant-then-matmul "
                          f"oracle, {threads} threads), shared expert excluded"}


class FP8Layer:
    """C4: one DeepSeek-V3-style FP8 MoE layer (H 7168, 256 routed + 1 shared expert, I 2048,
    top-8 sigmoid routing with group-limited selection: 8 groups, top 4), at 1 decode
    token or a 4096-token prefill."""
    dtype = "fp8-e4m3"
    data = "synthetic (random-init FP8 weights + fp32 block scales, N(0,1) bf16 tokens and router logits)"

    def __init__(self, device, tokens=1, hidden=7168, experts=256, inter=2048, k=8, seed=0):
        from whallm_amd import synthetic as S
        self.H, self.E, self.I, self.K, self.T = hidden, experts, inter, k, tokens
        self.name = "c4-decode" if tokens == 1 else "c4-prefill"
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        log(f"[bench] generating {experts} + 1 FP8 experts (H {hidden}, I {inter}) on device")
        self.experts = S.fp8_experts_device(experts, hidden, inter, device, g)
        self.shared = S.fp8_experts_device(1, hidden, inter, device, g)
        # prefill runs on the weights repacked once into the prefill tile layout (the grouped
        # GEMM's loads); decode reads the row layout (the fused GEMV's)
        if tokens > 1:
            import whallm_amd as wa
            self.run_experts, self.run_shared = wa.prefill_layout(self.experts), wa.prefill_layout(self.shared)
        else:
            self.run_experts, self.run_shared = self.experts, self.shared
        self.bias = torch.randn(experts, device=device, generator=g) * 0.1
        self.gen = g
        self.graphs = None

    def expert_bytes(self):
        return 3 * self.H * self.I + 4 * (2 * self.I // 128) * (self.H // 128) + 4 * (self.H // 128) * (self.I // 128)

    def algorithmic_bytes(self):
        if self.T == 1:   # the routed experts and the shared one, plus logits, x and y
            return (self.K + 1) * self.expert_bytes() + self.E * 4 + 2 * self.H * 2
        return (self.E + 1) * self.expert_bytes() + self.T * self.H * 2 * 2 + self.T * self.E * 4

    def flops(self):
        return 2 * 3 * self.H * self.I * (self.K + 1) * self.T

    def tokens_per_step(self):
        return self.T

    def prepare_inputs(self, steps):
        n = min(steps, 4) if self.T > 1 else steps
        self.step_logits = torch.randn(n, self.T, self.E, device=self.device, generator=self.gen)
        self.step_x = torch.randn(n, self.T, self.H, device=self.device, generator=self.gen).to(torch.bfloat16)

    def _body_at(self, j):
        import whallm_amd as wa
        idx, w = wa.route_scored(self.step_logits[j], self.bias, self.K, func="sigmoid", route_scale=2.5,
                                 n_groups=8, topk_groups=4)
        self.y = wa.moe_fp8(self.step_x[j], idx, w, self.run_experts, self.run_shared, None)

    def capture(self):
        self.graphs = capture_steps(self.device, self._body_at, len(self.step_logits))

    def step(self, i):
        self.graphs[i % len(self.graphs)].replay()

    def config(self):
        return {"workload": f"{self.name}: DeepSeek-V3-style FP8 MoE layer, {self.T} token(s)/step",
                "hidden": self.H, "experts": self.E, "moe_intermediate": self.I, "top_k": self.K,
                "shared_experts": 1, "routing": "sigmoid + bias select, 8 groups / top-4 groups, route_scale 2.5",
                "weights": "FP8-E4M3 of N(0,1) clipped to +-448, fp32 128x128 block scales",
                "tokens": self.T, "activations": "bf16",
                "hbm_resident_weight_gb": round((self.E + 1) * self.expert_bytes() / 1e9, 2)}

    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        from whallm_amd import synthetic as S
        threads = len(os.sched_getaffinity(0))
        logits = self.step_logits[0][:1].cpu().numpy()
        x = self.step_x[0][:1].float().cpu().numpy()
        idx, w = M.route_scored(logits, self.bias.cpu().numpy(), self.K, func="sigmoid", route_scale=2.5,
                                n_groups=8, topk_groups=4)
        I = self.I

        def expert(tab, e):
            w13, s13 = tab.w13[e].cpu().numpy(), tab.w13_scales[e].cpu().numpy()
            return M.FP8Expert(w13[:I], s13[:I // 128], w13[I:], s13[I // 128:], tab.w2[e].cpu().numpy(),
                               tab.w2_scales[e].cpu().numpy())

        ids = [int(e) for e in idx[0]]
        ex = {e: expert(self.experts, e) for e in ids}
        sh = expert(self.shared, 0)
        started = time.perf_counter()
        with ThreadPoolExecutor(threads) as pool:
            outs = list(pool.map(lambda e: M.fp8_expert_ffn(x, ex[e]), ids))
        s_out = M.fp8_expert_ffn(x, sh)
        M.combine(np.stack(outs, axis=1), w, s_out, None)
        elapsed = time.perf_counter() - started
        return {"value": round(1.0 / elapsed, 4), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"1 token through the layer ({self.K} routed + shared FP8 experts; numpy fp32 "
                          f"dequant-then-matmul oracle, {threads} threads over experts)"}


class MtpVerify:
    """C5: MTP verify step: 1 accepted + 3 draft tokens (M 4) through a 4-layer FP8 MoE stack
    (C4 layers with the rmsnorm residual glue), a random bf16 LM head to fp32 logits over a
    129,280-token vocabulary, then greedy acceptance on the device."""
    name = "c5-verify"
    dtype = "fp8-e4m3"
    data = "synthetic (random-init FP8 experts and bf16 LM head, N(0,1) residual inputs and router logits)"

    def __init__(self, device, layers=4, hidden=7168, experts=256, inter=2048, k=8, tokens=4, vocab=129280, seed=0):
        from whallm_amd import synthetic as S
        self.L, self.H, self.E, self.I, self.K, self.T, self.V = layers, hidden, experts, inter, k, tokens, vocab
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        log(f"[bench] generating {layers} x ({experts} + 1) FP8 experts and a {vocab} x {hidden} LM head")
        self.layers = [S.fp8_experts_device(experts, hidden, inter, device, g) for _ in range(layers)]
        self.shared = [S.fp8_experts_device(1, hidden, inter, device, g) for _ in range(layers)]
        self.bias = [torch.randn(experts, device=device, generator=g) * 0.1 for _ in range(layers)]
        self.head = (torch.randn(vocab, hidden, device=device, generator=g) * hidden ** -0.5).to(torch.bfloat16)
        from whallm_amd.verify import VerifyStep
        self.verify = VerifyStep(self.layers, self.shared, self.bias, self.head, k=k)
        self.gen = g
        self.graphs = None

    def expert_bytes(self):
        return 3 * self.H * self.I + 4 * (2 * self.I // 128) * (self.H // 128) + 4 * (self.H // 128) * (self.I // 128)

    def algorithmic_bytes(self):
        # distinct experts a 4-token step can touch: at most T*K routed + 1 shared per layer
        return self.L * (min(self.E, self.T * self.K) + 1) * self.expert_bytes() + self.V * self.H * 2 \
            + self.T * self.V * 4

    def tokens_per_step(self):
        return self.T

    def prepare_inputs(self, steps):
        self.step_logits = torch.randn(steps, self.L, self.T, self.E, device=self.device, generator=self.gen)
        self.step_r = torch.randn(steps, self.T, self.H, device=self.device, generator=self.gen)
        self.drafts = torch.zeros(self.T - 1, dtype=torch.int32, device=self.device)

    def _body_at(self, j):
        # the package's verify step: MoE layers, the LM head in fp32 (wm_linear_bf16), acceptance
        self.accept, self.vocab_logits = self.verify(self.step_logits[j], self.step_r[j], self.drafts)

    def capture(self):
        self.graphs = capture_steps(self.device, self._body_at, len(self.step_logits))

    def step(self, i):
        self.graphs[i].replay()

    def accept_ms(self, launches: int) -> float:
        """Device time of the acceptance kernels alone (HIP events around direct launches)."""
        import whallm_amd as wa
        stream = torch.cuda.current_stream(self.device)
        total = 0.0
        for _ in range(launches):
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record(stream)
            wa.mtp_verify_greedy(self.vocab_logits, self.drafts)
            b.record(stream)
            b.synchronize()
            total += a.elapsed_time(b)
        return total / launches

    def config(self):
        return {"workload": "c5-verify: MTP verify (whallm_amd.verify.VerifyStep), 4 tokens (1 accepted + 3 drafts) "
                            "through a 4-layer FP8 MoE stack, bf16 LM head to 129280 fp32 logits, greedy acceptance "
                            "on the device",
                "hidden": self.H, "experts": self.E, "moe_intermediate": self.I, "top_k": self.K, "layers": self.L,
                "tokens": self.T, "vocab": self.V}

    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        threads = len(os.sched_getaffinity(0))
        logits = self.vocab_logits.cpu().numpy()
        drafts = self.drafts.cpu().numpy()
        started = time.perf_counter()
        reps = 0
        while time.perf_counter() - started < min(budget_s, 5.0):
            M.verify_greedy(drafts, logits)
            reps += 1
        elapsed = (time.perf_counter() - started) / reps
        return {"value": round(1.0 / elapsed, 3), "unit": "verifications/s", "cores": 1, "kind": "port",
                "sample": f"greedy acceptance of {self.T - 1} drafts over [{self.T}, {self.V}] fp32 logits "
                          f"(numpy oracle, {reps} repeats); the MoE layers are not part of this sample"}


class NormRouter:
    """The fused pre-MoE step (wm_norm_router): residual add, RMSNorm, router GEMV and shared
    gate in one launch, at the C2 decode (1 token), C3 prefill (16,384 tokens, H 2048,
    512 experts + shared gate) and C4 prefill (4,096 tokens, H 7168, 256 experts) shapes."""
    dtype = "bf16"
    data = "synthetic (N(0,1) fp32 residual, bf16 N(0,1) layer output, bf16 N(0,0.05) router and gate)"
    SHAPES = {"router-c2": (1, 2048, 512, True), "router-c3": (16384, 2048, 512, True),
              "router-c4": (4096, 7168, 256, False)}

    def __init__(self, device, name, seed=0):
        self.name = name
        self.T, self.H, self.E, gate = self.SHAPES[name]
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.r = torch.randn(self.T, self.H, device=device, generator=g)
        self.y = torch.randn(self.T, self.H, device=device, generator=g).to(torch.bfloat16)
        self.router = (torch.randn(self.E, self.H, device=device, generator=g) * 0.05).to(torch.bfloat16)
        self.gate = (torch.randn(self.H, device=device, generator=g) * 0.05).to(torch.bfloat16) if gate else None
        self.r_out = torch.empty_like(self.r)
        import whallm_amd as wa
        self.packed = wa.repack_router(self.router, self.gate)   # one-time, outside the timed step
        self.graph = None

    def algorithmic_bytes(self):
        rows = self.E + (self.gate is not None)
        return rows * self.H * 2 + self.T * self.H * (4 + 2 + 2 + 4) + self.T * rows * 4

    def flops(self):
        return 2 * self.T * self.H * (self.E + (self.gate is not None))

    def tokens_per_step(self):
        return self.T

    def prepare_inputs(self, steps):
        pass

    def _body(self):
        import whallm_amd as wa
        self.out = wa.norm_router(self.r, self.y, self.router, self.gate, residual_out=self.r_out,
                                  router_packed=self.packed)

    def capture(self):
        self._body()
        torch.cuda.synchronize(self.device)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._body()
        torch.cuda.synchronize(self.device)

    def step(self, i):
        self.graph.replay()

    def config(self):
        return {"workload": f"{self.name}: fused residual add + RMSNorm + router GEMV (+ shared gate) before the MoE",
                "hidden": self.H, "experts": self.E, "tokens": self.T, "shared_gate": self.gate is not None}

    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        f = lambda t: None if t is None else t.float().cpu().numpy()
        n = min(self.T, 256)
        r, y, w, g = f(self.r[:n]), f(self.y[:n]), f(self.router), f(self.gate)
        started = time.perf_counter()
        reps = 0
        while time.perf_counter() - started < min(budget_s, 10.0):
            M.norm_router(r, y, w, g)
            reps += 1
        elapsed = (time.perf_counter() - started) / reps
        return {"value": round(n / elapsed, 3), "unit": "tokens/s", "cores": len(os.sched_getaffinity(0)),
                "kind": "port", "sample": f"oracle.norm_router (numpy, float64 matmul) on {n} tokens, {reps} repeats"}


class ResidentSingleton:
    """BASELINE.md's one published workload, the reference's resident-expert-singleton
    microbenchmark (Scripts/benchmark_qwen_speed.py:198-211, docs/qwen-speed-optimization.md:
    102-126): StreamingExperts over 10 resident MXFP4 experts at the Qwen model's hidden 2560 /
    intermediate 640, one token, indices [[[8, 3, 5, 9, 0, 6, 1, 7, 4, 2]]], router-order
    output [1, 1, 10, 2560], the experts handed out by get_many as views of one batched
    tensor, no expert I/O.

    Timed the reference's way: three warm-up calls, then 15 samples of three synchronised
    operator calls each (host work included: the operator's id read, table build and
    launches); ms_per_step is the p50 sample. The device time of the two expert kernels alone
    (graph replays of the resolved call, HIP events) gives the roofline."""
    name = "qwen-resident"
    dtype = "mxfp4"
    data = "synthetic (random-init MXFP4 experts, bf16 N(0,1) token)"
    PUBLISHED_P50_MS = 1.63458   # Apple M1 (Virtual), MLX 0.32.2
    IDS = [8, 3, 5, 9, 0, 6, 1, 7, 4, 2]

    def __init__(self, device, hidden=2560, inter=640, seed=0):
        from types import SimpleNamespace
        from whallm_amd import operators as O
        from whallm_amd import synthetic as S
        self.H, self.I, self.E, self.K, self.T = hidden, inter, 10, 10, 1
        self.device = device
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        self.experts = S.mxfp4_experts_device(self.E, hidden, inter, device, g)
        payloads = tuple(O.QwenExpertWeights(self.experts.gate_up[i], self.experts.gate_up_scales[i],
                                             self.experts.down[i], self.experts.down_scales[i])
                         for i in range(self.E))
        cache = SimpleNamespace(slots=self.E, current_batched=lambda _l: None,
                                get_many=lambda _l, ids: O.ResidentExperts(payloads, {i: i for i in ids}))
        self.op = O.StreamingExperts(0, cache)
        self.hidden = torch.randn(1, 1, hidden, device=device, generator=g).to(torch.bfloat16)
        self.indices = torch.tensor([[self.IDS]], dtype=torch.int32, device=device)

    def blob_bytes(self):
        return 2 * self.I * self.H // 2 + 2 * self.I * self.H // 32 + self.H * self.I // 2 + self.H * self.I // 32

    def algorithmic_bytes(self):
        # the 10 expert blobs, the token's input row and the 10 output rows (bf16)
        return self.E * self.blob_bytes() + self.H * 2 + self.K * self.H * 2

    def measure(self, steps: int, warmup: int):
        import whallm_amd as wa
        dev = self.device
        for _ in range(3):
            self.op(self.hidden, self.indices)
        torch.cuda.synchronize(dev)
        samples = []
        t_all = time.perf_counter()
        for _ in range(15):
            t0 = time.perf_counter()
            for _ in range(3):
                self.out = self.op(self.hidden, self.indices)
            torch.cuda.synchronize(dev)
            samples.append((time.perf_counter() - t0) / 3 * 1e3)
        wall = time.perf_counter() - t_all
        p50, p95 = float(np.percentile(samples, 50)), float(np.percentile(samples, 95))
        # device time of the resolved call's two expert kernels: graph replays
        table, idx = self.op.table(self.indices)
        out = torch.empty(1, 1, self.K, self.H, dtype=torch.bfloat16, device=dev)
        graphs = capture_steps(dev, lambda j: wa.experts_mxfp4(self.hidden, idx, table, out=out), 1)
        for _ in range(warmup):
            graphs[0].replay()
        stream = torch.cuda.current_stream(dev)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(steps):
            graphs[0].replay()
        b.record(stream)
        torch.cuda.synchronize(dev)
        k_ms = a.elapsed_time(b) / steps
        assert torch.equal(out, self.out), "graph replay differs from the operator call"
        achieved = self.algorithmic_bytes() / (k_ms / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": "gate_up_act_kernel + down_kernel (per-pair), graph-replayed",
                    "kernel_ms": round(k_ms, 5), "algorithmic_bytes_per_launch": self.algorithmic_bytes()}
        self.p50, self.p95, self.samples = p50, p95, samples
        return p50, 1e3 / p50, roofline, wall

    def config(self):
        return {"workload": "qwen-resident: BASELINE.md's resident-expert-singleton case, StreamingExperts over 10 "
                            "resident MXFP4 experts, 1 token, router-order output",
                "hidden": self.H, "moe_intermediate": self.I, "experts": self.E, "top_k": self.K,
                "indices": self.IDS, "timing": "3 warm-up calls, 15 samples x 3 synchronised calls, p50",
                "p50_ms": round(self.p50, 5), "p95_ms": round(self.p95, 5),
                "published_p50_ms": self.PUBLISHED_P50_MS,
                "published_hardware": "Apple M1 (Virtual), Apple Paravirtual GPU, MLX 0.32.2"}

    def cpu_baseline(self, budget_s: float):
        from oracle import moe as M
        threads = len(os.sched_getaffinity(0))
        x = self.hidden.float().cpu().numpy().reshape(1, self.H)

        def fetch(t, e):
            a = t[e].cpu().numpy()
            return a.view(np.uint32) if a.dtype == np.int32 else a

        ex = [M.MXFP4Expert(fetch(self.experts.gate_up, e), fetch(self.experts.gate_up_scales, e),
                            fetch(self.experts.down, e), fetch(self.experts.down_scales, e)) for e in self.IDS]
        with ThreadPoolExecutor(threads) as pool:
            def call():
                return np.stack(list(pool.map(lambda e: M.expert_ffn(x, e)[0], ex)))
            for _ in range(3):
                call()
            samples = []
            for _ in range(15):
                t0 = time.perf_counter()
                for _ in range(3):
                    call()
                samples.append((time.perf_counter() - t0) / 3)
        p50 = float(np.percentile(samples, 50))
        return {"value": round(1.0 / p50, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
                "sample": f"the same call on the numpy oracle (fp32 dequant-then-matmul, {threads} threads over the "
                          f"10 experts), 15 samples x 3 calls, p50 {p50 * 1e3:.2f} ms"}


WORKLOADS = {"c2-decode": DecodeStack, "layer-c2": LayerCalls, "c3-prefill": Prefill, "c4-decode": FP8Layer, "c4-prefill": FP8Layer,
             "c5-verify": MtpVerify, "router-c2": NormRouter, "router-c3": NormRouter, "router-c4": NormRouter,
             "qwen-resident": ResidentSingleton}


# ----------------------------------------------------------------------------- main

def profiled_traffic(name: str):
    """HBM bytes per launch of the dominant kernel from the committed rocprofv3 counter
    summary profiles/<name>_traffic.txt (FETCH_SIZE + WRITE_SIZE, each scaled by the
    factor a copy kernel of known size gives), or None when it has not been profiled."""
    path = os.path.join(HERE, "profiles", f"{name}_traffic.txt")
    try:
        with open(path) as f:
            for line in f:
                if line.startswith("hbm_bytes_per_launch:"):
                    return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def measure(wl, steps: int, warmup: int):
    """Times `steps` graph replays of the workload after `warmup` untimed ones (HIP events
    on the replay stream, synchronised on both sides); returns (ms per step, tokens/s,
    roofline object, wall seconds of the timed region)."""
    device = wl.device
    if hasattr(wl, "measure"):
        return wl.measure(steps, warmup)
    total = warmup + steps
    wl.prepare_inputs(total)
    wl.capture()
    for i in range(warmup):
        wl.step(i)
    torch.cuda.synchronize(device)

    stream = torch.cuda.current_stream(device)
    start_ev = torch.cuda.Event(enable_timing=True)
    end_ev = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start_ev.record(stream)
    for i in range(warmup, total):
        wl.step(i)
    end_ev.record(stream)
    torch.cuda.synchronize(device)
    wall = time.perf_counter() - t0
    gpu_ms = start_ev.elapsed_time(end_ev)
    if hasattr(wl, "check"):
        wl.check()
    ms_per_step = gpu_ms / steps
    value = wl.tokens_per_step() / (ms_per_step / 1e3)
    if isinstance(wl, LayerCalls):
        per_layer_ms = ms_per_step / wl.L
        achieved = wl.algorithmic_bytes() / (ms_per_step / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": "moe_layer_kernel<2048, 512> (one launch per layer call), 48 calls per step",
                    "layer_call_us": round(per_layer_ms * 1e3, 3),
                    "algorithmic_bytes_per_launch": wl.algorithmic_bytes() // wl.L}
    elif isinstance(wl, DecodeStack):
        # the HIP events over the timed region (graphs replayed back to back on this stream):
        # for the persistent kernel, one launch a step, its duration plus the gap to the next
        k_ms = ms_per_step
        if wl.impl == "persistent":
            kernel = "decode_persistent_kernel (one launch = one token through 48 layers)"
        else:
            kernel = "decode step: 48 x (route, gate_up_act, down_combine, residual_rmsnorm)"
        achieved = wl.algorithmic_bytes() / (k_ms / 1e3) / 1e9
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": profiled_traffic("decode_persistent_c2"),
                    "kernel": kernel, "kernel_ms": round(k_ms, 5),
                    "algorithmic_bytes_per_launch": wl.algorithmic_bytes()}
    elif isinstance(wl, FP8Layer):
        achieved = wl.algorithmic_bytes() / (ms_per_step / 1e3) / 1e9
        tflops = wl.flops() / (ms_per_step / 1e3) / 1e12
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "tflops": round(tflops, 2), "frac_of_fp8_peak": round(tflops / FP8_PEAK_TFLOPS, 4),
                    "kernel": "FP8 MoE layer step (route_scored, FP8 expert kernels, combine) from one graph",
                    "algorithmic_bytes_per_launch": wl.algorithmic_bytes()}
    elif isinstance(wl, NormRouter):
        achieved = wl.algorithmic_bytes() / (ms_per_step / 1e3) / 1e9
        tflops = wl.flops() / (ms_per_step / 1e3) / 1e12
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "tflops": round(tflops, 2),
                    "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
                    "kernel": "norm_router (one launch per step, graph replay)",
                    "algorithmic_bytes_per_launch": wl.algorithmic_bytes()}
    elif isinstance(wl, MtpVerify):
        achieved = wl.algorithmic_bytes() / (ms_per_step / 1e3) / 1e9
        a_ms = wl.accept_ms(20)
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                    "kernel": "verify step: 4 FP8 MoE layers + LM head + greedy acceptance, one graph",
                    "verify_latency_ms": round(ms_per_step, 4), "acceptance_kernel_ms": round(a_ms, 5),
                    "algorithmic_bytes_per_launch": wl.algorithmic_bytes()}
    else:
        # dominant kernel: the grouped gate_up GEMM, timed with the library's HIP events
        gu_ms, dn_ms = wl.kernel_ms(steps)
        achieved = wl.gate_up_flops() / (gu_ms / 1e3) / 1e12
        layer_tflops = wl.flops() / (ms_per_step / 1e3) / 1e12
        # fp4 x fp6 operands run the 32x32x64 f8f6f4 MFMA at the FP4/FP6 rate, fp4 x fp8 at the
        # FP8 rate; the two activation terms make every product two MFMA products, so useful
        # FLOPs top out at half the instruction's rate (mfma_instruction_frac counts the
        # instructions against that rate)
        rate = FP4_PEAK_TFLOPS if getattr(wl, "act_terms", "e2m3") == "e2m3" else FP8_PEAK_TFLOPS
        traffic = profiled_traffic("prefill_c3_gate_up" + ("" if wl.act_terms == "e4m3" else "_e2m3"))
        roofline = {"bound": "mfma", "achieved": round(achieved, 1), "peak": FP4_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / FP4_PEAK_TFLOPS, 4), "traffic": traffic,
                    "mfma_instruction_frac": round(2 * achieved / rate, 4),
                    "mfma_instruction_rate_tflops": rate,
                    "frac_of_fp8_peak": round(achieved / FP8_PEAK_TFLOPS, 4),
                    "kernel": "gate_up_mx_kernel<Mx4> (grouped gate/up GEMM + SwiGLU, one launch per layer)",
                    "kernel_ms": round(gu_ms, 5), "down_kernel_ms": round(dn_ms, 5),
                    "algorithmic_flops_per_launch": wl.gate_up_flops(),
                    "layer_tflops": round(layer_tflops, 1)}

    return ms_per_step, value, roofline, wall


def prefill_e2m3(pf, args):
    """The same C3 layer on the faster E2M3 activation terms (the bench's other prefill path),
    timed the same way, as a secondary record beside the bf16-exact default."""
    import dataclasses
    pf2 = Prefill.__new__(Prefill)
    pf2.__dict__.update(pf.__dict__)
    pf2.act_terms = "e2m3"
    pf2.tiled = dataclasses.replace(pf.tiled, act_terms="e2m3")
    pf2.tiled_shared = dataclasses.replace(pf.tiled_shared, act_terms="e2m3")
    pf2.graph = None
    ms, value, roof, _ = measure(pf2, min(args.steps, 20), args.warmup)
    return {"value": round(value, 1), "unit": "tokens/s", "ms_per_step": round(ms, 5), "config": pf2.config(),
            "roofline": roof}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    # untimed: the kernels settle over their first ~15 back-to-back launches (clock ramp,
    # cold caches; the per-dispatch durations in profiles/)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2-decode", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--decode-impl", default="persistent", choices=["persistent", "layers"],
                    help="c2-decode: one persistent kernel per token, or the per-layer kernel chain")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-prefill", action="store_true",
                    help="c2-decode: leave out the 16K-token prefill half (the C3 layer) of the line")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (each box has one MI355X); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.config == "c2-decode":
        wl = DecodeStack(device, impl=args.decode_impl)
    elif args.config == "c4-prefill":
        wl = FP8Layer(device, tokens=4096)
    elif args.config.startswith("router-"):
        wl = NormRouter(device, args.config)
    else:
        wl = WORKLOADS[args.config](device)
    ms_per_step, value, roofline, wall = measure(wl, args.steps, args.warmup)

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] timing the CPU baseline")
        cpu = wl.cpu_baseline(args.cpu_budget)
        cpu["host"] = cpu_model()

    # The metric has two halves (decode and the 16K-token prefill): the default run times the
    # prefill layer too, after the decode stack's weights are freed, and carries it in the
    # same line; `value` stays the decode half (BASELINE's headline config).
    prefill = None
    if args.config == "c2-decode" and not args.no_prefill:
        dtype, data, config = wl.dtype, wl.data, wl.config()
        del wl
        torch.cuda.empty_cache()
        log("[bench] c3-prefill half")
        pf = Prefill(device)
        # the full warmup: a prefill layer's duration falls over its first ~10 back-to-back runs
        # (the clocks ramp under the sustained load; profiles/prefill_c3_kernel_stats.txt)
        p_ms, p_value, p_roof, p_wall = measure(pf, min(args.steps, 20), args.warmup)
        e2m3 = prefill_e2m3(pf, args)
        p_cpu = None
        if not args.no_cpu_baseline:
            log("[bench] timing the prefill CPU baseline")
            p_cpu = pf.cpu_baseline(args.cpu_budget)
            p_cpu["host"] = cpu_model()
        prefill = {"value": round(p_value, 1), "unit": "tokens/s", "ms_per_step": round(p_ms, 5),
                   "steps": min(args.steps, 20), "warmup": args.warmup, "dtype": pf.dtype, "data": pf.data,
                   "config": pf.config(), "roofline": p_roof, "cpu_baseline": p_cpu,
                   "wall_s_timed_region": round(p_wall, 4), "e2m3": e2m3}
    else:
        dtype, data, config = wl.dtype, wl.data, wl.config()
    if args.config == "c3-prefill":
        config = dict(config, e2m3=prefill_e2m3(wl, args))

    # BASELINE.md publishes one number, for the qwen-resident workload (p50 ms per call)
    published = getattr(WORKLOADS[args.config], "PUBLISHED_P50_MS", None)
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None if published is None else round(published / ms_per_step, 2), "dtype": dtype, "data": data,
        "config": config, "roofline": roofline, "cpu_baseline": cpu,
        "wall_s_timed_region": round(wall, 4),
    }
    if prefill is not None:
        line["prefill"] = prefill
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
