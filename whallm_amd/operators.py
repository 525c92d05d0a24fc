"""The reference runtime's expert-FFN operators, over the HIP kernels of libwhallm_moe.

Same names, constructor arguments, call signatures, cache protocol and error
behaviour as:

* ``SparseMoE`` / ``StreamingExperts`` / ``MLP`` (runtime/deepseek_v4_ssd/qwen4_exp.py:763-1051),
* ``_StreamingSwitchGLU`` and the DeepSeek gate / shared expert / activation
  (runtime/deepseek_v4_ssd/model.py:318-546, deepseek_v41/moe.py:30-112),
* the weight containers of expert_cache.py:32-75,

with torch device tensors in place of mlx arrays. The cache is duck-typed as in the
reference: ``current_batched(layer)`` (a whole-layer table: no host sync, the fused
kernels index experts on the device), ``get_many(layer, ids)`` / ``iter_ready(layer, ids)``
(individual resident experts: addressed in place when they are views of one pool, as the
reference's slot views are, else gathered into one table), plus the
optional recording hooks. Routed experts, the bf16 shared ``MLP`` (with its sigmoid gate
and the add) and the combines run on the library's kernels. Only an activation other than
(clamped) SwiGLU takes a generic path: library GEMMs (hipBLASLt through torch) over
weights the library dequantizes, one expert at a time with a host loop over the touched
experts; it exists for the reference tests' arbitrary activations and is never on the
SwiGLU hot path.
"""
from __future__ import annotations

import math
import threading
import time
from dataclasses import dataclass, replace

import torch

from .ops import (FP8Experts, MXFP4Experts, combine_pairs, dequant_fp8_blocks, dequant_fp8_e8m0, dequant_mxfp4,
                  experts_fp8,
                  experts_mxfp4, linear_bf16, mlp_bf16, moe_fp8, moe_mxfp4, route_scored, route_softmax_topk)

# Whole-layer prefill groups rows by expert from this many rows (qwen4_exp.py:789).
GROUPED_PREFILL_ROWS = 64
# MTP verification rows handled by the ready path (qwen4_exp.py:787).
READY_VERIFICATION_ROWS = 16


# ----------------------------------------------------------------------------- containers (expert_cache.py:32-75)

@dataclass(frozen=True)
class ExpertWeights:
    """One DeepSeek expert: MXFP4 w1 (gate), w2 (down), w3 (up) regions, optionally the
    fused w13 = [w3; w1] (expert_layout.py:43-51)."""
    w1: torch.Tensor
    w1_scales: torch.Tensor
    w2: torch.Tensor
    w2_scales: torch.Tensor
    w3: torch.Tensor
    w3_scales: torch.Tensor
    w13: torch.Tensor | None = None
    w13_scales: torch.Tensor | None = None


@dataclass(frozen=True)
class BatchedExperts(ExpertWeights):
    """ExpertWeights with a leading expert axis (expert_cache.py:51-59)."""


@dataclass(frozen=True)
class QwenExpertWeights:
    """One Qwen expert blob: gate_up = [gate; up] rows, down (expert_cache.py:62-67)."""
    gate_up: torch.Tensor
    gate_up_scales: torch.Tensor
    down: torch.Tensor
    down_scales: torch.Tensor


@dataclass(frozen=True)
class QwenBatchedExperts(QwenExpertWeights):
    """QwenExpertWeights with a leading expert axis (expert_cache.py:70-75)."""


@dataclass(frozen=True)
class ResidentExperts:
    """Experts made resident for one call; slots maps expert id -> index into
    individual_weights (expert_cache.py:44-47)."""
    individual_weights: tuple
    slots: dict


# ----------------------------------------------------------------------------- activations

class ClampedSwiGLU:
    """activation(up, gate) = silu(min(gate, limit)) * clip(up, -limit, limit); limit 0 is
    plain SwiGLU (deepseek_v41/moe.py:30-43). Fused into the expert kernels."""

    def __init__(self, limit: float = 0.0):
        self.limit = float(limit)

    def __call__(self, up: torch.Tensor, gate: torch.Tensor) -> torch.Tensor:
        up, gate = up.float(), gate.float()
        if self.limit > 0:
            up = up.clamp(-self.limit, self.limit)
            gate = gate.clamp(max=self.limit)
        return torch.nn.functional.silu(gate) * up


class SwiGLU(ClampedSwiGLU):
    """mlx-lm SwitchGLU's default activation: silu(gate) * up."""

    def __init__(self):
        super().__init__(0.0)


def _fused_limit(activation) -> float | None:
    """The swiglu_limit the kernels apply for ``activation``, or None when it is not SwiGLU."""
    if activation is None:
        return 0.0
    if isinstance(activation, ClampedSwiGLU):
        return activation.limit
    return None


# ----------------------------------------------------------------------------- tables

def _as_table(weights, activation_limit: float = 0.0):
    """A batched weight container -> the library's expert table (MXFP4Experts / FP8Experts)."""
    if isinstance(weights, (MXFP4Experts, FP8Experts)):
        return weights
    if isinstance(weights, QwenExpertWeights):   # gate rows first (qwen4_exp.py:816-818)
        return MXFP4Experts(weights.gate_up, weights.gate_up_scales, weights.down, weights.down_scales,
                            swiglu_limit=activation_limit)
    if isinstance(weights, ExpertWeights):       # w13 = [w3 (up); w1 (gate)] (model.py:516-523)
        if weights.w13 is not None and weights.w13_scales is not None:
            w13, w13s = weights.w13, weights.w13_scales
        else:
            axis = weights.w1.dim() - 2
            w13 = torch.cat([weights.w3, weights.w1], dim=axis)
            w13s = torch.cat([weights.w3_scales, weights.w1_scales], dim=axis)
        return MXFP4Experts(w13, w13s, weights.w2, weights.w2_scales, up_first=True,
                            swiglu_limit=activation_limit)
    raise TypeError(f"unsupported expert weights {type(weights).__name__}")


def _stack_tables(tables: list):
    """One table over the experts of ``tables`` (each a single expert, in order)."""
    first = tables[0]
    fields = [torch.stack([t.tensors()[i] for t in tables]) for i in range(4)]
    return type(first)(*fields, up_first=first.up_first, swiglu_limit=first.swiglu_limit)


def _pool_regions(regs: list):
    """For single experts (``regs``: each expert's four region tensors) whose regions are
    views of shared storages at one stride per region (the slot views of a pool, or [i] of
    region-major tensors, which is how the reference's get_many hands out resident experts,
    expert_cache.py:488-497): the four regions as slot-major views over those storages and
    each expert's slot in them, so the library addresses the experts as base + slot * stride
    and nothing is copied. None when the regions lie otherwise."""
    n = len(regs)
    slot_of = None
    fields = []
    for r in range(4):
        t0 = regs[0][r]
        if t0.dim() != 2:
            return None
        shape, stride, dtype = t0.shape, t0.stride(), t0.dtype
        size = t0.element_size()
        storage = t0.untyped_storage()
        base = storage.data_ptr()
        end = base + storage.nbytes()
        offs = []
        for reg in regs:  # one address per view: inside t0's storage means a view of it
            t = reg[r]
            if t.shape != shape or t.stride() != stride or t.dtype != dtype:
                return None
            at = t.data_ptr() - base
            if at < 0 or base + at >= end or at % size:
                return None
            offs.append(at // size)
        lo = min(offs)
        if slot_of is None:       # slot numbers from the first region's offsets
            unit = 0
            for o in offs:
                unit = math.gcd(unit, o - lo)
            unit = unit or t0.numel()
            slot_of = [(o - lo) // unit for o in offs]
            if len(set(slot_of)) != n:
                return None
        top_slot = max(slot_of)
        top = slot_of.index(top_slot)
        step = (offs[top] - lo) // top_slot if top_slot else t0.numel()
        if step < t0.numel():
            return None
        for o, sl in zip(offs, slot_of):
            if o - lo != sl * step:
                return None
        fields.append(t0.as_strided((top_slot + 1, *shape), (step, *stride), lo))
    return fields, slot_of


def _load_host_meta():
    """The compiled form of _pool_regions (csrc/host_meta.cpp, built beside the library by
    whallm_amd.build), or None when it is not built."""
    import importlib.util
    import warnings

    from .build import host_meta_path
    path = host_meta_path()
    if not path.exists():
        return None
    try:
        spec = importlib.util.spec_from_file_location("_host_meta", path)
        module = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(module)
        return module
    except ImportError as exc:
        warnings.warn(f"{path.name} did not load ({exc}); the pool check runs in Python")
        return None


_host_meta = _load_host_meta()


def _pool_fields(regs: list):
    """_pool_regions through the compiled helper when it is built (the same rules; reading
    tensor metadata from Python is most of a resident-expert call's host time)."""
    if _host_meta is not None:
        return _host_meta.pool_regions([t for reg in regs for t in reg], len(regs))
    return _pool_regions(regs)


class _PinnedRing:
    """Small int32 host-to-device copies through pinned memory: each copy is queued on the
    current stream and the host does not wait for it. A ring of slots; a slot is written
    again only after the event recorded behind its last copy has completed. Calls from
    several threads take the ring one at a time."""
    SLOTS, WORDS = 32, 4096

    def __init__(self):
        self.host = torch.empty(self.SLOTS * self.WORDS, dtype=torch.int32, pin_memory=True)
        self.view = self.host.numpy()
        self.events = [None] * self.SLOTS
        self.next = 0
        self.lock = threading.Lock()

    def to_device(self, values: list, device: torch.device) -> torch.Tensor:
        n = len(values)
        if n > self.WORDS:
            return torch.tensor(values, dtype=torch.int32, device=device)
        with self.lock:
            slot = self.next
            self.next = (slot + 1) % self.SLOTS
            if self.events[slot] is not None:
                self.events[slot].synchronize()
            lo = slot * self.WORDS
            self.view[lo:lo + n] = values
            out = torch.empty(n, dtype=torch.int32, device=device)
            out.copy_(self.host[lo:lo + n], non_blocking=True)
            event = torch.cuda.Event()
            event.record(torch.cuda.current_stream(device))
            self.events[slot] = event
        return out


_ring: _PinnedRing | None = None


def _device_i32(values: list, device: torch.device) -> torch.Tensor:
    """int32 [len(values)] on ``device``, copied without a host wait (_PinnedRing)."""
    global _ring
    if device.type != "cuda":  # host tensors (the CPU tests of this module's logic)
        return torch.tensor(values, dtype=torch.int32, device=device)
    if _ring is None:
        _ring = _PinnedRing()
    return _ring.to_device(values, device)


def _resident_table(resident: ResidentExperts, experts: list[int], limit: float, ids: list[int],
                    indices: torch.Tensor):
    """(table, indices into it) for the individual experts of ``experts`` (sorted unique ids)
    and the call's ids (``ids``, host ints in ``indices``' order): the table addresses the
    experts in place when their regions share a pool (_pool_regions), else gathers them by a
    copy. The ids are mapped to table positions on the host (they are there already), and the
    slot map and those positions reach the device in one copy."""
    weights = []
    for e in experts:
        if e not in resident.slots:
            raise ValueError(f"expert {e} is not resident")
        weights.append(resident.individual_weights[resident.slots[e]])
    singles = None
    if all(type(w) is QwenExpertWeights for w in weights):  # the regions as they are (_as_table)
        regs = [(w.gate_up, w.gate_up_scales, w.down, w.down_scales) for w in weights]
        cls, up_first, lim = MXFP4Experts, False, limit
    else:
        singles = [_as_table(w, limit) for w in weights]
        regs = [t.tensors()[:4] for t in singles]
        cls, up_first, lim = type(singles[0]), singles[0].up_first, singles[0].swiglu_limit
    pos = {e: i for i, e in enumerate(experts)}
    compact = [pos[e] for e in ids]
    pool = _pool_fields(regs)
    if pool is None:
        if singles is None:
            singles = [_as_table(w, limit) for w in weights]
        return _stack_tables(singles), _device_i32(compact, indices.device).reshape(indices.shape)
    fields, slot_of = pool
    n = len(slot_of)
    buf = _device_i32(slot_of + compact, fields[0].device)
    return cls(*fields, slots=buf[:n], experts=n, up_first=up_first, swiglu_limit=lim), buf[n:].reshape(indices.shape)


def _host_ids(indices: torch.Tensor, expert_count: int | None) -> list[int]:
    """The call's expert ids as host ints (one device read), checked against the model."""
    ids = indices.reshape(-1).to("cpu").tolist()
    if ids and (min(ids) < 0 or (expert_count is not None and max(ids) >= expert_count)):
        raise ValueError("expert ID is outside the model")
    return ids


def _generic_experts(x: torch.Tensor, indices: torch.Tensor, table, activation) -> torch.Tensor:
    """Per-pair outputs [T, K, H] for an activation the kernels do not fuse: the library
    dequantizes each touched expert, the projections run as library GEMMs (the
    _StreamingSwitchGLU arithmetic of model.py:395-426 with mx.quantized_matmul's
    dequant-then-matmul). It loops over the touched experts on the host (one
    synchronisation for the id list) and is never taken for SwiGLU or the clamped SwiGLU,
    which the expert kernels fuse; it exists for arbitrary activation callables only."""
    T, K = indices.shape
    H, I = table.hidden, table.inter
    flat = indices.reshape(-1).long()
    out = torch.empty(T * K, H, dtype=torch.bfloat16, device=x.device)
    slots = None if table.slots is None else table.slots.to("cpu", torch.int64)
    fp8 = isinstance(table, FP8Experts)
    for e in torch.unique(flat).tolist():
        rows = (flat == e).nonzero().squeeze(1)
        slot = e if slots is None else int(slots[e])
        w13, w13s, w2, w2s = (t[slot] if t.dim() == 3 else t for t in table.tensors()[:4])
        if fp8:
            deq = dequant_fp8_e8m0 if table.scale_format == 1 else dequant_fp8_blocks
            wa, wd, src = deq(w13, w13s), deq(w2, w2s), x[rows // K].float()
        else:
            wa, wd = dequant_mxfp4(w13, w13s, torch.bfloat16), dequant_mxfp4(w2, w2s, torch.bfloat16)
            src = x[rows // K]
        first, second = (src @ wa.T).split(I, dim=-1)
        up, gate = (first, second) if table.up_first else (second, first)
        h = activation(up, gate).to(wd.dtype)
        out[rows] = (h @ wd.T).to(torch.bfloat16)
    return out.view(T, K, H)


def resolve_table(cache, layer: int, indices: torch.Tensor, limit: float = 0.0):
    """(expert table, indices into it) for one call: the whole-layer table when the cache
    has one (no host synchronisation: the kernels map ids to slots on the device), else the
    resident experts from iter_ready (single-token decode with ready_expert_decode) or
    get_many, gathered into one table (qwen4_exp.py:857-944, model.py:325-371). Those two
    cache calls take host id lists, as the reference's do, so that path synchronises once
    to read the ids (timed into record_routing_sync, as expert_cache.py does)."""
    current = getattr(cache, "current_batched", None)
    batched = current(layer) if callable(current) else None
    if batched is not None:
        capture = getattr(cache, "capture_prefill_seed_routes", None)
        if capture is not None:
            capture(layer, indices)
        if getattr(cache, "route_cache_enabled", False):
            cache.observe_batched_routes(layer, indices.to("cpu", torch.int32).numpy())
        record = getattr(cache, "record_gather_qmm", None)
        if callable(record):   # separate w1 / w3 regions cost the reference a third gather_qmm
            record(3 if isinstance(batched, ExpertWeights) and batched.w13 is None else 2)
        return replace(_as_table(batched), swiglu_limit=limit), indices
    started = time.perf_counter()
    model = getattr(cache, "model", None)
    ids = _host_ids(indices, getattr(model, "expert_count", None))
    record_sync = getattr(cache, "record_routing_sync", None)
    if record_sync is not None:
        record_sync(time.perf_counter() - started)
    unique = sorted(set(ids))
    rows = indices.numel() // indices.shape[-1]
    if rows == 1 and getattr(cache, "ready_expert_decode", False) and hasattr(cache, "iter_ready"):
        ready = cache.iter_ready(layer, ids)
        try:
            got = dict(ready)
        finally:
            close = getattr(ready, "close", None)
            if close is not None:
                close()
        resident = ResidentExperts(tuple(got[e] for e in unique), {e: i for i, e in enumerate(unique)})
    else:
        resident = cache.get_many(layer, ids)
    return _resident_table(resident, unique, limit, ids, indices)


# ----------------------------------------------------------------------------- Qwen operators

class Linear:
    """A bias-free bf16 linear (mlx nn.Linear(in, out, bias=False)); weight [out, in]."""

    def __init__(self, inputs: int, outputs: int, device="cuda", weight: torch.Tensor | None = None):
        self.weight = weight if weight is not None else torch.zeros(outputs, inputs, dtype=torch.bfloat16,
                                                                    device=device)

    def __call__(self, value: torch.Tensor) -> torch.Tensor:
        return torch.nn.functional.linear(value, self.weight)


class MLP:
    """The bf16 shared expert: down(silu(gate(x)) * up(x)) (qwen4_exp.py:763-771), on the
    library's fused kernels (wm_mlp_bf16)."""

    def __init__(self, dimensions: int, intermediate: int, device="cuda"):
        self.gate_proj = Linear(dimensions, intermediate, device)
        self.up_proj = Linear(dimensions, intermediate, device)
        self.down_proj = Linear(intermediate, dimensions, device)

    def __call__(self, value: torch.Tensor, gate: torch.Tensor | None = None,
                 add: torch.Tensor | None = None) -> torch.Tensor:
        """down(silu(gate_proj(x)) * up_proj(x)), scaled by sigmoid(x . gate) and added to
        ``add`` when those are given (the shared-expert term of SparseMoE, qwen4_exp.py:1045)."""
        return mlp_bf16(value, self.gate_proj.weight, self.up_proj.weight, self.down_proj.weight, gate, add)


class StreamingExperts:
    """Routed Qwen experts: __call__(value [.., H], indices [.., K]) -> [.., K, H] in router
    order (qwen4_exp.py:796-904).

    The reference's flags are kept. ``grouped_prefill`` / ``sorted_prefill`` / ``wave_slots`` /
    ``ready_verification`` choose how it submits MLX work; here every call is one launch
    sequence whose rows the library groups by expert itself (the decode GEMV for up to
    256 (token, expert) pairs, the grouped GEMM above that), so they change no result.
    """

    def __init__(self, layer: int, cache):
        self.layer = layer
        self.cache = cache
        self.grouped_prefill = False
        self.sorted_prefill = False
        self.ready_verification = False
        self.wave_slots = 0
        self.wave_count = 0
        self.wave_pairs = 0
        self.wave_peak_experts = 0

    @staticmethod
    def _one(value: torch.Tensor, weights) -> torch.Tensor:
        """One expert over rows ``value`` [n, H] (qwen4_exp.py:814-818)."""
        table = _as_table(weights)
        n = value.reshape(-1, value.shape[-1]).shape[0]
        idx = torch.zeros(n, 1, dtype=torch.int32, device=value.device)
        return experts_mxfp4(value.reshape(n, -1), idx, table)[:, 0].reshape(*value.shape[:-1], -1)

    def table(self, indices: torch.Tensor, limit: float = 0.0):
        """(expert table, indices into it) for one call; see ``resolve_table``."""
        return resolve_table(self.cache, self.layer, indices, limit)

    def __call__(self, value: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        if value.shape[:-1] != indices.shape[:-1]:
            raise ValueError("value and indices disagree on the token axes")
        if getattr(self.cache, "route_trace_enabled", False):
            self.cache.record_routes(self.layer, indices.to("cpu", torch.int32).numpy())
        table, idx = self.table(indices)
        return experts_mxfp4(value, idx, table)


class SparseMoE:
    """Qwen MoE block (qwen4_exp.py:997-1051): softmax top-k router, streamed routed experts,
    sigmoid-gated shared expert, routing-weighted combine.

    ``shared_expert`` is the reference's bf16 ``MLP`` by default; set it to a one-expert
    ``MXFP4Experts`` to run the shared expert inside the fused layer kernels, or to None
    for a layer without one.
    """

    def __init__(self, args, layer: int, cache, device="cuda"):
        H, E = args.hidden_size, args.num_experts
        self.gate = Linear(H, E, device)
        self.experts = StreamingExperts(layer, cache)
        self.shared_expert = MLP(H, args.shared_expert_intermediate_size, device)
        self.shared_expert_gate = Linear(H, 1, device)
        self.top_k = args.num_experts_per_tok
        self.norm_topk_prob = args.norm_topk_prob
        self.cache = cache
        self.layer = layer

    def route(self, value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        """(probabilities [.., E] fp32, indices [.., K] int32) of the router (qwen4_exp.py:1009-1013).
        The router linear accumulates in fp32 as the native engine's GEMV does
        (Native/QwenNative/engine.mm:2080-2091)."""
        logits = linear_bf16(value, self.gate.weight)
        indices, _, probabilities = route_softmax_topk(logits, self.top_k, True, probabilities=True)
        return probabilities, indices

    def _gates(self, value: torch.Tensor, routes=None):
        """(indices, scores, shared) as qwen4_exp.py:1036-1046; shared is None when the shared
        expert runs inside the layer kernel."""
        if routes is None:
            logits = linear_bf16(value, self.gate.weight)
            indices, scores = route_softmax_topk(logits, self.top_k, self.norm_topk_prob)
        else:
            probabilities, indices = routes
            indices = indices.to(torch.int32)
            scores = torch.gather(probabilities.float(), -1, indices.long())
            if self.norm_topk_prob:
                scores = scores / scores.sum(dim=-1, keepdim=True)
        if getattr(self.cache, "route_trace_enabled", False):
            self.cache.record_routes(self.layer, indices.to("cpu", torch.int32).numpy())
        # The shared term is added to the routed combine by the library (_layer); True marks a
        # layer that has a bf16 shared MLP.
        shared = self.shared_expert is not None and not isinstance(self.shared_expert, MXFP4Experts)
        return indices, scores, shared

    def _layer(self, value: torch.Tensor, indices, scores, shared) -> torch.Tensor:
        table, idx = self.experts.table(indices)
        if isinstance(self.shared_expert, MXFP4Experts):
            return moe_mxfp4(value, idx, scores.contiguous(), table, self.shared_expert,
                             self.shared_expert_gate.weight.reshape(-1))
        y = moe_mxfp4(value, idx, scores.contiguous(), table)
        if not shared:
            return y
        # y + sigmoid(x . g) * MLP(x) on the MLP kernels (wm_mlp_bf16)
        return self.shared_expert(value, self.shared_expert_gate.weight.reshape(-1), y)

    def __call__(self, value: torch.Tensor, routes=None) -> torch.Tensor:
        indices, scores, shared = self._gates(value, routes)
        return self._layer(value, indices, scores, shared)

    def merged(self, values: list[torch.Tensor]) -> list[torch.Tensor]:
        """Each value through this block with one routed-expert call for all of them
        (qwen4_exp.py:1020-1034)."""
        gates = [self._gates(value) for value in values]
        axis = values[0].dim() - 2
        joined = torch.cat(values, dim=axis)
        indices = torch.cat([g[0] for g in gates], dim=axis)
        scores = torch.cat([g[1] for g in gates], dim=axis)
        y = self._layer(joined, indices, scores, gates[0][2])
        return list(torch.split(y, [v.shape[axis] for v in values], dim=axis))

    @staticmethod
    def _combine(routed: torch.Tensor, scores: torch.Tensor, shared: torch.Tensor) -> torch.Tensor:
        """sum_k scores_k * routed_k + shared (qwen4_exp.py:1048-1051), fp32 accumulation in k
        order (wm_combine_pairs)."""
        return combine_pairs(routed, scores.float(), shared)


# ----------------------------------------------------------------------------- DeepSeek operators

class _StreamingSwitchGLU:
    """DeepSeek routed experts: __call__(x [.., H], indices [.., K]) -> [.., K, H] in router
    order (model.py:318-385). ``activation(up, gate)``: ClampedSwiGLU / SwiGLU (or None)
    run fused in the expert kernels; any other callable takes the dequantize-then-GEMM
    path (the reference tests' ``lambda up, _gate: up``, test_runtime.py:2509-2745)."""

    def __init__(self, layer: int, cache, activation=None):
        self.layer = layer
        self.cache = cache
        self.activation = activation

    def _table(self, indices: torch.Tensor, limit: float):
        return resolve_table(self.cache, self.layer, indices, limit)

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        if x.shape[:-1] != indices.shape[:-1]:
            raise ValueError("x and indices disagree on the token axes")
        if getattr(self.cache, "route_trace_enabled", False):
            self.cache.record_routes(self.layer, indices.to("cpu", torch.int32).numpy())
        limit = _fused_limit(self.activation)
        table, idx = self._table(indices, 0.0 if limit is None else limit)
        if limit is None:
            H = x.shape[-1]
            T = x.numel() // H
            out = _generic_experts(x.reshape(T, H), idx.reshape(T, -1), table, self.activation)
            return out.reshape(*indices.shape, H)
        if isinstance(table, FP8Experts):
            return experts_fp8(x, idx, table)
        return experts_mxfp4(x, idx, table)

    def forward_with_resident(self, x: torch.Tensor, indices: torch.Tensor, resident: ResidentExperts):
        """Token-shaped expert math from one pre-acquired union (model.py:387-395)."""
        ids = _host_ids(indices, None)
        unique = sorted(set(ids))
        limit = _fused_limit(self.activation)
        table, idx = _resident_table(resident, unique, 0.0 if limit is None else limit, ids, indices)
        if limit is None:
            H = x.shape[-1]
            T = x.numel() // H
            return _generic_experts(x.reshape(T, H), idx.reshape(T, -1), table, self.activation).reshape(
                *indices.shape, H)
        return (experts_fp8 if isinstance(table, FP8Experts) else experts_mxfp4)(x, idx, table)


class Gate:
    """DeepSeek router over precomputed logits-producing weight (deepseek_v41/moe.py:46-74):
    scores f(x . W^T / temp), selection on scores + bias (ties -> lower index), weights
    from the unbiased scores, normalised (sum + 1e-20) and scaled by route_scale. ``n_groups``
    > 1 adds DeepSeek-V3 group-limited selection."""

    def __init__(self, dim: int, experts: int, topk: int, score_func: str = "sqrtsoftplus",
                 route_scale: float = 1.0, norm_topk_prob: bool = True, gate_temp: float = 1.0,
                 n_groups: int = 1, topk_groups: int = 1, device="cuda"):
        self.weight = torch.zeros(experts, dim, dtype=torch.bfloat16, device=device)
        self.bias = torch.zeros(experts, dtype=torch.float32, device=device)
        self.topk, self.score_func, self.route_scale = topk, score_func, route_scale
        self.norm_topk_prob, self.gate_temp = norm_topk_prob, gate_temp
        self.n_groups, self.topk_groups = n_groups, topk_groups

    def __call__(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        logits = linear_bf16(x, self.weight)
        if self.gate_temp != 1.0:
            logits = logits / self.gate_temp
        indices, weights = route_scored(logits, self.bias, self.topk, self.score_func, self.route_scale,
                                        self.norm_topk_prob and self.topk > 1, self.n_groups, self.topk_groups)
        return weights, indices


def route_reduce(routed: torch.Tensor, scores: torch.Tensor, add: torch.Tensor | None = None) -> torch.Tensor:
    """sum_k routed_k * scores_k (+ add) (model.py:544-546, :540-541), fp32 accumulation in k
    order, bf16 out (wm_combine_pairs)."""
    return combine_pairs(routed, scores.float(), add)


def streaming_moe(gate: Gate, switch_mlp: _StreamingSwitchGLU, shared, x: torch.Tensor) -> torch.Tensor:
    """The DeepSeek MoE forward (model.py:526-541): routed experts reduced by the routing
    weights, plus the ungated shared expert. ``shared`` is a one-expert table (fused into
    the layer kernel when the activation is SwiGLU) or a callable on x."""
    weights, indices = gate(x)
    limit = _fused_limit(switch_mlp.activation)
    if limit is not None and isinstance(shared, (MXFP4Experts, FP8Experts)):
        table, idx = switch_mlp._table(indices, limit)
        shared = replace(shared, swiglu_limit=limit)
        if isinstance(table, FP8Experts):
            return moe_fp8(x, idx, weights, table, shared, None)
        return moe_mxfp4(x, idx, weights, table, shared, None)
    return route_reduce(switch_mlp(x, indices), weights, shared(x).to(torch.bfloat16))
