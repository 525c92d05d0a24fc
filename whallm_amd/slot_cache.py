"""HBM expert slot cache over a pinned host pool (the reference's ExpertArena /
ExpertCache, Native/QwenNative/engine.mm:649-778, runtime/deepseek_v4_ssd/expert_cache.py).

The slot memory and the expert -> slot map are torch device tensors owned here;
the native handle (libwhallm_moe) runs the replacement policy and enqueues the
fills on its own copy stream. ``table(file)`` returns an ``MXFP4Experts`` view over
the slots whose ``slots`` map routes expert ids to slots, so every expert kernel
reads resident experts without a host-side gather.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib
from .ops import MXFP4Experts
from .route_cache import RouteCachePolicy


def qwen_blob_bytes(hidden: int, inter: int) -> int:
    """One expert blob: gate_up | gate_up scales | down | down scales (manifest.py:41-45)."""
    return 2 * inter * hidden // 2 + 2 * inter * hidden // 32 + hidden * inter // 2 + hidden * inter // 32


def blob_table(mem: torch.Tensor, hidden: int, inter: int, *, slots=None, experts=None,
               up_first: bool = False, swiglu_limit: float = 0.0) -> MXFP4Experts:
    """The expert table over blobs in slot order (uint8 [count, blob]: gate_up | gate_up scales |
    down | down scales, the Qwen blob of manifest.py:37-42); ``up_first`` when the gate_up
    rows are up then gate (DeepSeek's w13 = w3 | w1)."""
    H, I = hidden, inter
    count = mem.shape[0]
    o1 = 2 * I * H // 2
    o2 = o1 + 2 * I * H // 32
    o3 = o2 + H * I // 2
    return MXFP4Experts(
        gate_up=mem[:, :o1].view(torch.int32).view(count, 2 * I, H // 8),
        gate_up_scales=mem[:, o1:o2].view(count, 2 * I, H // 32),
        down=mem[:, o2:o3].view(torch.int32).view(count, H, I // 8),
        down_scales=mem[:, o3:].view(count, H, I // 32),
        slots=slots, experts=experts, up_first=up_first, swiglu_limit=swiglu_limit)


class SlotCacheError(RuntimeError):
    pass


class SlotCache:
    """``slots`` resident expert blobs of one model shape, filled from ``host_pool``
    (pinned uint8 [files * experts * blob]) on demand.

    With ``device=None`` the handle runs the policy only (plan(); no device memory),
    which is what host-side tests use. ``up_first`` / ``swiglu_limit`` are carried into the
    tables (DeepSeek blobs: w13 = up rows then gate rows, clamped SwiGLU).
    """

    def __init__(self, slots: int, hidden: int, inter: int, files: int, experts: int,
                 host_pool: torch.Tensor | None = None, device: torch.device | str | None = None,
                 up_first: bool = False, swiglu_limit: float = 0.0):
        self.slots, self.hidden, self.inter, self.files, self.experts = slots, hidden, inter, files, experts
        self.up_first, self.swiglu_limit = bool(up_first), float(swiglu_limit)
        self.blob = qwen_blob_bytes(hidden, inter)
        lib = _lib.load()
        self.device = None if device is None else torch.device(device)
        self.slot_memory = self.map = None
        self.host_pool = host_pool
        if self.device is not None:
            if host_pool is None or host_pool.dtype != torch.uint8 or host_pool.is_cuda:
                raise ValueError("a device-backed cache needs a host uint8 pool")
            if not host_pool.is_pinned():
                raise ValueError("the host pool must be pinned (torch pin_memory / hipHostMalloc)")
            if host_pool.numel() < files * experts * self.blob or not host_pool.is_contiguous():
                raise ValueError("the host pool must hold files * experts contiguous blobs")
            self.slot_memory = torch.empty(slots * self.blob, dtype=torch.uint8, device=self.device)
            self.map = torch.full((files, experts), -1, dtype=torch.int32, device=self.device)
        err = ctypes.create_string_buffer(512)
        handle = lib.wm_slot_cache_open(
            slots, self.blob, files, experts,
            None if self.slot_memory is None else self.slot_memory.data_ptr(),
            None if self.map is None else self.map.data_ptr(),
            None if self.device is None else host_pool.data_ptr(), err, len(err))
        if not handle:
            raise SlotCacheError(err.value.decode(errors="replace"))
        self._handle = ctypes.c_void_p(handle)
        self.route_policy: RouteCachePolicy | None = None
        self.route_phase = "decode"

    def _check(self, status: int, what: str) -> None:
        if status != 0:
            raise SlotCacheError(f"{what}: {_lib.load().wm_slot_cache_error(self._handle).decode(errors='replace')}")

    def plan(self, file: int, experts) -> tuple[list[int], list[int]]:
        """(slots, filled flags) for ``experts`` of ``file``; no copies (ExpertArena::plan)."""
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        out = np.empty(ids.size, np.int32)
        filled = np.empty(ids.size, np.int32)
        self._check(_lib.load().wm_slot_cache_plan(self._handle, file, ids.ctypes.data, ids.size, out.ctypes.data,
                                                   filled.ctypes.data), "plan")
        return out.tolist(), filled.tolist()

    def acquire(self, file: int, experts) -> list[int]:
        """Make ``experts`` of ``file`` resident; the current torch stream waits for the fills.
        In route mode the request counts as routes of ``file`` (expert_cache.py:1483)."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        if self.route_policy is not None:
            self.observe(file, ids)
        out = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire(self._handle, file, ids.ctypes.data, ids.size, out.ctypes.data,
                                                      ctypes.c_void_p(stream)), "acquire")
        return out.tolist()

    # ---- route mode (ExpertCache with eviction_policy "route", expert_cache.py:806-815, 1088-1181)

    def enable_route_policy(self, top_k: int) -> RouteCachePolicy:
        """Evict by the route-history policy (files = layers) instead of LFU."""
        self.route_policy = RouteCachePolicy(self.files, self.experts, self.slots, top_k)
        self._push_route()
        return self.route_policy

    def _push_route(self) -> None:
        pol = self.route_policy
        scores = np.ascontiguousarray(pol.scores, np.float64)
        quotas = np.ascontiguousarray(pol.quotas, np.int32)
        self._check(_lib.load().wm_slot_cache_set_route(self._handle, scores.ctypes.data, quotas.ctypes.data),
                    "set_route")

    def observe(self, file: int, selected, phase: str | None = None) -> None:
        """Routes of ``file`` (expert ids, top_k per token) for the route policy; a batched
        prefill that bypasses the slots reports its routes here (observe_batched_routes)."""
        if self.route_policy is not None and self.route_policy.observe(file, selected, phase or self.route_phase):
            self._push_route()

    def begin_route_request(self) -> None:
        """A new prompt (begin_route_request, expert_cache.py:1105-1109)."""
        if self.route_policy is not None:
            self.route_policy.begin_prefill()

    def set_route_phase(self, phase: str) -> None:
        """"prefill" or "decode"; leaving a prefill rebalances (trace_routes, :1088-1103)."""
        previous, self.route_phase = self.route_phase, phase
        if self.route_policy is not None and previous == "prefill" and phase != "prefill":
            self.route_policy.rebalance()
            self._push_route()

    def record_read(self, file: int, seconds: float) -> None:
        if self.route_policy is not None:
            self.route_policy.record_read(file, seconds)

    def disable_route_policy(self) -> None:
        self.route_policy = None
        self._check(_lib.load().wm_slot_cache_set_route(self._handle, None, None), "set_route")

    # ---- whole-file reads and prompt-tail seeding (engine.mm:1647-1678)

    def layer_buffer(self) -> torch.Tensor:
        """A device buffer for one whole file (experts x blob bytes)."""
        return torch.empty(self.experts * self.blob, dtype=torch.uint8, device=self.device)

    def read_layer(self, file: int, buffer: torch.Tensor) -> None:
        """Start reading the whole of ``file`` into ``buffer`` on the copy stream (after the
        current stream's earlier work, which may still read the buffer)."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        if buffer.device != self.device or buffer.dtype != torch.uint8 or buffer.numel() < self.experts * self.blob \
                or not buffer.is_contiguous():
            raise ValueError("the layer buffer must be a contiguous uint8 device tensor of experts * blob bytes")
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_read_layer(self._handle, file, ctypes.c_void_p(buffer.data_ptr()),
                                                         ctypes.c_void_p(stream)), "read_layer")

    def wait_layer(self, file: int) -> None:
        """The current stream waits for the last read_layer of ``file``."""
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_wait_layer(self._handle, file, ctypes.c_void_p(stream)), "wait_layer")

    def layer_table(self, buffer: torch.Tensor) -> MXFP4Experts:
        """The experts of a whole-file buffer as an expert table (expert e = blob e)."""
        return self._blob_table(buffer.view(self.experts, self.blob), self.experts, None)

    def seed(self, file: int, experts, uses, buffer: torch.Tensor) -> list[int]:
        """Keep ``experts`` of ``file`` (least valuable first, e.g. hot_tail_experts) resident
        with use counts ``uses`` (or None), copied from the whole-file ``buffer``."""
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        cnt = None if uses is None else np.ascontiguousarray(np.asarray(uses, np.int32).reshape(-1))
        if cnt is not None and cnt.size != ids.size:
            raise ValueError("uses must match experts")
        out = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_seed(self._handle, file, ids.ctypes.data,
                                                   None if cnt is None else cnt.ctypes.data, ids.size,
                                                   ctypes.c_void_p(buffer.data_ptr()), out.ctypes.data,
                                                   ctypes.c_void_p(stream)), "seed")
        return out.tolist()

    def _blob_table(self, mem: torch.Tensor, count: int, slots) -> MXFP4Experts:
        return blob_table(mem.view(count, self.blob), self.hidden, self.inter, slots=slots, experts=self.experts,
                          up_first=self.up_first, swiglu_limit=self.swiglu_limit)

    def table(self, file: int) -> MXFP4Experts:
        """The resident experts of ``file`` as an expert table (views of the slot memory)."""
        return self._blob_table(self.slot_memory.view(self.slots, self.blob), self.slots, self.map[file])

    def stats(self) -> dict:
        out = (ctypes.c_int64 * 4)()
        _lib.load().wm_slot_cache_stats(self._handle, out)
        return {"hits": out[0], "misses": out[1], "bytes": out[2], "fills": out[3]}

    def close(self) -> None:
        if getattr(self, "_handle", None):
            _lib.load().wm_slot_cache_close(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
