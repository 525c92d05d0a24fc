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
from .ops import MXFP4Experts, experts_mxfp4


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
        self.route_policy = False
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
        out = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire(self._handle, file, ids.ctypes.data, ids.size, out.ctypes.data,
                                                      ctypes.c_void_p(stream)), "acquire")
        return out.tolist()

    def acquire_ready(self, file: int, experts) -> tuple[list[int], list[bool]]:
        """The cached-first acquire (engine.mm:2204-2234): (slots, ready flags). Ready experts
        were resident already and may be used by work enqueued now; the others are being
        filled on the copy stream until ``wait_fills()``."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        out = np.empty(ids.size, np.int32)
        ready = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire_ready(self._handle, file, ids.ctypes.data, ids.size,
                                                            out.ctypes.data, ready.ctypes.data,
                                                            ctypes.c_void_p(stream)), "acquire_ready")
        return out.tolist(), [bool(r) for r in ready]

    def start_fills(self) -> None:
        """Enqueues the fills ``acquire_split`` held back (engine.mm:2225-2231: the reads
        follow the ready pairs' submission)."""
        self._check(_lib.load().wm_slot_cache_start_fills(self._handle), "start_fills")

    def wait_fills(self) -> None:
        """The current stream waits for the fills of earlier ``acquire_ready`` calls."""
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_wait_fills(self._handle, ctypes.c_void_p(stream)), "wait_fills")

    def acquire_split(self, file: int, indices: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, bool]:
        """The cached-first acquire of one call's pairs (engine.mm:2204-2230): plans the call's
        experts and splits ``indices`` on the current stream into (ready, late) id tensors (-1
        where a pair is in the other set) with no host -> device copy. The fills are held back
        until ``start_fills`` (or the next call on the cache), so the ready pairs can be
        enqueued first. Returns (ready, late, whether any pair is late). ``indices`` is read on
        the host, as the reference's acquire is."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        idx = indices.to(torch.int32).contiguous()
        unique = np.ascontiguousarray(sorted(set(idx.cpu().reshape(-1).tolist())), np.int32)
        unique = unique[(unique >= 0) & (unique < self.experts)]
        slots = np.empty(unique.size, np.int32)
        ready = np.empty(unique.size, np.int32)
        ready_idx, late_idx = torch.empty_like(idx), torch.empty_like(idx)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire_split(
            self._handle, file, unique.ctypes.data, unique.size, slots.ctypes.data, ready.ctypes.data,
            idx.data_ptr(), idx.numel(), ready_idx.data_ptr(), late_idx.data_ptr(), ctypes.c_void_p(stream)),
            "acquire_split")
        return ready_idx, late_idx, not bool(ready.all())

    def experts_ready_first(self, file: int, x: torch.Tensor, indices: torch.Tensor,
                            out: torch.Tensor | None = None) -> torch.Tensor:
        """Per-pair outputs [.., K, H] of ``file``'s experts in router order, the pairs whose
        experts are resident computed while the missing ones are copied in, the rest after
        (the native engine's ready-then-late order, engine.mm:2204-2234). The result equals
        one call with every expert resident, bit for bit."""
        ready_idx, late_idx, any_late = self.acquire_split(file, indices)
        table = self.table(file)
        out = experts_mxfp4(x, ready_idx, table, out=out)
        self.start_fills()
        self.wait_fills()
        if any_late:
            experts_mxfp4(x, late_idx, table, out=out)
        return out

    def acquire_files(self, requests: dict) -> dict:
        """One plan over several files ({file: expert ids}): every requested expert is resident
        together afterwards (the persistent decode stack reads all layers in one launch)."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        files = np.ascontiguousarray(list(requests), np.int32)
        lists = [np.asarray(requests[int(f)], np.int32).reshape(-1) for f in files]
        counts = np.ascontiguousarray([a.size for a in lists], np.int32)
        ids = np.ascontiguousarray(np.concatenate(lists) if lists else np.zeros(0, np.int32), np.int32)
        out = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire_files(self._handle, files.size, files.ctypes.data,
                                                            counts.ctypes.data, ids.ctypes.data, out.ctypes.data,
                                                            ctypes.c_void_p(stream)), "acquire_files")
        got, at = {}, 0
        for f, n in zip(files.tolist(), counts.tolist()):
            got[f] = out[at:at + n].tolist()
            at += n
        return got

    # ---- route mode: the native route-history policy (expert_cache.py:806-815, 1088-1181)

    def enable_route_policy(self, top_k: int) -> None:
        """Evict by the cache's route-history policy (files = layers) instead of LFU; acquires
        then count as routes of the current phase."""
        self._check(_lib.load().wm_slot_cache_route_policy(self._handle, int(top_k)), "route_policy")
        self.route_policy = True

    def disable_route_policy(self) -> None:
        self._check(_lib.load().wm_slot_cache_route_policy(self._handle, 0), "route_policy")
        self.route_policy = False

    def observe(self, file: int, selected, phase: str | None = None) -> None:
        """Routes of ``file`` that bypassed the slots (observe_batched_routes, :1115-1118):
        token-major expert ids, top_k per token."""
        ids = np.ascontiguousarray(np.asarray(selected, np.int32).reshape(-1))
        prefill = (phase or self.route_phase) == "prefill"
        self._check(_lib.load().wm_slot_cache_route_observe(self._handle, file, ids.ctypes.data, ids.size,
                                                            int(prefill)), "route_observe")

    def begin_route_request(self) -> None:
        """A new prompt: its routes become the prior (begin_route_request, :1105-1109)."""
        if self.route_policy:
            self._check(_lib.load().wm_slot_cache_route_begin_request(self._handle), "route_begin_request")

    def set_route_phase(self, phase: str) -> None:
        """"prefill" or "decode"; leaving a prefill rebalances (trace_routes, :1088-1103)."""
        if phase not in ("prefill", "decode"):
            raise ValueError("phase must be 'prefill' or 'decode'")
        self.route_phase = phase
        self._check(_lib.load().wm_slot_cache_route_phase(self._handle, int(phase == "prefill")), "route_phase")

    def record_read(self, file: int, seconds: float) -> None:
        if self.route_policy:
            self._check(_lib.load().wm_slot_cache_route_record_read(self._handle, file, float(seconds)),
                        "route_record_read")

    def rebalance(self) -> None:
        self._check(_lib.load().wm_slot_cache_route_rebalance(self._handle), "route_rebalance")

    def route_state(self) -> dict:
        """The policy's arrays: scores and short / long rates [files, experts], quotas,
        decode / prompt tokens and read cost per file, rebalances and slot capacity."""
        F, E = self.files, self.experts
        scores, short, long_ = (np.empty((F, E), np.float64) for _ in range(3))
        quotas = np.empty(F, np.int32)
        tokens = np.empty(2 * F, np.int64)
        cost = np.empty(F, np.float64)
        counters = np.empty(2, np.int64)
        self._check(_lib.load().wm_slot_cache_route_state(
            self._handle, scores.ctypes.data, quotas.ctypes.data, short.ctypes.data, long_.ctypes.data,
            tokens.ctypes.data, cost.ctypes.data, counters.ctypes.data), "route_state")
        return {"scores": scores, "quotas": quotas, "short": short, "long": long_, "decode_tokens": tokens[:F],
                "prompt_tokens": tokens[F:], "read_cost": cost, "rebalances": int(counters[0]),
                "capacity": int(counters[1])}

    # ---- whole-file reads and prompt-tail seeding (engine.mm:1647-1678)

    def layer_buffer(self) -> torch.Tensor:
        """A device buffer for one whole file (experts x blob bytes)."""
        return torch.empty(self.experts * self.blob, dtype=torch.uint8, device=self.device)

    def read_layer(self, file: int, buffer: torch.Tensor, experts=None) -> None:
        """Start reading ``file`` into ``buffer`` on the copy stream (after the current stream's
        earlier work, which may still read the buffer): the whole file, or only ``experts``
        (sorted unique ids; consecutive ids are read together, up to 32 blobs a copy)."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        if buffer.device != self.device or buffer.dtype != torch.uint8 or buffer.numel() < self.experts * self.blob \
                or not buffer.is_contiguous():
            raise ValueError("the layer buffer must be a contiguous uint8 device tensor of experts * blob bytes")
        stream = ctypes.c_void_p(torch.cuda.current_stream(self.device).cuda_stream)
        if experts is None:
            self._check(_lib.load().wm_slot_cache_read_layer(self._handle, file, ctypes.c_void_p(buffer.data_ptr()),
                                                             stream), "read_layer")
            return
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        self._check(_lib.load().wm_slot_cache_read_experts(self._handle, file, ids.ctypes.data, ids.size,
                                                           ctypes.c_void_p(buffer.data_ptr()), stream), "read_experts")

    def wait_layer(self, file: int) -> None:
        """The current stream waits for the last read_layer of ``file``."""
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_wait_layer(self._handle, file, ctypes.c_void_p(stream)), "wait_layer")

    def layer_table(self, buffer: torch.Tensor) -> MXFP4Experts:
        """The experts of a whole-file buffer as an expert table (expert e = blob e)."""
        return self._blob_table(buffer.view(self.experts, self.blob), self.experts, None)

    def seed_tail(self, file: int, routes: torch.Tensor, limit: int, buffer: torch.Tensor) -> tuple[list, list]:
        """Prompt-tail seeding (expert_cache.py:1399-1430): the experts of the last 128 token
        rows of ``routes`` (int32 [T, K] on the device) ranked by count, latest use and id on
        the device; the first ``limit`` that are not resident go into free slots from the
        whole-file ``buffer``. Returns (experts, slots), least valuable first."""
        if routes.dtype != torch.int32 or not routes.is_contiguous() or routes.device != self.device:
            raise ValueError("routes must be a contiguous int32 device tensor [tokens, k]")
        k = routes.shape[-1]
        rows = routes.numel() // k if k else 0
        experts = np.empty(max(limit, 1), np.int32)
        slots = np.empty(max(limit, 1), np.int32)
        count = np.zeros(1, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_seed_tail(self._handle, file, ctypes.c_void_p(routes.data_ptr()), rows, k,
                                                        limit, ctypes.c_void_p(buffer.data_ptr()), experts.ctypes.data,
                                                        slots.ctypes.data, count.ctypes.data,
                                                        ctypes.c_void_p(stream)), "seed_tail")
        n = int(count[0])
        return experts[:n].tolist(), slots[:n].tolist()

    def seed(self, file: int, experts, uses, buffer: torch.Tensor) -> list[int]:
        """Keep ``experts`` of ``file`` (least valuable first) resident with use counts ``uses``
        (or None), copied from the whole-file ``buffer`` (the native engine's seed_layer)."""
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
        out = (ctypes.c_int64 * 5)()
        _lib.load().wm_slot_cache_stats(self._handle, out)
        return {"hits": out[0], "misses": out[1], "bytes": out[2], "fills": out[3], "copies": out[4]}

    def close(self) -> None:
        if getattr(self, "_handle", None):
            _lib.load().wm_slot_cache_close(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
