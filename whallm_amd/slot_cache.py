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


def qwen_blob_bytes(hidden: int, inter: int) -> int:
    """One expert blob: gate_up | gate_up scales | down | down scales (manifest.py:41-45)."""
    return 2 * inter * hidden // 2 + 2 * inter * hidden // 32 + hidden * inter // 2 + hidden * inter // 32


class SlotCacheError(RuntimeError):
    pass


class SlotCache:
    """``slots`` resident expert blobs of one model shape, filled from ``host_pool``
    (pinned uint8 [files * experts * blob]) on demand.

    With ``device=None`` the handle runs the policy only (plan(); no device memory),
    which is what host-side tests use.
    """

    def __init__(self, slots: int, hidden: int, inter: int, files: int, experts: int,
                 host_pool: torch.Tensor | None = None, device: torch.device | str | None = None):
        self.slots, self.hidden, self.inter, self.files, self.experts = slots, hidden, inter, files, experts
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
        """Make ``experts`` of ``file`` resident; the current torch stream waits for the fills."""
        if self.device is None:
            raise SlotCacheError("policy-only cache")
        ids = np.ascontiguousarray(np.asarray(experts, np.int32).reshape(-1))
        out = np.empty(ids.size, np.int32)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        self._check(_lib.load().wm_slot_cache_acquire(self._handle, file, ids.ctypes.data, ids.size, out.ctypes.data,
                                                      ctypes.c_void_p(stream)), "acquire")
        return out.tolist()

    def table(self, file: int) -> MXFP4Experts:
        """The resident experts of ``file`` as an expert table (views of the slot memory)."""
        H, I, b = self.hidden, self.inter, self.blob
        mem = self.slot_memory.view(self.slots, b)
        o1 = 2 * I * H // 2
        o2 = o1 + 2 * I * H // 32
        o3 = o2 + H * I // 2
        return MXFP4Experts(
            gate_up=mem[:, :o1].view(torch.int32).view(self.slots, 2 * I, H // 8),
            gate_up_scales=mem[:, o1:o2].view(self.slots, 2 * I, H // 32),
            down=mem[:, o2:o3].view(torch.int32).view(self.slots, H, I // 8),
            down_scales=mem[:, o3:].view(self.slots, H, I // 32),
            slots=self.map[file], experts=self.experts)

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
