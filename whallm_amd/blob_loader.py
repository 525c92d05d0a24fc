"""Installed expert files into pinned host memory: the slot cache's host pool filled from
the reference's on-disk format instead of synthetic weights.

An installed model directory holds `manifest.json` and one file per MoE layer,
`experts/layer_XX.bin` = expert_count blobs of expert_blob_size bytes, each blob laid out
by the manifest's `expertRegions` (name, dtype, shape, offset, length)
(runtime/deepseek_v4_ssd/manifest.py:21-42, :150-175; expert_layout.py:8-119). The
checks follow InstalledModel.open for the files read here: unique paths, files inside the
directory with the manifest's sizes, layer files of expert_count whole blobs; the regions
must partition the blob and form an MXFP4 expert.

The pool holds every blob in slot order, gate_up | gate_up scales | down | down scales
(the Qwen blob, so one table layout serves the slot cache for both models):
  - Qwen (gate_up.weight U32, gate_up.scale U8, down.weight U32, down.scale U8): read as
    is when the file already has that order (GateUpMXFP4Layout);
  - DeepSeek (w1 / w2 / w3 packed E2M1 bytes, E8M0 scales): rewritten to
    w3 | w1 | w3.scale | w1.scale | w2 | w2.scale, so w13 = up rows then gate rows is one
    region (up_first) and so are its scales, as in the reference's fused slot
    (expert_layout.py:8-62, ExpertCache.store's region copy, expert_cache.py:498-510).
Weight bytes are little-endian 32-bit words of eight E2M1 codes, low nibble first, as the
reference views them (expert_cache.py:488-497).
"""
from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path

import torch

from .ops import MXFP4Experts
from .slot_cache import SlotCache, blob_table

QWEN_REGIONS = ("gate_up.weight", "gate_up.scale", "down.weight", "down.scale")
DEEPSEEK_REGIONS = ("w1.weight", "w1.scale", "w2.weight", "w2.scale", "w3.weight", "w3.scale")
# the regions of each kind in slot order
SLOT_ORDER = {"qwen": QWEN_REGIONS,
              "deepseek": ("w3.weight", "w1.weight", "w3.scale", "w1.scale", "w2.weight", "w2.scale")}
MAX_IOV = 1024  # buffers per scatter read (the usual IOV_MAX)


def _read_scatter(fd: int, offset: int, bufs: list, path) -> None:
    """Fill ``bufs`` in order from the file at ``offset`` (preadv, resumed after short reads)."""
    while bufs:
        got = os.preadv(fd, bufs, offset)
        if got <= 0:
            raise ValueError(f"short read of {path}")
        offset += got
        while bufs and got >= len(bufs[0]):
            got -= len(bufs[0])
            bufs = bufs[1:]
        if got:
            bufs[0] = bufs[0][got:]


@dataclass(frozen=True)
class Region:
    name: str
    dtype: str
    shape: tuple
    offset: int
    length: int


class ExpertFiles:
    """The expert layer files of an installed model directory (validated on open)."""

    def __init__(self, root: str | Path):
        self.root = Path(root).expanduser().resolve()
        with (self.root / "manifest.json").open("rb") as f:
            raw = json.load(f)
        files = {item["path"]: int(item["size"]) for item in raw.get("files", [])}
        if len(files) != len(raw.get("files", [])):
            raise ValueError("installed manifest contains duplicate file paths")
        self.regions = {r["name"]: Region(r["name"], r["dtype"], tuple(r["shape"]), int(r["offset"]), int(r["length"]))
                        for r in raw.get("expertRegions", [])}
        names = set(self.regions)
        if names == set(QWEN_REGIONS):
            self.kind = "qwen"
        elif names == set(DEEPSEEK_REGIONS):
            self.kind = "deepseek"
        else:
            raise ValueError("expert blob does not contain the required regions")
        # the regions must partition the blob: contiguous, no gaps, no overlaps
        at = 0
        for r in sorted(self.regions.values(), key=lambda r: r.offset):
            if r.offset != at or r.length <= 0:
                raise ValueError(f"expert region {r.name} does not partition the blob")
            at += r.length
        self.blob = at
        layers = sorted(p for p in files if p.startswith("experts/layer_") and p.endswith(".bin"))
        if not layers or [f"experts/layer_{i:02d}.bin" for i in range(len(layers))] != layers:
            raise ValueError("installed model has no contiguous experts/layer_XX.bin files")
        sizes = {files[p] for p in layers}
        if len(sizes) != 1 or next(iter(sizes)) % self.blob:
            raise ValueError("installed expert layer has an invalid size")
        self.layers = len(layers)
        self.experts = next(iter(sizes)) // self.blob
        for p in layers:
            target = (self.root / p).resolve()
            if self.root not in target.parents or not target.is_file():
                raise ValueError(f"installed model has an unsafe or missing file: {p}")
            if target.stat().st_size != files[p]:
                raise ValueError(f"installed file size does not match the manifest: {p}")
        self._check_shapes()

    def _check_shapes(self) -> None:
        r = self.regions
        if self.kind == "qwen":
            gu, gus, dn, dns = (r[n] for n in QWEN_REGIONS)
            two_i, h8 = gu.shape
            h, i8 = dn.shape
            ok = (gu.dtype == "U32" and dn.dtype == "U32" and gus.dtype == "U8" and dns.dtype == "U8"
                  and gus.shape == (two_i, 8 * h8 // 32) and dns.shape == (h, 8 * i8 // 32)
                  and h == 8 * h8 and 2 * 8 * i8 == two_i)
            self.hidden, self.inter = h, two_i // 2
        else:
            w1, w1s, w2, w2s, w3, w3s = (r[n] for n in DEEPSEEK_REGIONS)
            i, h2 = w1.shape
            h, i2 = w2.shape
            ok = (w1.shape == w3.shape and w1s.shape == w3s.shape and w1s.shape == (i, 2 * h2 // 32)
                  and w2s.shape == (h, 2 * i2 // 32) and h == 2 * h2 and i == 2 * i2
                  and all(r[n].dtype in ("I8", "U8") for n in ("w1.weight", "w2.weight", "w3.weight"))
                  and all(r[n].dtype in ("F8_E8M0", "U8") for n in ("w1.scale", "w2.scale", "w3.scale")))
            self.hidden, self.inter = h, i
        if not ok:
            raise ValueError("expert region shapes do not form an MXFP4 expert")

    @property
    def in_slot_order(self) -> bool:
        """True when the file's blobs are already in slot order (no rewrite on read)."""
        at = 0
        for name in SLOT_ORDER[self.kind]:
            if self.regions[name].offset != at:
                return False
            at += self.regions[name].length
        return True

    def read(self, layers=None, pinned: bool = True) -> torch.Tensor:
        """uint8 host pool [len(layers)][experts][blob] in slot order, one whole-file read per
        layer; pool file n holds model layer layers[n]. Pinned (page-locked) for the slot
        cache's copies unless ``pinned`` is False."""
        layers = list(range(self.layers)) if layers is None else [int(l) for l in layers]
        if any(not 0 <= l < self.layers for l in layers):
            raise ValueError("layer out of range")
        pool = torch.empty(len(layers) * self.experts * self.blob, dtype=torch.uint8, pin_memory=pinned)
        view = pool.numpy().reshape(len(layers), self.experts, self.blob)
        # each region's place in the slot, taken in the file's order: one scatter read per
        # batch of experts lands every region in its slot position with no second copy
        slot_at, at = {}, 0
        for name in SLOT_ORDER[self.kind]:
            slot_at[name] = at
            at += self.regions[name].length
        file_order = sorted(self.regions.values(), key=lambda r: r.offset)
        batch = max(1, MAX_IOV // len(file_order))
        for n, layer in enumerate(layers):
            path = self.root / f"experts/layer_{layer:02d}.bin"
            fd = os.open(path, os.O_RDONLY)
            try:
                for e0 in range(0, self.experts, batch):
                    bufs = [memoryview(view[n, e, slot_at[r.name]:slot_at[r.name] + r.length])
                            for e in range(e0, min(e0 + batch, self.experts)) for r in file_order]
                    _read_scatter(fd, e0 * self.blob, bufs, path)
            finally:
                os.close(fd)
        return pool

    def table(self, pool: torch.Tensor, layer: int, swiglu_limit: float = 0.0) -> MXFP4Experts:
        """Expert table over file ``layer`` of a pool from read() (or a device copy of it)."""
        mem = pool.view(-1, self.experts, self.blob)[layer]
        return blob_table(mem, self.hidden, self.inter, up_first=self.kind == "deepseek",
                          swiglu_limit=swiglu_limit)

    def slot_cache(self, slots: int, pool: torch.Tensor, device, swiglu_limit: float = 0.0) -> SlotCache:
        """An HBM slot cache of ``slots`` blobs filled from ``pool`` (from read())."""
        return SlotCache(slots, self.hidden, self.inter, pool.numel() // (self.experts * self.blob), self.experts,
                         pool, device, up_first=self.kind == "deepseek", swiglu_limit=swiglu_limit)
