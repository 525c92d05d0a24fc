"""Synthetic installed-model directories in the reference's on-disk format (manifest.json with
`files` and `expertRegions`, experts/layer_XX.bin of expert_count blobs;
runtime/deepseek_v4_ssd/manifest.py:21-42, :150-175) at small shapes, with the source
arrays they were written from."""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np

from whallm_amd import synthetic as S


def regions(kind: str, hidden: int, inter: int):
    """(name, dtype, shape, length) in the reference's file order for ``kind``."""
    H, I = hidden, inter
    if kind == "qwen":   # QWEN_EXPERT_REGIONS (manifest.py:37-42) at H, I
        return [("gate_up.weight", "U32", [2 * I, H // 8], 2 * I * H // 2),
                ("gate_up.scale", "U8", [2 * I, H // 32], 2 * I * H // 32),
                ("down.weight", "U32", [H, I // 8], H * I // 2),
                ("down.scale", "U8", [H, I // 32], H * I // 32)]
    # EXPERT_REGIONS (manifest.py:21-28) at H, I
    return [("w1.weight", "I8", [I, H // 2], I * H // 2), ("w1.scale", "F8_E8M0", [I, H // 32], I * H // 32),
            ("w2.weight", "I8", [H, I // 2], H * I // 2), ("w2.scale", "F8_E8M0", [H, I // 32], H * I // 32),
            ("w3.weight", "I8", [I, H // 2], I * H // 2), ("w3.scale", "F8_E8M0", [I, H // 32], I * H // 32)]


def source_arrays(kind: str, rng: np.random.Generator, experts: int, hidden: int, inter: int) -> dict:
    """Per-region uint8 arrays [experts, length] of random MXFP4 experts."""
    H, I = hidden, inter
    if kind == "qwen":
        a = S.mxfp4_experts_np(rng, experts, H, I)
        return {"gate_up.weight": a["gate_up"].view(np.uint8).reshape(experts, -1),
                "gate_up.scale": a["gate_up_scales"].reshape(experts, -1),
                "down.weight": a["down"].view(np.uint8).reshape(experts, -1),
                "down.scale": a["down_scales"].reshape(experts, -1)}
    out = {}
    for name, _, shape, length in regions(kind, H, I):
        if name.endswith(".scale"):
            out[name] = rng.integers(S.SCALE_LOW, S.SCALE_HIGH + 1, size=(experts, length), dtype=np.uint8)
        else:
            out[name] = rng.integers(0, 256, size=(experts, length), dtype=np.uint8)
    return out


def write_install(root: Path, kind: str, layers: int, experts: int, hidden: int, inter: int, seed: int,
                  order=None, extra_files=True):
    """Write manifest.json and experts/layer_XX.bin; ``order`` permutes the regions in the
    blob (default: the reference's order). Returns the source arrays per layer."""
    root = Path(root)
    (root / "experts").mkdir(parents=True, exist_ok=True)
    regs = regions(kind, hidden, inter)
    if order is not None:
        regs = [regs[i] for i in order]
    entries, at = [], 0
    for name, dtype, shape, length in regs:
        entries.append({"name": name, "dtype": dtype, "shape": shape, "offset": at, "length": length})
        at += length
    blob = at
    rng = np.random.default_rng(seed)
    sources, files = [], []
    for layer in range(layers):
        src = source_arrays(kind, rng, experts, hidden, inter)
        data = np.concatenate([src[e["name"]] for e in entries], axis=1)
        path = f"experts/layer_{layer:02d}.bin"
        (root / path).write_bytes(data.tobytes())
        files.append({"path": path, "size": experts * blob})
        sources.append(src)
    if extra_files:   # files outside the expert path are listed and ignored
        (root / "common.bin").write_bytes(b"\0" * 64)
        files.append({"path": "common.bin", "size": 64})
    manifest = {"modelId": kind, "files": files, "expertRegions": entries, "commonTensors": []}
    (root / "manifest.json").write_text(json.dumps(manifest))
    return sources


def slot_blob(kind: str, src: dict, e: int) -> np.ndarray:
    """Expert e's blob in slot order (gate_up | scales | down | scales; DeepSeek w13 = w3 | w1)."""
    names = (("gate_up.weight", "gate_up.scale", "down.weight", "down.scale") if kind == "qwen" else
             ("w3.weight", "w1.weight", "w3.scale", "w1.scale", "w2.weight", "w2.scale"))
    return np.concatenate([src[n][e] for n in names])
