"""Torch-facing calls into libwhallm_moe: device tensors in, device tensors out.

Every function requires CUDA (HIP) tensors and enqueues on the current torch
stream; nothing here computes on the CPU or falls back to torch math.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import MXFP4ExpertsC


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _require_device(*tensors: torch.Tensor | None) -> torch.device:
    device = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError("whallm_amd ops take device (HIP) tensors")
        if device is None:
            device = t.device
        elif t.device != device:
            raise ValueError("all tensors must be on one device")
    if device is None:
        raise ValueError("no device tensor given")
    return device


def _contig(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    return t.contiguous()


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)


# ----------------------------------------------------------------------------- expert tables

@dataclass(frozen=True)
class MXFP4Experts:
    """Device regions of a set of MXFP4 experts, addressed as base + slot * stride.

    The four tensors are the reference's Qwen blob regions (manifest.py:37-42):
    gate_up u32 [.., 2I, H/8], gate_up_scales u8 [.., 2I, H/32], down u32
    [.., H, I/8], down_scales u8 [.., H, I/32], with a leading expert/slot axis
    (QwenBatchedExperts, expert_cache.py:70-75) or none for a single expert
    (QwenExpertWeights, :62-67). ``slots`` (int32 [E]) maps expert -> slot when
    the regions are a slot pool rather than a whole layer. ``tiled`` marks regions in the
    prefill tile layout (``prefill_layout``): same shapes and bytes, reordered for the
    grouped GEMM, and accepted by the grouped-GEMM path only.
    """
    gate_up: torch.Tensor
    gate_up_scales: torch.Tensor
    down: torch.Tensor
    down_scales: torch.Tensor
    slots: torch.Tensor | None = None
    experts: int | None = None
    up_first: bool = False
    swiglu_limit: float = 0.0
    tiled: bool = False
    act_terms: str = "e4m3"

    @property
    def hidden(self) -> int:
        return self.gate_up.shape[-1] * 8

    @property
    def inter(self) -> int:
        return self.gate_up.shape[-2] // 2

    @property
    def count(self) -> int:
        if self.experts is not None:
            return self.experts
        return self.gate_up.shape[0] if self.gate_up.dim() == 3 else 1

    def c_struct(self) -> MXFP4ExpertsC:
        # each region's shape and strides read once (this runs on every call of the
        # resident-expert path)
        regions = (self.gate_up, self.gate_up_scales, self.down, self.down_scales)
        shapes = [t.shape for t in regions]
        strides = [t.stride() for t in regions]
        for name, t, shape, st in zip(("gate_up", "gate_up_scales", "down", "down_scales"), regions, shapes, strides):
            if name.endswith("scales"):
                if t.dtype != torch.uint8:
                    raise ValueError(f"{name} must be uint8")
            elif t.dtype not in (torch.int32, torch.uint32):
                raise ValueError(f"{name} must hold 32-bit words, got {t.dtype}")
            if st[-1] != 1 or st[-2] != shape[-1]:
                raise ValueError(f"{name} rows must be contiguous")
        H, I = shapes[0][-1] * 8, shapes[0][-2] // 2
        if shapes[2][-2:] != (H, I // 8) or shapes[1][-2:] != (2 * I, H // 32) or shapes[3][-2:] != (H, I // 32):
            raise ValueError("expert region shapes do not agree")
        # bytes between experts: a leading expert axis, or none for a single expert
        step = [st[0] * (4 if i % 2 == 0 else 1) if len(st) == 3 else 0 for i, st in enumerate(strides)]
        count = self.experts if self.experts is not None else (shapes[0][0] if len(shapes[0]) == 3 else 1)
        return MXFP4ExpertsC(
            regions[0].data_ptr(), regions[1].data_ptr(), regions[2].data_ptr(), regions[3].data_ptr(),
            step[0], step[1], step[2], step[3],
            0 if self.slots is None else self.slots.data_ptr(), count, H, I, int(self.up_first),
            float(self.swiglu_limit), int(self.tiled), _act_terms(self.act_terms))

    def tensors(self):
        return (self.gate_up, self.gate_up_scales, self.down, self.down_scales, self.slots)


def _act_terms(name: str) -> int:
    """The grouped GEMM's activation terms: "e4m3" (two E4M3 terms per 32 values, bf16-exact
    above 2^-13 of the block maximum, the default) or "e2m3" (two E2M3 terms, ~7 significant
    bits of the block maximum, twice the MFMA rate against MXFP4 weights)."""
    if name not in ("e4m3", "e2m3"):
        raise ValueError('act_terms must be "e4m3" or "e2m3"')
    return 0 if name == "e4m3" else 1


def split_rows_e4m3(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 rows [.., H] (H a multiple of 128) -> (uint8 terms [rows, H/128, 256], int32 scales
    [rows, H/128]): the bf16-exact E4M3 term pairs as the prefill GEMMs read activations
    (wm_split_rows_e4m3)."""
    device = _require_device(x)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    rows = x.numel() // H if H else 0
    terms = torch.empty(rows, H // 128, 256, dtype=torch.uint8, device=device)
    scales = torch.empty(rows, H // 128, dtype=torch.int32, device=device)
    _lib.call("wm_split_rows_e4m3", _ptr(x), rows, H, _ptr(terms), _ptr(scales), _stream(device))
    return terms, scales


def split_rows_e2m3(x: torch.Tensor) -> torch.Tensor:
    """bf16 rows [.., H] (H a multiple of 128) -> uint8 [rows, H/128, 208]: the two E2M3 terms
    per 32 values with their E8M0 exponents, as the prefill GEMMs read activations
    (wm_split_rows_e2m3; bytes 200-207 of each step are padding and left unwritten)."""
    device = _require_device(x)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    rows = x.numel() // H if H else 0
    out = torch.empty(rows, H // 128, 208, dtype=torch.uint8, device=device)
    _lib.call("wm_split_rows_e2m3", _ptr(x), rows, H, _ptr(out), _stream(device))
    return out


def prefill_layout(experts):
    """A copy of ``experts`` (MXFP4Experts or FP8Experts) in the prefill tile layout
    (wm_repack_prefill_mxfp4 / wm_repack_prefill_fp8): one expert after another (``slots``
    resolved), each 16-row group's 128-wide K step contiguous (MXFP4: each step's scale
    bytes one run; FP8: block scales unchanged). Same shapes and bytes as the row layout;
    only the grouped-GEMM path (any batch size) takes it. A one-time repack, like the
    reference's install-time blob repack (Sources/DeepSeekRepack/Repacker.swift:17-124)."""
    if experts.tiled:
        return experts
    device = _require_device(*experts.tensors())
    E = experts.count
    fp8 = isinstance(experts, FP8Experts)
    regions = ((experts.w13, experts.w13_scales, experts.w2, experts.w2_scales) if fp8 else
               (experts.gate_up, experts.gate_up_scales, experts.down, experts.down_scales))
    lead = (E,) if regions[0].dim() == 3 or E > 1 else ()
    out = [torch.empty(*lead, *t.shape[-2:], dtype=t.dtype, device=device) for t in regions]
    table = experts.c_struct()
    _lib.call("wm_repack_prefill_fp8" if fp8 else "wm_repack_prefill_mxfp4", ctypes.byref(table),
              *(_ptr(t) for t in out), _stream(device))
    kw = {"scale_format": experts.scale_format} if fp8 else {}
    kw["act_terms"] = experts.act_terms
    cls = FP8Experts if fp8 else MXFP4Experts
    return cls(*out, experts=E if lead else None, up_first=experts.up_first, swiglu_limit=experts.swiglu_limit,
               tiled=True, **kw)


# ----------------------------------------------------------------------------- formats

def dequant_mxfp4(packed: torch.Tensor, scales: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """[.., O, K/8] words + [.., O, K/32] E8M0 -> [.., O, K] (dequant.py:63-68, exact)."""
    device = _require_device(packed, scales)
    if dtype not in (torch.float32, torch.bfloat16):
        raise ValueError("dtype must be float32 or bfloat16")
    packed = packed.contiguous()
    scales = _contig(scales, torch.uint8, "scales")
    cols = packed.shape[-1] * 8
    rows = packed.numel() // packed.shape[-1] if packed.numel() else 0
    if scales.shape[-1] * 32 != cols or scales.numel() != rows * (cols // 32):
        raise ValueError("scales do not match the packed weights")
    out = torch.empty(*packed.shape[:-1], cols, dtype=dtype, device=device)
    _lib.call("wm_dequant_mxfp4", _ptr(packed), _ptr(scales), rows, cols, _ptr(out),
              int(dtype == torch.bfloat16), _stream(device))
    return out


def dequant_fp8_blocks(weight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """FP8 E4M3 [R, C] + fp32 [ceil(R/128), ceil(C/128)] -> fp32 (mimo/weights.py:17-43)."""
    device = _require_device(weight, scales)
    weight = _contig(weight, torch.uint8, "weight")
    scales = _contig(scales, torch.float32, "scales")
    R, C = weight.shape
    if scales.shape != (-(-R // 128), -(-C // 128)):
        raise ValueError("FP8 scale shape does not match 128x128 block padding")
    out = torch.empty(R, C, dtype=torch.float32, device=device)
    _lib.call("wm_dequant_fp8_blocks", _ptr(weight), _ptr(scales), R, C, _ptr(out), _stream(device))
    return out


def dequant_fp8_e8m0(weight: torch.Tensor, scales: torch.Tensor) -> torch.Tensor:
    """FP8 E4M3 [R, C] + E8M0 u8 [ceil(R/32), ceil(C/32)] -> fp32 (deepseek_v41/dequant.py:45-50)."""
    device = _require_device(weight, scales)
    weight = _contig(weight, torch.uint8, "weight")
    scales = _contig(scales, torch.uint8, "scales")
    R, C = weight.shape
    if scales.shape != (-(-R // 32), -(-C // 32)):
        raise ValueError("E8M0 scale shape does not match 32x32 block padding")
    out = torch.empty(R, C, dtype=torch.float32, device=device)
    _lib.call("wm_dequant_fp8_e8m0", _ptr(weight), _ptr(scales), R, C, _ptr(out), _stream(device))
    return out


# ----------------------------------------------------------------------------- routing

def route_softmax_topk(logits: torch.Tensor, k: int, norm_topk_prob: bool = True, probabilities: bool = False):
    """logits [.., E] fp32 -> (indices int32 [.., k], weights fp32 [.., k][, probabilities [.., E]])."""
    device = _require_device(logits)
    logits = _contig(logits, torch.float32, "logits")
    E = logits.shape[-1]
    T = logits.numel() // E if E else 0
    idx = torch.empty(*logits.shape[:-1], k, dtype=torch.int32, device=device)
    w = torch.empty(*logits.shape[:-1], k, dtype=torch.float32, device=device)
    probs = torch.empty_like(logits) if probabilities else None
    _lib.call("wm_route_softmax_topk", _ptr(logits), T, E, k, int(norm_topk_prob), _ptr(idx), _ptr(w), _ptr(probs),
              _stream(device))
    return (idx, w, probs) if probabilities else (idx, w)


SCORE_FUNCS = {"softmax": 0, "sigmoid": 1, "sqrtsoftplus": 2}


def route_scored(logits: torch.Tensor, bias: torch.Tensor | None, k: int, func: str = "sigmoid",
                 route_scale: float = 1.0, norm_topk_prob: bool = True, n_groups: int = 1, topk_groups: int = 1):
    """DeepSeek routing (deepseek_v41/moe.py:58-74, + DeepSeek-V3 group-limited selection)."""
    device = _require_device(logits, bias)
    logits = _contig(logits, torch.float32, "logits")
    if bias is not None:
        bias = _contig(bias, torch.float32, "bias")
    E = logits.shape[-1]
    T = logits.numel() // E if E else 0
    idx = torch.empty(*logits.shape[:-1], k, dtype=torch.int32, device=device)
    w = torch.empty(*logits.shape[:-1], k, dtype=torch.float32, device=device)
    _lib.call("wm_route_scored", _ptr(logits), _ptr(bias), T, E, k, SCORE_FUNCS[func], float(route_scale),
              int(norm_topk_prob), n_groups, topk_groups, _ptr(idx), _ptr(w), _stream(device))
    return idx, w


def linear_bf16(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x [.., H] bf16 @ weight [O, H]^T bf16 -> fp32 [.., O] (the router linear)."""
    device = _require_device(x, weight)
    x = _contig(x, torch.bfloat16, "x")
    weight = _contig(weight, torch.bfloat16, "weight")
    H = x.shape[-1]
    O = weight.shape[0]
    if weight.shape[1] != H:
        raise ValueError("weight does not match x")
    T = x.numel() // H if H else 0
    out = torch.empty(*x.shape[:-1], O, dtype=torch.float32, device=device)
    _lib.call("wm_linear_bf16", _ptr(x), _ptr(weight), T, H, O, _ptr(out), _stream(device))
    return out


# ----------------------------------------------------------------------------- permute

@dataclass
class Permutation:
    order: torch.Tensor
    inverse: torch.Tensor
    offsets: torch.Tensor
    tiles: torch.Tensor
    tile_count: torch.Tensor


def permute(indices: torch.Tensor, experts: int, tile_rows: int = 128) -> Permutation:
    """Stable expert sort of the flattened (token, k) pairs (see wm_permute)."""
    device = _require_device(indices)
    flat = _contig(indices, torch.int32, "indices").reshape(-1)
    P = flat.numel()
    order = torch.empty(P, dtype=torch.int32, device=device)
    inverse = torch.empty(P, dtype=torch.int32, device=device)
    offsets = torch.empty(experts + 1, dtype=torch.int32, device=device)
    max_tiles = -(-P // tile_rows) + experts
    tiles = torch.empty(max_tiles, 2, dtype=torch.int32, device=device)
    count = torch.empty(1, dtype=torch.int32, device=device)
    ws_bytes = _lib.load().wm_permute_workspace_size(P, experts)
    ws = _workspace(ws_bytes, device)
    _lib.call("wm_permute", _ptr(flat), P, experts, tile_rows, _ptr(order), _ptr(inverse), _ptr(offsets),
              _ptr(tiles), _ptr(count), _ptr(ws), ws_bytes, _stream(device))
    return Permutation(order, inverse, offsets, tiles, count)


# ----------------------------------------------------------------------------- expert FFN

def _check_indices(indices: torch.Tensor, experts: int, validate: bool) -> None:
    if validate and indices.numel():
        bad = (indices < 0) | (indices >= experts)
        if bool(bad.any()):
            raise ValueError("expert ID is outside the model")


def moe_mxfp4(x: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor, experts: MXFP4Experts,
              shared: MXFP4Experts | None = None, shared_gate: torch.Tensor | None = None,
              validate: bool = False) -> torch.Tensor:
    """One MoE layer: y = sum_k w_k FFN_k(x) + sigmoid(x . g) FFN_shared(x); bf16 [.., H]."""
    device = _require_device(x, indices, weights, *experts.tensors(), *(shared.tensors() if shared else ()),
                             shared_gate)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    T = x.numel() // H if H else 0
    k = indices.shape[-1]
    idx = _contig(indices, torch.int32, "indices").reshape(T, k)
    w = _contig(weights, torch.float32, "weights").reshape(T, k)
    _check_indices(idx, experts.count, validate)
    sg = None if shared_gate is None else _contig(shared_gate, torch.bfloat16, "shared_gate").reshape(-1)
    table = experts.c_struct()
    sh = shared.c_struct() if shared is not None else None
    ws_bytes = _lib.load().wm_moe_mxfp4_workspace_size(T, k, ctypes.byref(table))
    ws = _workspace(ws_bytes, device)
    y = torch.empty_like(x)
    _lib.call("wm_moe_mxfp4", _ptr(x), T, _ptr(idx), _ptr(w), k, ctypes.byref(table),
              ctypes.byref(sh) if sh is not None else None, _ptr(sg), _ptr(y), _ptr(ws), ws_bytes, _stream(device))
    return y


def _pair_out(out: torch.Tensor | None, x: torch.Tensor, k: int, device) -> torch.Tensor:
    H = x.shape[-1]
    if out is None:
        return torch.empty(*x.shape[:-1], k, H, dtype=torch.bfloat16, device=device)
    if out.dtype != torch.bfloat16 or not out.is_contiguous() or out.numel() != x.numel() * k or out.device != device:
        raise ValueError("out must be a contiguous bf16 tensor of [.., K, H] on the device")
    return out


def experts_mxfp4(x: torch.Tensor, indices: torch.Tensor, experts: MXFP4Experts,
                  validate: bool = False, out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-pair expert outputs in router order: [.., K, H] bf16 (StreamingExperts contract).
    A pair with a negative id leaves its row of ``out`` as it is (a masked pair); an unknown
    or non-resident expert gives a zero row."""
    device = _require_device(x, indices, *experts.tensors(), out)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    T = x.numel() // H if H else 0
    k = indices.shape[-1]
    idx = _contig(indices, torch.int32, "indices").reshape(T, k)
    _check_indices(idx, experts.count, validate)
    table = experts.c_struct()
    ws_bytes = _lib.load().wm_moe_mxfp4_workspace_size(T, k, ctypes.byref(table))
    ws = _workspace(ws_bytes, device)
    out = _pair_out(out, x, k, device)
    _lib.call("wm_experts_mxfp4", _ptr(x), T, _ptr(idx), k, ctypes.byref(table), _ptr(out), _ptr(ws), ws_bytes,
              _stream(device))
    return out


def combine_pairs(rows: torch.Tensor, weights: torch.Tensor, add: torch.Tensor | None = None) -> torch.Tensor:
    """y = sum_k weights[.., k] * rows[.., k, :] (+ add), fp32 in k order, bf16 [.., H]
    (SparseMoE._combine, qwen4_exp.py:1048-1051; _route_reduce, model.py:544-546)."""
    device = _require_device(rows, weights, add)
    rows = _contig(rows, torch.bfloat16, "rows")
    H, k = rows.shape[-1], rows.shape[-2]
    T = rows.numel() // (H * k) if H and k else 0
    w = _contig(weights, torch.float32, "weights")
    if w.numel() != T * k:
        raise ValueError("weights must be [.., K] matching rows")
    a = None if add is None else _contig(add, torch.bfloat16, "add")
    if a is not None and a.numel() != T * H:
        raise ValueError("add must be [.., H] matching rows")
    y = torch.empty(*rows.shape[:-2], H, dtype=torch.bfloat16, device=device)
    _lib.call("wm_combine_pairs", _ptr(rows), _ptr(w), T, k, H, _ptr(a), _ptr(y), _stream(device))
    return y


def mlp_bf16(x: torch.Tensor, gate_w: torch.Tensor, up_w: torch.Tensor, down_w: torch.Tensor,
             gate_vec: torch.Tensor | None = None, add: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """add + sigmoid(x . gate_vec) * down(silu(x gate_w^T) * (x up_w^T)), bf16 [.., H]: the
    reference's bf16 shared expert (qwen4_exp.py:763-771, :1045) on the library's kernels.
    ``out`` may be ``add`` (in place)."""
    device = _require_device(x, gate_w, up_w, down_w, gate_vec, add, out)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    T = x.numel() // H if H else 0
    I = gate_w.shape[0]
    gw, uw, dw = (_contig(t, torch.bfloat16, n) for t, n in ((gate_w, "gate_w"), (up_w, "up_w"), (down_w, "down_w")))
    if gw.shape != (I, H) or uw.shape != (I, H) or dw.shape != (H, I):
        raise ValueError("weights must be gate/up [I, H] and down [H, I]")
    gv = None if gate_vec is None else _contig(gate_vec, torch.bfloat16, "gate_vec").reshape(-1)
    if gv is not None and gv.numel() != H:
        raise ValueError("gate_vec must have H elements")
    a = None if add is None else _contig(add, torch.bfloat16, "add")
    if a is not None and a.numel() != T * H:
        raise ValueError("add must match x")
    y = torch.empty_like(x) if out is None else out
    if y.dtype != torch.bfloat16 or not y.is_contiguous() or y.numel() != T * H:
        raise ValueError("out must be a contiguous bf16 tensor shaped like x")
    ws_bytes = _lib.load().wm_mlp_bf16_workspace_size(T, H, I)
    ws = _workspace(ws_bytes, device)
    _lib.call("wm_mlp_bf16", _ptr(x), T, H, I, _ptr(gw), _ptr(uw), _ptr(dw), _ptr(gv), _ptr(a), _ptr(y), _ptr(ws),
              ws_bytes, _stream(device))
    return y


@dataclass(frozen=True)
class FP8Experts:
    """Device regions of a set of FP8-E4M3 experts, addressed as base + slot * stride.

    w13 uint8 [.., 2I, H] (W1 = gate rows first, then W3 = up; ``up_first`` swaps them) and
    w2 uint8 [.., H, I], with block scales in one of two formats (``scale_format``):
    0, fp32 128x128 blocks (the DeepSeek-V3 / MiMo checkpoints, mimo/weights.py:17-43):
    w13_scales fp32 [.., 2I/128, H/128], w2_scales fp32 [.., H/128, I/128];
    1, one E8M0 byte per 32x32 block (the V4.1 release, deepseek_v41/dequant.py:45-50):
    w13_scales uint8 [.., 2I/32, H/32], w2_scales uint8 [.., H/32, I/32].
    """
    w13: torch.Tensor
    w13_scales: torch.Tensor
    w2: torch.Tensor
    w2_scales: torch.Tensor
    slots: torch.Tensor | None = None
    experts: int | None = None
    up_first: bool = False
    swiglu_limit: float = 0.0
    tiled: bool = False
    scale_format: int = 0
    act_terms: str = "e4m3"

    @property
    def hidden(self) -> int:
        return self.w13.shape[-1]

    @property
    def inter(self) -> int:
        return self.w13.shape[-2] // 2

    @property
    def count(self) -> int:
        if self.experts is not None:
            return self.experts
        return self.w13.shape[0] if self.w13.dim() == 3 else 1

    def c_struct(self) -> _lib.FP8ExpertsC:
        def stride(t: torch.Tensor) -> int:
            return t.stride(0) * t.element_size() if t.dim() == 3 else 0

        if self.scale_format not in (0, 1):
            raise ValueError("scale_format must be 0 (fp32 128x128 blocks) or 1 (E8M0 32x32 blocks)")
        sdt, blk = (torch.float32, 128) if self.scale_format == 0 else (torch.uint8, 32)
        for name, t, dt in (("w13", self.w13, torch.uint8), ("w2", self.w2, torch.uint8),
                            ("w13_scales", self.w13_scales, sdt), ("w2_scales", self.w2_scales, sdt)):
            if t.dtype != dt:
                raise ValueError(f"{name} must be {dt}, got {t.dtype}")
            if t.stride(-1) != 1 or t.stride(-2) != t.shape[-1]:
                raise ValueError(f"{name} rows must be contiguous")
        H, I = self.hidden, self.inter
        if H % 128 or I % 128:
            raise ValueError("FP8 experts need hidden and intermediate multiples of 128")
        if self.w2.shape[-2:] != (H, I) or self.w13_scales.shape[-2:] != (2 * I // blk, H // blk) \
                or self.w2_scales.shape[-2:] != (H // blk, I // blk):
            raise ValueError("FP8 expert region shapes do not agree")
        return _lib.FP8ExpertsC(
            self.w13.data_ptr(), self.w13_scales.data_ptr(), self.w2.data_ptr(), self.w2_scales.data_ptr(),
            stride(self.w13), stride(self.w13_scales), stride(self.w2), stride(self.w2_scales),
            0 if self.slots is None else self.slots.data_ptr(), self.count, H, I, int(self.up_first),
            float(self.swiglu_limit), int(self.tiled), int(self.scale_format), _act_terms(self.act_terms))

    def tensors(self):
        return (self.w13, self.w13_scales, self.w2, self.w2_scales, self.slots)


def moe_fp8(x: torch.Tensor, indices: torch.Tensor, weights: torch.Tensor, experts: FP8Experts,
            shared: FP8Experts | None = None, shared_gate: torch.Tensor | None = None,
            validate: bool = False) -> torch.Tensor:
    """One FP8 MoE layer (DeepSeek form: shared_gate None = ungated shared expert); bf16 [.., H]."""
    device = _require_device(x, indices, weights, *experts.tensors(), *(shared.tensors() if shared else ()),
                             shared_gate)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    T = x.numel() // H if H else 0
    k = indices.shape[-1]
    idx = _contig(indices, torch.int32, "indices").reshape(T, k)
    w = _contig(weights, torch.float32, "weights").reshape(T, k)
    _check_indices(idx, experts.count, validate)
    sg = None if shared_gate is None else _contig(shared_gate, torch.bfloat16, "shared_gate").reshape(-1)
    table = experts.c_struct()
    sh = shared.c_struct() if shared is not None else None
    ws_bytes = _lib.load().wm_moe_fp8_workspace_size(T, k, ctypes.byref(table))
    ws = _workspace(ws_bytes, device)
    y = torch.empty_like(x)
    _lib.call("wm_moe_fp8", _ptr(x), T, _ptr(idx), _ptr(w), k, ctypes.byref(table),
              ctypes.byref(sh) if sh is not None else None, _ptr(sg), _ptr(y), _ptr(ws), ws_bytes, _stream(device))
    return y


def experts_fp8(x: torch.Tensor, indices: torch.Tensor, experts: FP8Experts, validate: bool = False,
                out: torch.Tensor | None = None) -> torch.Tensor:
    """Per-pair FP8 expert outputs in router order: [.., K, H] bf16 (_StreamingSwitchGLU
    contract); masked pairs (negative ids) leave their rows of ``out`` as they are."""
    device = _require_device(x, indices, *experts.tensors(), out)
    x = _contig(x, torch.bfloat16, "x")
    H = x.shape[-1]
    T = x.numel() // H if H else 0
    k = indices.shape[-1]
    idx = _contig(indices, torch.int32, "indices").reshape(T, k)
    _check_indices(idx, experts.count, validate)
    table = experts.c_struct()
    ws_bytes = _lib.load().wm_moe_fp8_workspace_size(T, k, ctypes.byref(table))
    ws = _workspace(ws_bytes, device)
    out = _pair_out(out, x, k, device)
    _lib.call("wm_experts_fp8", _ptr(x), T, _ptr(idx), k, ctypes.byref(table), _ptr(out), _ptr(ws), ws_bytes,
              _stream(device))
    return out


# ----------------------------------------------------------------------------- decode stack

def residual_rmsnorm(residual: torch.Tensor, y: torch.Tensor | None, eps: float = 1e-6) -> torch.Tensor:
    """residual += y (in place), returns bf16 rmsnorm(residual)."""
    device = _require_device(residual, y)
    if residual.dtype != torch.float32 or not residual.is_contiguous():
        raise ValueError("residual must be a contiguous float32 tensor")
    H = residual.shape[-1]
    T = residual.numel() // H if H else 0
    if y is not None:
        y = _contig(y, torch.bfloat16, "y")
    x = torch.empty(residual.shape, dtype=torch.bfloat16, device=device)
    _lib.call("wm_residual_rmsnorm", _ptr(residual), _ptr(y), T, H, float(eps), _ptr(x), _stream(device))
    return x


def repack_router(router: torch.Tensor, shared_gate: torch.Tensor | None = None) -> torch.Tensor:
    """The router rows (+ the shared gate row) in the prefill GEMM's fragment order
    (wm_repack_router): a one-time copy that norm_router(..., router_packed=) reads at 16+
    tokens as contiguous 1 KB fragments."""
    device = _require_device(router, shared_gate)
    router = _contig(router, torch.bfloat16, "router")
    E, H = router.shape
    if shared_gate is not None:
        shared_gate = _contig(shared_gate, torch.bfloat16, "shared_gate").reshape(-1)
        if shared_gate.numel() != H:
            raise ValueError("shared_gate must hold hidden values")
    nbytes = _lib.load().wm_router_packed_bytes(E, H, int(shared_gate is not None))
    if nbytes == 0:
        raise ValueError("the packed router needs hidden a multiple of 32")
    packed = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _lib.call("wm_repack_router", _ptr(router), _ptr(shared_gate), E, H, _ptr(packed), _stream(device))
    return packed


def norm_router(residual: torch.Tensor, y: torch.Tensor | None, router: torch.Tensor,
                shared_gate: torch.Tensor | None = None, norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                residual_out: torch.Tensor | None = None, router_packed: torch.Tensor | None = None):
    """One launch (wm_norm_router): v = residual + y, x = bf16(rmsnorm(v) * norm_weight),
    router logits = x @ router^T (fp32) and the shared gate logit x @ shared_gate (fp32, or
    None). Returns (x, logits, shared_logit); ``residual_out`` (a separate fp32 buffer)
    receives v. The residual itself is not written (other blocks still read it).
    ``router_packed`` (repack_router of the same router and gate) speeds up 16+ tokens."""
    device = _require_device(residual, y, router, shared_gate, norm_weight, residual_out, router_packed)
    if residual.dtype != torch.float32 or not residual.is_contiguous():
        raise ValueError("residual must be a contiguous float32 tensor")
    H = residual.shape[-1]
    T = residual.numel() // H if H else 0
    y = None if y is None else _contig(y, torch.bfloat16, "y")
    router = _contig(router, torch.bfloat16, "router")
    if y is not None and y.shape != residual.shape:
        raise ValueError("y must match residual")
    if router.dim() != 2 or router.shape[1] != H:
        raise ValueError("router must be [experts, hidden]")
    if shared_gate is not None:
        shared_gate = _contig(shared_gate, torch.bfloat16, "shared_gate").reshape(-1)
        if shared_gate.numel() != H:
            raise ValueError("shared_gate must hold hidden values")
    if norm_weight is not None:
        norm_weight = _contig(norm_weight, torch.bfloat16, "norm_weight").reshape(-1)
        if norm_weight.numel() != H:
            raise ValueError("norm_weight must hold hidden values")
    if residual_out is not None and (residual_out.dtype != torch.float32 or residual_out.shape != residual.shape
                                     or not residual_out.is_contiguous()):
        raise ValueError("residual_out must be a contiguous float32 tensor shaped like residual")
    E = router.shape[0]
    x = torch.empty(residual.shape, dtype=torch.bfloat16, device=device)
    logits = torch.empty(*residual.shape[:-1], E, dtype=torch.float32, device=device)
    shared_logit = (torch.empty(residual.shape[:-1], dtype=torch.float32, device=device)
                    if shared_gate is not None else None)
    packed_bytes = 0 if router_packed is None else router_packed.numel() * router_packed.element_size()
    _lib.call("wm_norm_router", _ptr(residual), _ptr(y), _ptr(norm_weight), T, H, float(eps), _ptr(router), E,
              _ptr(shared_gate), _ptr(router_packed), packed_bytes, _ptr(x), _ptr(residual_out), _ptr(logits),
              _ptr(shared_logit), _stream(device))
    return x, logits, shared_logit


class MoEStack:
    """L chained MXFP4 MoE layers run by one wm_moe_stack_mxfp4 call (device routing,
    no host synchronisation, graph-capturable). Holds the C tables of every layer."""

    def __init__(self, layers: list[MXFP4Experts], shared: list[MXFP4Experts] | None = None,
                 shared_gates: list[torch.Tensor] | None = None, k: int = 10, norm_topk_prob: bool = True,
                 eps: float = 1e-6):
        self.layers, self.shared, self.shared_gates = layers, shared, shared_gates
        self.k, self.norm, self.eps = k, norm_topk_prob, eps
        n = len(layers)
        self._tables = (MXFP4ExpertsC * n)(*[e.c_struct() for e in layers])
        self._shared = (MXFP4ExpertsC * n)(*[e.c_struct() for e in shared]) if shared else None
        self._gates = (ctypes.c_void_p * n)(*[g.data_ptr() for g in shared_gates]) if shared_gates else None
        self.device = layers[0].gate_up.device
        self._ws = None

    def workspace_bytes(self, tokens: int) -> int:
        return _lib.load().wm_moe_stack_mxfp4_workspace_size(tokens, self.k, ctypes.byref(self._tables[0]))

    def __call__(self, logits: torch.Tensor, residual: torch.Tensor, x_out: torch.Tensor | None = None,
                 cancel=None):
        """logits fp32 [L, T, E]; residual fp32 [T, H] updated in place; x_out bf16 [T, H] (optional).

        ``cancel`` (optional) is a callable polled before each layer is enqueued, like the
        reference's cancel callback (Native/QwenNative/capi.h:36-37): when it returns true the
        call raises ``Cancelled`` (status 2); the layers enqueued before it still run, so the
        caller restores the residual."""
        _require_device(logits, residual, x_out)
        L = len(self.layers)
        T = residual.shape[0]
        if logits.shape[0] != L or logits.shape[1] != T or logits.dtype != torch.float32 or not logits.is_contiguous():
            raise ValueError("logits must be contiguous float32 [layers, tokens, experts]")
        need = self.workspace_bytes(T)
        if self._ws is None or self._ws.numel() < need:
            self._ws = _workspace(need, self.device)
        hook = None if cancel is None else _lib.CANCEL_FN(lambda _ctx: 1 if cancel() else 0)
        _lib.call("wm_moe_stack_mxfp4", _ptr(logits), L, T, self.k, int(self.norm), self._tables, self._shared,
                  self._gates, _ptr(residual), float(self.eps), _ptr(x_out), _ptr(self._ws), self._ws.numel(),
                  hook, None, _stream(self.device))
        return residual


# ----------------------------------------------------------------------------- persistent decode

def repack_down_slices(experts: MXFP4Experts) -> tuple[torch.Tensor, torch.Tensor]:
    """Down regions of every expert in the slice-major layout of the persistent decode
    kernel: words [E, 8, H, I/64] int32 and scales [E, 8, H, I/256] uint8."""
    device = _require_device(*experts.tensors())
    E, H, I = experts.count, experts.hidden, experts.inter
    down = experts.down if experts.down.dim() == 3 else experts.down.unsqueeze(0)
    scales = experts.down_scales if experts.down_scales.dim() == 3 else experts.down_scales.unsqueeze(0)
    dst = torch.empty(E, 8, H, I // 64, dtype=torch.int32, device=device)
    dst_s = torch.empty(E, 8, H, I // 256, dtype=torch.uint8, device=device)
    _lib.call("wm_repack_down_slices", _ptr(down), _ptr(scales), down.stride(0) * 4, scales.stride(0), E, H, I,
              _ptr(dst), _ptr(dst_s), _stream(device))
    return dst, dst_s


class DecodeStackError(_lib.WhallmError):
    """A persistent decode launch ended early (its status word was nonzero)."""


class DecodeLayer:
    """One MoE decode layer for one token in one call (wm_moe_layer_decode): the pre-norm,
    the router GEMV and softmax top-k, the routed and shared experts and the residual add,
    as a decoder layer calls its MoE half between attention blocks (qwen4_exp.py:1146).
    Holds the call's state buffer on the device (zero-filled; reused by calls in stream
    order). Shapes with a fused kernel run as one launch; others as the per-layer kernels."""

    STATUS_TEXT = {1: "a grid-wide wait ran out", 4: "no valid route (fewer than k selectable logits)"}

    def __init__(self, experts: MXFP4Experts, router: torch.Tensor, shared: MXFP4Experts | None = None,
                 shared_gate: torch.Tensor | None = None, k: int = 10, norm_weight: torch.Tensor | None = None,
                 eps: float = 1e-6, norm_topk_prob: bool = True):
        self.device = experts.gate_up.device
        self.experts, self.shared, self.k, self.eps, self.norm_topk = experts, shared, k, eps, norm_topk_prob
        self.E, self.H, self.I = experts.count, experts.hidden, experts.inter
        self.router = _contig(router, torch.bfloat16, "router")
        if self.router.shape != (self.E, self.H):
            raise ValueError("router must be [experts, hidden]")
        self.shared_gate = None if shared_gate is None else _contig(shared_gate, torch.bfloat16, "shared_gate")
        self.norm_weight = None if norm_weight is None else _contig(norm_weight, torch.bfloat16, "norm_weight")
        self._table = experts.c_struct()
        self._shared = shared.c_struct() if shared is not None else None
        lib = _lib.load()
        self.state = torch.zeros(lib.wm_moe_layer_decode_state_size(self.E, self.H, self.I, k), dtype=torch.uint8,
                                 device=self.device)
        self.status_offset = lib.wm_moe_layer_decode_status_offset(self.E, self.I)

    def __call__(self, residual: torch.Tensor, residual_out: torch.Tensor | None = None, y: torch.Tensor | None = None,
                 x_out: torch.Tensor | None = None, logits_out: torch.Tensor | None = None,
                 indices_out: torch.Tensor | None = None, weights_out: torch.Tensor | None = None):
        """residual fp32 [H] -> residual_out (default: residual, updated in place) = residual +
        bf16(y); the optional outputs receive y, x, the logits and the routes."""
        if residual.dtype != torch.float32 or not residual.is_contiguous() or residual.numel() != self.H:
            raise ValueError("residual must be a contiguous float32 [hidden] tensor")
        if residual_out is None:
            residual_out = residual
        _lib.call("wm_moe_layer_decode", _ptr(residual), _ptr(residual_out), _ptr(self.norm_weight), float(self.eps),
                  _ptr(self.router), _ptr(self.shared_gate), self.E, self.k, int(self.norm_topk),
                  ctypes.byref(self._table), ctypes.byref(self._shared) if self._shared is not None else None,
                  _ptr(y), _ptr(x_out), _ptr(logits_out), _ptr(indices_out), _ptr(weights_out), _ptr(self.state),
                  self.state.numel(), _stream(self.device))
        return residual_out

    def status(self) -> int:
        """0 done, 1 a grid-wide wait ran out, 4 no valid route; nonzero needs reset(). Synchronises."""
        return int(self.state[self.status_offset:self.status_offset + 4].view(torch.int32).item())

    def raise_for_status(self) -> None:
        st = self.status()
        if st != 0:
            self.reset()
            raise DecodeStackError(f"decode layer: {self.STATUS_TEXT.get(st, f'status {st}')}")

    def reset(self):
        self.state.zero_()


class PersistentDecodeStack:
    """One-token decode through L MXFP4 MoE layers in one persistent kernel launch
    (wm_moe_decode_persistent_mxfp4); keeps the per-layer descriptor table and the message
    state on the device.

    ``down_layout``: "slices" repacks every layer's down regions slice-major once (the
    fastest reads; the tables must not change afterwards), "rows" reads them in place in
    the reference row layout. Tables with a slot map (a slot cache's ``table(file)``,
    whose slots are refilled over time) are always read in place.
    """

    # status word values (wm_moe_decode_persistent_mxfp4)
    STATUS_TEXT = {1: "a message wait ran out", 2: "cancelled", 3: "a selected expert is not resident",
                   4: "no valid route (a logits row has fewer than k selectable values)"}

    def __init__(self, layers: list[MXFP4Experts], shared: list[MXFP4Experts],
                 shared_gates: list[torch.Tensor] | None = None, k: int = 10, eps: float = 1e-6,
                 down_layout: str = "slices"):
        if not layers or len(shared) != len(layers):
            raise ValueError("one shared expert per layer is required")
        if down_layout not in ("slices", "rows"):
            raise ValueError("down_layout must be 'slices' or 'rows'")
        if any(e.slots is not None for e in layers):
            down_layout = "rows"  # a private copy would go stale when the slots are refilled
        self.down_layout = down_layout
        self.device = layers[0].gate_up.device
        self.k, self.eps = k, eps
        self.L, self.E = len(layers), layers[0].count
        self.H, self.I = layers[0].hidden, layers[0].inter
        self.layers, self.shared, self.shared_gates = layers, shared, shared_gates
        self._keep = []
        descs = []
        for l, (e, s) in enumerate(zip(layers, shared)):
            if e.hidden != self.H or e.inter != self.I or e.count != self.E or s.hidden != self.H or s.inter != self.I:
                raise ValueError("layers differ in shape")
            if e.gate_up.dim() != 3:
                raise ValueError("routed experts need a leading expert axis")
            if s.slots is not None:
                raise ValueError("the shared expert must be resident (no slot map)")
            if down_layout == "slices":
                d, ds = repack_down_slices(e)
                sd, sds = repack_down_slices(s)
                self._keep += [d, ds, sd, sds]
                down = (d.data_ptr(), ds.data_ptr(), d.stride(0) * 4, ds.stride(0))
                sdown = (sd.data_ptr(), sds.data_ptr())
            else:
                down = (e.down.data_ptr(), e.down_scales.data_ptr(), e.down.stride(0) * 4, e.down_scales.stride(0))
                sdown = (s.down.data_ptr(), s.down_scales.data_ptr())
            g = shared_gates[l] if shared_gates is not None else None
            if g is not None and (g.dtype != torch.bfloat16 or g.numel() != self.H):
                raise ValueError("shared gate must be bf16 [H]")
            descs.append(_lib.DecodeLayerC(
                e.gate_up.data_ptr(), e.gate_up_scales.data_ptr(), down[0], down[1],
                e.gate_up.stride(0) * 4, e.gate_up_scales.stride(0), down[2], down[3],
                0 if e.slots is None else e.slots.data_ptr(),
                s.gate_up.data_ptr(), s.gate_up_scales.data_ptr(), sdown[0], sdown[1],
                0 if g is None else g.data_ptr()))
        table = (_lib.DecodeLayerC * self.L)(*descs)
        raw = bytes(table)
        self.table = torch.frombuffer(bytearray(raw), dtype=torch.uint8).to(self.device)
        lib = _lib.load()
        self.state = torch.zeros(lib.wm_decode_state_size(self.L, self.E), dtype=torch.uint8, device=self.device)
        self.status_offset = lib.wm_decode_status_offset(self.L, self.E)

    def __call__(self, logits: torch.Tensor, residual: torch.Tensor, x_out: torch.Tensor | None = None,
                 check: bool = True, cancel: torch.Tensor | None = None, trace: torch.Tensor | None = None):
        """logits fp32 [L, E] (or [L, 1, E]); residual fp32 [H] (or [1, H]) updated in place.

        With ``check`` the call waits for the launch and raises ``DecodeStackError`` (or
        ``Cancelled``) when it ended early, after resetting the state; residual and x_out are
        then unchanged. ``check=False`` leaves the launch running: read ``status()`` later.
        ``cancel``: an int32 tensor (pinned host memory or on the device) the caller may set
        nonzero while the launch runs; the launch stops after the layer that reads it.
        ``trace``: fp32 [L, H] on the device, receives the residual after every layer."""
        _require_device(logits, residual, x_out)
        if logits.dtype != torch.float32 or not logits.is_contiguous() or logits.numel() != self.L * self.E:
            raise ValueError("logits must be contiguous float32 [layers, experts]")
        if residual.dtype != torch.float32 or not residual.is_contiguous() or residual.numel() != self.H:
            raise ValueError("residual must be contiguous float32 [hidden] (one token)")
        if cancel is not None and (cancel.dtype != torch.int32 or cancel.numel() < 1
                                   or not (cancel.is_cuda or cancel.is_pinned())):
            raise ValueError("cancel must be an int32 tensor on the device or in pinned host memory")
        if trace is not None and (trace.dtype != torch.float32 or not trace.is_contiguous()
                                  or trace.numel() != self.L * self.H or trace.device != self.device):
            raise ValueError("trace must be a contiguous float32 [layers, hidden] device tensor")
        _lib.call("wm_moe_decode_persistent_mxfp4", _ptr(logits), self.L, self.E, self.k, self.H, self.I,
                  _ptr(self.table), _ptr(residual), float(self.eps), _ptr(x_out), _ptr(self.state),
                  self.state.numel(), 1 if self.down_layout == "rows" else 0, _ptr(cancel), _ptr(trace),
                  _stream(self.device))
        if check:
            self.raise_for_status()
        return residual

    def status(self) -> int:
        """The launch's outcome: 0 done, 1 a message wait ran out, 2 cancelled, 3 a selected
        expert is not resident, 4 no valid route. Nonzero needs reset() before the next launch.
        Synchronises."""
        return int(self.state[self.status_offset:self.status_offset + 4].view(torch.int32).item())

    def raise_for_status(self) -> None:
        """Raises (after reset()) when the last launch ended early."""
        st = self.status()
        if st != 0:
            self.reset()
            kind = _lib.Cancelled if st == 2 else DecodeStackError
            raise kind(f"persistent decode: {self.STATUS_TEXT.get(st, f'status {st}')}")

    def reset(self):
        self.state.zero_()

    def xcd_local(self) -> bool:
        """Whether the device places block b of the launch on XCC b % 8, so that
        messages read within one XCD use XCD-local stores (checked once per device)."""
        lib = _lib.load()
        r = lib.wm_decode_xcd_local(_stream(self.device))
        if r < 0:
            raise _lib.WhallmError(f"wm_decode_xcd_local: {lib.wm_last_error().decode(errors='replace')}")
        return bool(r)


# ----------------------------------------------------------------------------- MTP acceptance

def _mtp_rows(t: torch.Tensor, name: str) -> tuple[torch.Tensor, int, int]:
    t = _contig(t, torch.float32, name)
    if t.dim() != 2:
        raise ValueError(f"{name} must be [rows, vocab]")
    return t, t.shape[0], t.shape[1]


def mtp_verify_greedy(target_logits: torch.Tensor, drafts: torch.Tensor) -> torch.Tensor:
    """Greedy MTP acceptance (Sampler.verify at temperature 0, native_qwen.py:395-400).

    target_logits fp32 [n + 1, V], drafts int32 [n] -> device int32 [2] =
    (accepted drafts, next token). Enqueued; no host synchronisation."""
    device = _require_device(target_logits, drafts)
    target_logits, rows, vocab = _mtp_rows(target_logits, "target_logits")
    drafts = _contig(drafts.reshape(-1), torch.int32, "drafts")
    n = drafts.numel()
    if rows != n + 1:
        raise ValueError("target_logits needs one row per draft plus the bonus row")
    out = torch.empty(2, dtype=torch.int32, device=device)
    ws = _workspace(_lib.load().wm_mtp_workspace_size(n, vocab), device)
    _lib.call("wm_mtp_verify_greedy", _ptr(target_logits), _ptr(drafts), n, vocab, _ptr(out), _ptr(ws), ws.numel(),
              _stream(device))
    return out


def mtp_verify_rejection(target_logp: torch.Tensor, draft_logp: torch.Tensor, drafts: torch.Tensor,
                         uniforms: torch.Tensor) -> torch.Tensor:
    """Rejection-sampling MTP acceptance (native_qwen.py:401-408, dspark.py:875-898).

    target_logp fp32 [n + 1, V], draft_logp fp32 [n, V] (log-probabilities), drafts
    int32 [n], uniforms fp32 [n + 1] (u_0..u_{n-1} accept tests, u_n the sampling draw)
    -> device int32 [2] = (accepted drafts, next token)."""
    device = _require_device(target_logp, draft_logp, drafts, uniforms)
    target_logp, rows, vocab = _mtp_rows(target_logp, "target_logp")
    drafts = _contig(drafts.reshape(-1), torch.int32, "drafts")
    n = drafts.numel()
    if rows != n + 1:
        raise ValueError("target_logp needs one row per draft plus the bonus row")
    if n > 0:
        draft_logp, drows, dvocab = _mtp_rows(draft_logp, "draft_logp")
        if drows != n or dvocab != vocab:
            raise ValueError("draft_logp must be [n, vocab]")
    else:
        draft_logp = None
    uniforms = _contig(uniforms.reshape(-1), torch.float32, "uniforms")
    if uniforms.numel() != n + 1:
        raise ValueError("uniforms must hold n + 1 draws")
    out = torch.empty(2, dtype=torch.int32, device=device)
    ws = _workspace(_lib.load().wm_mtp_workspace_size(n, vocab), device)
    _lib.call("wm_mtp_verify_rejection", _ptr(target_logp), _ptr(draft_logp), _ptr(drafts), n, vocab, _ptr(uniforms),
              _ptr(out), _ptr(ws), ws.numel(), _stream(device))
    return out
