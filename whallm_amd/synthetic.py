"""Synthetic inputs of the benchmark configurations (random-init weights, no checkpoints).

MXFP4 expert weights: E2M1 codes uniform over the 16 values (so packed bytes are
uniform), E8M0 scale exponents uniform in [-8, -2] (bytes 119..125); activations
bf16 N(0, 1); router logits N(0, 1). ``*_np`` builders use numpy's
``default_rng(seed)`` (parity tests compare them against the oracle);
``*_device`` builders fill HBM directly with a seeded torch generator (the
full-size benchmark layers are tens of GB).
"""
from __future__ import annotations

import numpy as np
import torch

from .ops import FP8Experts, MXFP4Experts

SCALE_LOW, SCALE_HIGH = 119, 125  # 2**-8 .. 2**-2


def mxfp4_experts_np(rng: np.random.Generator, experts: int, hidden: int, inter: int) -> dict:
    """Region-major arrays of ``experts`` experts (QwenBatchedExperts layout)."""
    return {
        "gate_up": rng.integers(0, 2**32, size=(experts, 2 * inter, hidden // 8), dtype=np.uint32),
        "gate_up_scales": rng.integers(SCALE_LOW, SCALE_HIGH + 1, size=(experts, 2 * inter, hidden // 32),
                                       dtype=np.uint8),
        "down": rng.integers(0, 2**32, size=(experts, hidden, inter // 8), dtype=np.uint32),
        "down_scales": rng.integers(SCALE_LOW, SCALE_HIGH + 1, size=(experts, hidden, inter // 32), dtype=np.uint8),
    }


def experts_to_device(arrays: dict, device, **kw) -> MXFP4Experts:
    def t(a):
        a = np.ascontiguousarray(a)
        if a.dtype == np.uint32:
            a = a.view(np.int32)
        return torch.from_numpy(a).to(device)

    return MXFP4Experts(t(arrays["gate_up"]), t(arrays["gate_up_scales"]), t(arrays["down"]),
                        t(arrays["down_scales"]), **kw)


def mxfp4_experts_device(experts: int, hidden: int, inter: int, device, generator: torch.Generator) -> MXFP4Experts:
    """Region-major MXFP4 experts generated on the device."""
    def words(*shape):
        return torch.randint(-2**31, 2**31, shape, dtype=torch.int32, device=device, generator=generator)

    def scales(*shape):
        return torch.randint(SCALE_LOW, SCALE_HIGH + 1, shape, dtype=torch.uint8, device=device, generator=generator)

    return MXFP4Experts(words(experts, 2 * inter, hidden // 8), scales(experts, 2 * inter, hidden // 32),
                        words(experts, hidden, inter // 8), scales(experts, hidden, inter // 32))


def bf16_normal_np(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    """bf16 N(0, std) values as uint16 bit patterns (round to nearest even)."""
    v = (rng.standard_normal(shape) * std).astype(np.float32)
    bits = v.view(np.uint32).astype(np.uint64)
    return (((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16) & 0xFFFF).astype(np.uint16)


def bf16_bits_to_tensor(bits: np.ndarray, device) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(device).view(torch.bfloat16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def zipf_bias(experts: int, s: float = 1.1, rng: np.random.Generator | None = None) -> np.ndarray:
    """Per-expert logit bias log(p_e) for a Zipf(s) popularity over a random expert order:
    adding it to N(0,1) logits makes the routed load imbalanced (prefill config)."""
    ranks = np.arange(1, experts + 1, dtype=np.float64)
    p = ranks ** -s
    p /= p.sum()
    bias = np.log(p).astype(np.float32)
    if rng is not None:
        bias = bias[rng.permutation(experts)]
    return bias


E8M0_FP8_LOW, E8M0_FP8_HIGH = 120, 122  # E8M0 block scales 2**-7 .. 2**-5


def fp8_experts_np(rng: np.random.Generator, experts: int, hidden: int, inter: int,
                   scale_low: float = 2.0 ** -7, scale_high: float = 2.0 ** -5, scale_format: int = 0) -> dict:
    """FP8-E4M3 experts as uint8 codes of N(0, 1) clipped to +-448 (round to nearest even,
    via torch's float8_e4m3fn) with fp32 128x128 block scales uniform in [low, high)
    (scale_format 0), or E8M0 32x32 block scale bytes uniform in [120, 122] (scale_format 1,
    the V4.1 release's format)."""
    def codes(*shape):
        v = np.clip(rng.standard_normal(shape).astype(np.float32), -448, 448)
        return torch.from_numpy(v).to(torch.float8_e4m3fn).view(torch.uint8).numpy()

    if scale_format == 1:
        def scales(*shape):
            return rng.integers(E8M0_FP8_LOW, E8M0_FP8_HIGH + 1, size=shape, dtype=np.uint8)
        blk = 32
    else:
        def scales(*shape):
            return rng.uniform(scale_low, scale_high, size=shape).astype(np.float32)
        blk = 128

    return {
        "w13": codes(experts, 2 * inter, hidden), "w13_scales": scales(experts, 2 * inter // blk, hidden // blk),
        "w2": codes(experts, hidden, inter), "w2_scales": scales(experts, hidden // blk, inter // blk),
    }


def fp8_experts_to_device(arrays: dict, device, **kw) -> FP8Experts:
    if arrays["w13_scales"].dtype == np.uint8:
        kw.setdefault("scale_format", 1)
    return FP8Experts(*(torch.from_numpy(np.ascontiguousarray(arrays[n])).to(device)
                        for n in ("w13", "w13_scales", "w2", "w2_scales")), **kw)


def fp8_experts_device(experts: int, hidden: int, inter: int, device, generator: torch.Generator,
                       scale_low: float = 2.0 ** -7, scale_high: float = 2.0 ** -5, scale_format: int = 0) -> FP8Experts:
    """FP8 experts generated on the device (bench sizes), in either scale format."""
    def codes(*shape):
        v = torch.randn(shape, device=device, generator=generator).clamp_(-448, 448)
        return v.to(torch.float8_e4m3fn).view(torch.uint8)

    if scale_format == 1:
        def scales(*shape):
            return torch.randint(E8M0_FP8_LOW, E8M0_FP8_HIGH + 1, shape, dtype=torch.uint8, device=device,
                                 generator=generator)
        blk = 32
    else:
        def scales(*shape):
            return torch.rand(shape, device=device, generator=generator) * (scale_high - scale_low) + scale_low
        blk = 128

    return FP8Experts(codes(experts, 2 * inter, hidden), scales(experts, 2 * inter // blk, hidden // blk),
                      codes(experts, hidden, inter), scales(experts, hidden // blk, inter // blk),
                      scale_format=scale_format)
