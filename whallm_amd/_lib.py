"""ctypes binding of libwhallm_moe.so (the C ABI declared in include/whallm_moe.h).

The library is loaded from the package's own ``lib/`` folder. There is no
fallback: when it is missing or fails to load, every operation raises.
"""
from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_int32, c_int64, c_size_t, c_void_p, c_char_p, POINTER
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libwhallm_moe.so"


class MXFP4ExpertsC(ctypes.Structure):
    """wm_mxfp4_experts (include/whallm_moe.h)."""
    _fields_ = [
        ("gate_up", c_void_p), ("gate_up_scales", c_void_p), ("down", c_void_p), ("down_scales", c_void_p),
        ("gate_up_stride", c_int64), ("gate_up_scales_stride", c_int64),
        ("down_stride", c_int64), ("down_scales_stride", c_int64),
        ("slots", c_void_p), ("experts", c_int32), ("hidden", c_int32), ("inter", c_int32),
        ("up_first", c_int32), ("swiglu_limit", c_float), ("tiled", c_int32), ("act_terms", c_int32),
    ]


class FP8ExpertsC(ctypes.Structure):
    """wm_fp8_experts (include/whallm_moe.h)."""
    _fields_ = [
        ("w13", c_void_p), ("w13_scales", c_void_p), ("w2", c_void_p), ("w2_scales", c_void_p),
        ("w13_stride", c_int64), ("w13_scales_stride", c_int64), ("w2_stride", c_int64), ("w2_scales_stride", c_int64),
        ("slots", c_void_p), ("experts", c_int32), ("hidden", c_int32), ("inter", c_int32),
        ("up_first", c_int32), ("swiglu_limit", c_float), ("tiled", c_int32), ("scale_format", c_int32),
        ("act_terms", c_int32),
    ]


class DecodeLayerC(ctypes.Structure):
    """wm_decode_layer (include/whallm_moe.h)."""
    _fields_ = [
        ("gate_up", c_void_p), ("gate_up_scales", c_void_p), ("down", c_void_p), ("down_scales", c_void_p),
        ("gate_up_stride", c_int64), ("gate_up_scales_stride", c_int64),
        ("down_stride", c_int64), ("down_scales_stride", c_int64),
        ("slots", c_void_p),
        ("shared_gate_up", c_void_p), ("shared_gate_up_scales", c_void_p),
        ("shared_down", c_void_p), ("shared_down_scales", c_void_p), ("shared_gate", c_void_p),
    ]


_P = c_void_p
_SIGNATURES = {
    "wm_last_error": (c_char_p, []),
    "wm_version": (c_char_p, []),
    "wm_dequant_mxfp4": (c_int, [_P, _P, c_int64, c_int64, _P, c_int, _P]),
    "wm_dequant_fp8_blocks": (c_int, [_P, _P, c_int64, c_int64, _P, _P]),
    "wm_dequant_fp8_e8m0": (c_int, [_P, _P, c_int64, c_int64, _P, _P]),
    "wm_route_softmax_topk": (c_int, [_P, c_int32, c_int32, c_int32, c_int32, _P, _P, _P, _P]),
    "wm_route_scored": (c_int, [_P, _P, c_int32, c_int32, c_int32, c_int32, c_float, c_int32, c_int32, c_int32,
                                _P, _P, _P]),
    "wm_linear_bf16": (c_int, [_P, _P, c_int32, c_int32, c_int32, _P, _P]),
    "wm_permute_workspace_size": (c_size_t, [c_int64, c_int32]),
    "wm_permute": (c_int, [_P, c_int64, c_int32, c_int32, _P, _P, _P, _P, _P, _P, c_size_t, _P]),
    "wm_moe_mxfp4_workspace_size": (c_size_t, [c_int32, c_int32, POINTER(MXFP4ExpertsC)]),
    "wm_moe_mxfp4": (c_int, [_P, c_int32, _P, _P, c_int32, POINTER(MXFP4ExpertsC), POINTER(MXFP4ExpertsC), _P,
                             _P, _P, c_size_t, _P]),
    "wm_experts_mxfp4": (c_int, [_P, c_int32, _P, c_int32, POINTER(MXFP4ExpertsC), _P, _P, c_size_t, _P]),
    "wm_moe_mxfp4_noalloc_max_bytes": (c_size_t, []),
    "wm_moe_mxfp4_noalloc": (c_int, [_P, c_int32, _P, _P, c_int32, POINTER(MXFP4ExpertsC), POINTER(MXFP4ExpertsC), _P,
                                     _P, _P]),
    "wm_repack_prefill_mxfp4": (c_int, [POINTER(MXFP4ExpertsC), _P, _P, _P, _P, _P]),
    "wm_combine_pairs": (c_int, [_P, _P, c_int32, c_int32, c_int32, _P, _P, _P]),
    "wm_mlp_bf16_workspace_size": (c_size_t, [c_int32, c_int32, c_int32]),
    "wm_mlp_bf16": (c_int, [_P, c_int32, c_int32, c_int32, _P, _P, _P, _P, _P, _P, _P, c_size_t, _P]),
    "wm_repack_prefill_fp8": (c_int, [POINTER(FP8ExpertsC), _P, _P, _P, _P, _P]),
    "wm_residual_rmsnorm": (c_int, [_P, _P, c_int32, c_int32, c_float, _P, _P]),
    "wm_norm_router": (c_int, [_P, _P, _P, c_int32, c_int32, c_float, _P, c_int32, _P, _P, c_size_t, _P, _P, _P, _P,
                               _P]),
    "wm_router_packed_bytes": (c_size_t, [c_int32, c_int32, c_int32]),
    "wm_repack_router": (c_int, [_P, _P, c_int32, c_int32, _P, _P]),
    "wm_moe_stack_mxfp4_workspace_size": (c_size_t, [c_int32, c_int32, POINTER(MXFP4ExpertsC)]),
    "wm_moe_stack_mxfp4": (c_int, [_P, c_int32, c_int32, c_int32, c_int32, POINTER(MXFP4ExpertsC),
                                   POINTER(MXFP4ExpertsC), _P, _P, c_float, _P, _P, c_size_t, _P, _P, _P]),
    "wm_repack_down_slices": (c_int, [_P, _P, c_int64, c_int64, c_int32, c_int32, c_int32, _P, _P, _P]),
    "wm_decode_state_size": (c_size_t, [c_int32, c_int32]),
    "wm_decode_status_offset": (c_size_t, [c_int32, c_int32]),
    "wm_moe_layer_decode_state_size": (c_size_t, [c_int32, c_int32, c_int32, c_int32]),
    "wm_moe_layer_decode_status_offset": (c_size_t, [c_int32, c_int32]),
    "wm_moe_layer_decode": (c_int, [_P, _P, _P, c_float, _P, _P, c_int32, c_int32, c_int32, POINTER(MXFP4ExpertsC),
                                    POINTER(MXFP4ExpertsC), _P, _P, _P, _P, _P, _P, c_size_t, _P]),
    "wm_decode_xcd_local": (c_int, [_P]),
    "wm_slot_cache_open": (c_void_p, [c_int32, c_int64, c_int32, c_int32, _P, _P, _P, c_char_p, c_size_t]),
    "wm_slot_cache_close": (None, [_P]),
    "wm_slot_cache_error": (c_char_p, [_P]),
    "wm_slot_cache_plan": (c_int, [_P, c_int32, _P, c_int32, _P, _P]),
    "wm_slot_cache_acquire": (c_int, [_P, c_int32, _P, c_int32, _P, _P]),
    "wm_slot_cache_stats": (c_int, [_P, _P]),
    "wm_slot_cache_acquire_ready": (c_int, [_P, c_int32, _P, c_int32, _P, _P, _P]),
    "wm_slot_cache_acquire_split": (c_int, [_P, c_int32, _P, c_int32, _P, _P, _P, c_int64, _P, _P, _P]),
    "wm_slot_cache_acquire_files": (c_int, [_P, c_int32, _P, _P, _P, _P, _P]),
    "wm_slot_cache_read_experts": (c_int, [_P, c_int32, _P, c_int32, _P, _P]),
    "wm_slot_cache_seed_tail": (c_int, [_P, c_int32, _P, c_int64, c_int32, c_int32, _P, _P, _P, _P, _P]),
    "wm_slot_cache_route_policy": (c_int, [_P, c_int32]),
    "wm_slot_cache_route_observe": (c_int, [_P, c_int32, _P, c_int64, c_int32]),
    "wm_slot_cache_route_phase": (c_int, [_P, c_int32]),
    "wm_slot_cache_route_begin_request": (c_int, [_P]),
    "wm_slot_cache_route_record_read": (c_int, [_P, c_int32, ctypes.c_double]),
    "wm_slot_cache_route_rebalance": (c_int, [_P]),
    "wm_slot_cache_route_state": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P]),
    "wm_slot_cache_start_fills": (c_int, [_P]),
    "wm_slot_cache_wait_fills": (c_int, [_P, _P]),
    "wm_slot_cache_set_route": (c_int, [_P, _P, _P]),
    "wm_slot_cache_read_layer": (c_int, [_P, c_int32, _P, _P]),
    "wm_slot_cache_wait_layer": (c_int, [_P, c_int32, _P]),
    "wm_slot_cache_seed": (c_int, [_P, c_int32, _P, _P, c_int32, _P, _P, _P]),
    "wm_moe_fp8_workspace_size": (c_size_t, [c_int32, c_int32, POINTER(FP8ExpertsC)]),
    "wm_moe_fp8": (c_int, [_P, c_int32, _P, _P, c_int32, POINTER(FP8ExpertsC), POINTER(FP8ExpertsC), _P, _P, _P,
                           c_size_t, _P]),
    "wm_experts_fp8": (c_int, [_P, c_int32, _P, c_int32, POINTER(FP8ExpertsC), _P, _P, c_size_t, _P]),
    "wm_mtp_workspace_size": (c_size_t, [c_int32, c_int32]),
    "wm_mtp_verify_greedy": (c_int, [_P, _P, c_int32, c_int32, _P, _P, c_size_t, _P]),
    "wm_verify_step_fp8_workspace_size": (c_size_t, [c_int32, c_int32, c_int32, _P]),
    "wm_verify_step_fp8": (c_int, [c_int32, _P, _P, c_int32, _P, _P, _P, c_int32, c_int32, c_float, c_int32, c_int32,
                                   c_float, _P, c_int32, _P, _P, _P, _P, c_size_t, _P]),
    "wm_mtp_verify_rejection": (c_int, [_P, _P, _P, c_int32, c_int32, _P, _P, _P, c_size_t, _P]),
    "wm_split_rows_e2m3": (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p]),
    "wm_split_rows_e4m3": (c_int, [c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "wm_set_kernel_timing": (c_int, [c_int]),
    "wm_kernel_timing_ms": (c_int, [_P]),
    "wm_moe_decode_persistent_mxfp4": (c_int, [_P, c_int32, c_int32, c_int32, c_int32, c_int32, _P, _P, c_float,
                                               _P, _P, c_size_t, c_int32, _P, _P, _P]),
}

_lib = None


class WhallmError(RuntimeError):
    """A libwhallm_moe call returned a nonzero status."""


class Cancelled(WhallmError):
    """A call stopped by its cancel hook (status 2, Native/QwenNative/capi.h:1-5); the
    state it carried (a residual, a decode state) must be reset before reuse."""


# The reference's cancel callback type (wq_cancel_fn, Native/QwenNative/capi.h:36-37).
CANCEL_FN = ctypes.CFUNCTYPE(c_int, c_void_p)


def load() -> ctypes.CDLL:
    """The loaded library; raises when it is not built or cannot load."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m whallm_amd.build` "
            "(there is no CPU fallback for the expert path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (restype, argtypes) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def call(name: str, *args) -> None:
    """Calls an int-status entry point, raising WhallmError with wm_last_error()."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status != 0:
        kind = Cancelled if status == 2 else WhallmError
        raise kind(f"{name}: {lib.wm_last_error().decode(errors='replace')}")


def exported_symbols() -> list[str]:
    return sorted(_SIGNATURES)
