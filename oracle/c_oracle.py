"""Build and load the C restatement (oracle/c/oracle.c) — test infrastructure only."""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SOURCE = HERE / "c" / "oracle.c"
LIB = HERE / "c" / "liboracle.so"


def build(force: bool = False) -> Path:
    if force or not LIB.exists() or LIB.stat().st_mtime < SOURCE.stat().st_mtime:
        subprocess.run(["gcc", "-O2", "-std=c11", "-fPIC", "-shared", "-ffp-contract=off", str(SOURCE), "-lm",
                        "-o", str(LIB)], check=True)
    return LIB


_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        lib = ctypes.CDLL(str(build()))
        P = ctypes.c_void_p
        i64 = ctypes.c_int64
        lib.wm_oracle_quantize_bf16.argtypes = [P, i64, i64, P, P]
        lib.wm_oracle_quantize_fp8.argtypes = [P, P, i64, i64, P, P]
        lib.wm_oracle_dequant_mxfp4.argtypes = [P, P, i64, i64, P]
        lib.wm_oracle_topk.argtypes = [P, i64, i64, i64, P]
        lib.wm_oracle_e4m3.argtypes = [ctypes.c_uint8]
        lib.wm_oracle_e4m3.restype = ctypes.c_float
        lib.wm_oracle_ffn.argtypes = [P, i64, i64, i64, P, P, P, P]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def quantize_bf16(bits: np.ndarray, rows: int, cols: int):
    src = np.ascontiguousarray(bits, np.uint16)
    w = np.zeros(rows * cols // 2, np.uint8)
    s = np.zeros(rows * cols // 32, np.uint8)
    if load().wm_oracle_quantize_bf16(_p(src), rows, cols, _p(w), _p(s)) != 0:
        raise ValueError("invalid MXFP4 plan")
    return w.reshape(rows, cols // 2), s.reshape(rows, cols // 32)


def quantize_fp8(fp8: np.ndarray, inverse_scales: np.ndarray, rows: int, cols: int):
    src = np.ascontiguousarray(fp8, np.uint8)
    sc = np.ascontiguousarray(inverse_scales, np.uint16)
    w = np.zeros(rows * cols // 2, np.uint8)
    s = np.zeros(rows * cols // 32, np.uint8)
    if load().wm_oracle_quantize_fp8(_p(src), _p(sc), rows, cols, _p(w), _p(s)) != 0:
        raise ValueError("invalid MXFP4 FP8 plan")
    return w.reshape(rows, cols // 2), s.reshape(rows, cols // 32)


def dequant_mxfp4(packed: np.ndarray, scales: np.ndarray) -> np.ndarray:
    p = np.ascontiguousarray(packed).view(np.uint32)
    s = np.ascontiguousarray(scales, np.uint8)
    rows, cols = p.shape[0], p.shape[1] * 8
    out = np.zeros((rows, cols), np.float32)
    load().wm_oracle_dequant_mxfp4(_p(p), _p(s), rows, cols, _p(out))
    return out


def e4m3(b: int) -> float:
    return load().wm_oracle_e4m3(b)


def topk(scores: np.ndarray, k: int) -> np.ndarray:
    s = np.ascontiguousarray(scores, np.float32)
    out = np.zeros((s.shape[0], k), np.int32)
    load().wm_oracle_topk(_p(s), s.shape[0], s.shape[1], k, _p(out))
    return out


def ffn(x: np.ndarray, wgu: np.ndarray, wd: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    wgu = np.ascontiguousarray(wgu, np.float32)
    wd = np.ascontiguousarray(wd, np.float32)
    T, H = x.shape
    I = wgu.shape[0] // 2
    act = np.zeros((T, I), np.float32)
    y = np.zeros((T, H), np.float32)
    load().wm_oracle_ffn(_p(x), T, H, I, _p(wgu), _p(wd), _p(act), _p(y))
    return y
