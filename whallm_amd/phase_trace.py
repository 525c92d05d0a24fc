"""Per-layer phase trace of the persistent decode kernel (a profiling tool, not on the path).

    python -m whallm_amd.phase_trace [--tokens N]

Builds an instrumented copy of libwhallm_moe.so in whallm_amd/_build/trace/: the kernel source
is compiled with phase_trace.h first, which turns the kernel's WM_DS_TRACE / WM_DS_NOTE
hooks into stores of s_memrealtime (100 MHz, one clock for the whole chip) or of a value
into a device buffer [workgroup 256][layer 128][wave 4][point 16]; every other object is
the library's own. It then runs the C2 stack (48 layers x 512 MXFP4 experts, hidden 2048,
intermediate 512, top-10 + shared, synthetic weights) for a few tokens and prints, per
phase point, the min / median / max over the 256 workgroups of its time after the layer's
first S0, averaged over layers 2..45, and the mean re-poll rounds of each gather.
"""
from __future__ import annotations

import argparse
import ctypes
import subprocess
from pathlib import Path

import numpy as np

from . import build as hip_build

PACKAGE = Path(__file__).resolve().parent
TRACE_DIR = hip_build.BUILD / "trace"
TRACE_LIB = TRACE_DIR / "libwhallm_moe_trace.so"
HEADER = hip_build.CSRC / "phase_trace.h"

# point -> (wave role, name); compute waves 0..2, message wave 3
POINTS = [(0, 0, "compute: S0 (r and its norm in LDS)"), (0, 3, "compute: phase A done, own act gathered"),
          (3, 2, "message: shared gate published"),
          (0, 4, "compute: next A tile issued"), (0, 6, "compute: phase B done"), (3, 4, "message: partial published"),
          (3, 12, "message: partials gathered"), (3, 6, "message: r published"), (3, 13, "message: r gathered")]
NOTES = [(15, "partial"), (7, "r")]


def build_traced() -> Path:
    """Compile the library's decode_persistent.hip with the trace hooks and link it with the
    library's other objects."""
    hip_build.build()
    TRACE_DIR.mkdir(parents=True, exist_ok=True)
    src = hip_build.CSRC / "decode_persistent.hip"
    obj = TRACE_DIR / "decode_persistent_trace.o"
    cmd = [hip_build.hipcc(), *hip_build.HIP_FLAGS, f"-I{hip_build.INCLUDE}", f"-I{hip_build.CSRC}", "-include",
           str(HEADER), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on the traced kernel:\n{r.stderr}")
    objs = [str(o) for o in sorted(hip_build.BUILD.glob("*.o")) if o.stem != "decode_persistent"]
    r = subprocess.run([hip_build.hipcc(), f"--offload-arch={hip_build.ARCH}", "-shared", "-fPIC", *objs, str(obj),
                        "-o", str(TRACE_LIB)], capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link of the traced library failed:\n{r.stderr}")
    return TRACE_LIB


def run(tokens: int = 30, seed: int = 0) -> np.ndarray:
    """Trace `tokens` launches of the C2 stack; returns the trace [256, 48, 4, 16] in us."""
    import torch

    from . import _lib
    _lib.LIB_PATH = TRACE_LIB
    lib = _lib.load()
    lib.wm_trace_set.argtypes = [ctypes.c_void_p]
    lib.wm_trace_set.restype = ctypes.c_int
    from . import synthetic as S
    from .ops import PersistentDecodeStack
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    L, H, E, I, K = 48, 2048, 512, 512, 10
    layers = [S.mxfp4_experts_device(E, H, I, dev, g) for _ in range(L)]
    shared = [S.mxfp4_experts_device(1, H, I, dev, g) for _ in range(L)]
    gates = [(torch.randn(H, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(L)]
    stack = PersistentDecodeStack(layers, shared, gates, k=K)
    trace = torch.zeros(256 * 128 * 4 * 16, dtype=torch.int64, device=dev)
    if lib.wm_trace_set(ctypes.c_void_p(trace.data_ptr())) != 0:
        raise RuntimeError("wm_trace_set failed")
    logits = torch.empty(L, E, device=dev)
    residual = torch.empty(H, device=dev)
    for _ in range(tokens):
        logits.normal_(generator=g)
        residual.normal_(generator=g)
        stack(logits, residual, check=False)
    torch.cuda.synchronize()
    stack.raise_for_status()
    return trace.cpu().numpy().reshape(256, 128, 4, 16)[:, :L].astype(np.float64) / 100.0


def summary(t: np.ndarray) -> str:
    layers = range(2, t.shape[1] - 2)
    starts = [t[:, l, 3, 8].min() for l in range(t.shape[1])]
    periods = np.diff(starts)[1:-1]
    out = [f"per-layer period (first message-wave S0 to the next), layers 1..{t.shape[1] - 3}: "
           f"mean {periods.mean():.2f} us, min {periods.min():.2f}, max {periods.max():.2f}",
           "time after the layer's first S0, us: min / median / max over the 256 workgroups, "
           f"averaged over layers {layers.start}..{layers.stop - 1}"]
    for w, p, name in POINTS:
        d = np.array([[f(t[:, l, w, p] - starts[l]) for f in (np.min, np.median, np.max)] for l in layers]).mean(0)
        out.append(f"  {name:40s} {d[0]:6.2f} {d[1]:6.2f} {d[2]:6.2f}")
    for p, name in NOTES:
        v = t[:, layers.start:layers.stop, 3, p] * 100.0
        out.append(f"{name} gather: re-poll rounds mean {v.mean():.2f}, p90 {np.percentile(v, 90):.0f}, max {v.max():.0f}")
    return "\n".join(out)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--tokens", type=int, default=30)
    ap.add_argument("--save", default=None, help="also save the raw trace (.npy)")
    args = ap.parse_args()
    build_traced()
    t = run(args.tokens)
    if args.save:
        np.save(args.save, t)
    print(summary(t))


if __name__ == "__main__":
    main()
