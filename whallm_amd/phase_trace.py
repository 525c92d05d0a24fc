"""Phase traces of the decode kernels (a profiling tool, not on the path).

    python -m whallm_amd.phase_trace [--kernel persistent|layer] [--tokens N] [--layers L]

Builds an instrumented copy of libwhallm_moe.so in whallm_amd/lib/trace/: the kernel source
is compiled with phase_trace.h first, which turns the kernel's WM_DS_TRACE / WM_DS_NOTE
hooks into stores of s_memrealtime (100 MHz, one clock for the whole chip) or of a value
into a device buffer [workgroup 256][layer or call 128][wave 4][point 16]; every other
object is the library's own.
- persistent: runs the C2 stack (48 layers x 512 MXFP4 experts, hidden 2048, intermediate
  512, top-10 + shared, synthetic weights) for a few tokens and prints, per phase point, the
  min / median / max over the 256 workgroups of its time after the layer's first S0,
  averaged over layers 2..45, and the mean re-poll rounds of each gather;
- layer: runs the one-launch decode layer (wm_moe_layer_decode) at the C2 shape for a few
  calls and prints, per phase point, the min / median / max over the workgroups of its time
  after the call's first start, averaged over the calls after the first; with --layers L the
  calls cycle over L layers of distinct weights, as a stack runs them.
"""
from __future__ import annotations

import argparse
import ctypes
import subprocess
from pathlib import Path

import numpy as np

from . import build as hip_build

PACKAGE = Path(__file__).resolve().parent
TRACE_DIR = PACKAGE / "lib" / "trace"   # beside the library, so a prebuilt copy travels with it
TRACE_LIB = TRACE_DIR / "libwhallm_moe_trace.so"
HEADER = hip_build.CSRC / "phase_trace.h"
HEADERS = {"persistent": HEADER, "layer": hip_build.CSRC / "phase_trace_lds.h"}

# point -> (wave role, name); compute waves 0..2, message wave 3
POINTS = [(0, 0, "compute: S0 (r and its norm in LDS)"), (0, 3, "compute: phase A done, own act gathered"),
          (3, 2, "message: shared gate published"),
          (0, 4, "compute: next A tile issued"), (0, 6, "compute: phase B done"), (3, 4, "message: partial published"),
          (3, 12, "message: partials gathered"), (3, 6, "message: r published"), (3, 13, "message: r gathered")]
NOTES = [(15, "partial"), (7, "r")]


SOURCES = {"persistent": "decode_persistent", "layer": "decode_layer"}


def build_traced(kernel: str = "persistent") -> Path:
    """Compile the kernel's source with the trace hooks and link it with the library's other
    objects."""
    hip_build.build()
    TRACE_DIR.mkdir(parents=True, exist_ok=True)
    stem = SOURCES[kernel]
    src = hip_build.CSRC / f"{stem}.hip"
    obj = hip_build.BUILD / "trace" / f"{stem}_trace.o"
    obj.parent.mkdir(parents=True, exist_ok=True)
    cmd = [hip_build.hipcc(), *hip_build.HIP_FLAGS, f"-I{hip_build.INCLUDE}", f"-I{hip_build.CSRC}", "-include",
           str(HEADERS[kernel]), "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on the traced kernel:\n{r.stderr}")
    objs = [str(o) for o in sorted(hip_build.BUILD.glob("*.o")) if o.stem != stem]
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


LAYER_POINTS = [(0, 0, "start"), (0, 1, "x in LDS"), (0, 2, "logits published"), (0, 3, "logits in LDS"),
                (0, 8, "top-k done (wave 0)"), (0, 4, "routed"), (0, 12, "gate_up rows issued"),
                (0, 13, "first pair computed"), (0, 5, "gate_up published"),
                (1, 11, "flag stored, down rows issued (wave 1)"), (0, 10, "act flags complete"),
                (0, 6, "act gathered"), (0, 7, "done")]


def run_layer(calls: int = 40, seed: int = 0, layers: int = 1) -> np.ndarray:
    """Trace `calls` launches of the decode layer at C2; returns the trace [256, calls, 4, 16]
    in us (call c at slot (c + 1) % 128). With `layers` > 1 the calls cycle over that many
    layers of distinct weights (as a stack runs them: each call's experts cold in the caches
    and TLBs), else one layer's weights serve every call."""
    import torch

    from . import _lib
    _lib.LIB_PATH = TRACE_LIB
    lib = _lib.load()
    lib.wm_trace_set.argtypes = [ctypes.c_void_p]
    lib.wm_trace_set.restype = ctypes.c_int
    from . import synthetic as S
    from .ops import DecodeLayer
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    H, E, I, K = 2048, 512, 512, 10
    stack = []
    for _ in range(max(layers, 1)):
        experts = S.mxfp4_experts_device(E, H, I, dev, g)
        shared = S.mxfp4_experts_device(1, H, I, dev, g)
        gate = (torch.randn(H, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        router = (torch.randn(E, H, device=dev, generator=g) * 0.05).to(torch.bfloat16)
        stack.append(DecodeLayer(experts, router, shared, gate, k=K))
    for layer in stack[1:]:  # one state: the epoch (the trace slot) counts every call
        layer.state = stack[0].state
    trace = torch.zeros(256 * 128 * 4 * 16, dtype=torch.int64, device=dev)
    if lib.wm_trace_set(ctypes.c_void_p(trace.data_ptr())) != 0:
        raise RuntimeError("wm_trace_set failed")
    r = torch.randn(H, device=dev, generator=g)
    for c in range(min(calls, 126)):
        stack[c % len(stack)](r)
    torch.cuda.synchronize()
    for layer in stack:
        layer.raise_for_status()
    t = trace.cpu().numpy().reshape(256, 128, 4, 16)[:, 1:min(calls, 126) + 1].astype(np.float64) / 100.0
    return t


def summary_layer(t: np.ndarray) -> str:
    calls = range(1, t.shape[1])
    out = ["time after the call's first start, us: min / median / max over the 256 workgroups (wave 0), "
           f"averaged over calls {calls.start}..{calls.stop - 1}"]
    for w, p, name in LAYER_POINTS:
        d = np.array([[f(t[:, c, w, p] - t[:, c, 0, 0].min()) for f in (np.min, np.median, np.max)]
                      for c in calls]).mean(0)
        out.append(f"  {name:40s} {d[0]:6.2f} {d[1]:6.2f} {d[2]:6.2f}")
    return "\n".join(out)


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
    ap.add_argument("--kernel", default="persistent", choices=sorted(SOURCES))
    ap.add_argument("--tokens", type=int, default=30, help="tokens (persistent) or calls (layer)")
    ap.add_argument("--save", default=None, help="also save the raw trace (.npy)")
    ap.add_argument("--prebuilt", action="store_true", help="use the traced library built beforehand")
    ap.add_argument("--layers", type=int, default=1,
                    help="layer: cycle the calls over this many layers of distinct weights")
    args = ap.parse_args()
    if not args.prebuilt:
        build_traced(args.kernel)
    t = run(args.tokens) if args.kernel == "persistent" else run_layer(args.tokens, layers=args.layers)
    if args.save:
        np.save(args.save, t)
    print(summary(t) if args.kernel == "persistent" else summary_layer(t))


if __name__ == "__main__":
    main()
