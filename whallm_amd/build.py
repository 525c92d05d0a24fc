"""Build libwhallm_moe.so (HIP, gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` file is compiled to an object in ``whallm_amd/_build`` and
linked into ``whallm_amd/lib/libwhallm_moe.so``. Objects are rebuilt when their
source or any header is newer. ``python -m whallm_amd.build`` runs it.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIB = PACKAGE / "lib" / "libwhallm_moe.so"
INCLUDE = PACKAGE.parent / "include"
ARCH = "gfx950"

# Packed FP32 instructions are switched off for all device code: some of their
# forms have given silently wrong results on the GPU pool this is built for.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-fvisibility=hidden",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libwhallm_moe")
    return found


def _headers_mtime() -> float:
    headers = list(CSRC.glob("*.h")) + list(INCLUDE.glob("*.h"))
    return max((h.stat().st_mtime for h in headers), default=0.0)


def _compile(source: Path, force: bool) -> Path:
    obj = BUILD / (source.stem + ".o")
    if (not force and obj.exists()
            and obj.stat().st_mtime >= max(source.stat().st_mtime, _headers_mtime())):
        return obj
    cmd = [hipcc(), *HIP_FLAGS, f"-I{INCLUDE}", "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")
    return obj


def build(force: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError("no HIP sources under " + str(CSRC))
    jobs = jobs or min(8, os.cpu_count() or 1)
    with ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(lambda s: _compile(s, force), sources))
    newest = max(o.stat().st_mtime for o in objects)
    if force or not LIB.exists() or LIB.stat().st_mtime < newest:
        tmp = LIB.with_suffix(".so.tmp")
        # -z defs: an undefined symbol (a declaration without its definition) fails the link
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", *map(str, objects), "-o", str(tmp)]
        result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"link of {LIB.name} failed:\n{result.stderr}")
        os.replace(tmp, LIB)
    return LIB


HOST_META_SRC = CSRC / "host_meta.cpp"


def host_meta_path() -> Path:
    """Where the operator mirrors' host helper (csrc/host_meta.cpp) is built."""
    import sysconfig
    return LIB.parent / ("_host_meta" + sysconfig.get_config_var("EXT_SUFFIX"))


def build_host_meta(force: bool = False) -> Path:
    """Compile csrc/host_meta.cpp into a CPython extension against the installed torch (host
    code only, g++); returns its path."""
    import sysconfig

    import torch
    from torch.utils import cpp_extension

    out = host_meta_path()
    if not force and out.exists() and out.stat().st_mtime >= HOST_META_SRC.stat().st_mtime:
        return out
    LIB.parent.mkdir(exist_ok=True)
    tmp = out.with_name(out.name + ".tmp")
    cmd = ["g++", "-O2", "-shared", "-fPIC", "-std=c++17", "-DTORCH_EXTENSION_NAME=_host_meta",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{p}" for p in cpp_extension.include_paths()], f"-I{sysconfig.get_paths()['include']}",
           str(HOST_META_SRC), "-o", str(tmp),
           *[f"-L{p}" for p in cpp_extension.library_paths()], "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"g++ failed on {HOST_META_SRC.name}:\n{result.stderr}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    path = build(force="--force" in sys.argv)
    print(path)
    print(build_host_meta(force="--force" in sys.argv))
