"""The C-ABI library loads and exports what include/*.h declares (CPU: no kernel launches)."""
import ctypes
import re
from pathlib import Path

import pytest

from whallm_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    names = set()
    for header in (ROOT / "include").glob("*.h"):
        text = header.read_text()
        names.update(re.findall(r"WM_EXPORT\s+[\w\s\*]+?\b(wm_\w+)\s*\(", text))
    return sorted(names)


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "wm_moe_mxfp4" in names and "wm_permute" in names and len(names) >= 10


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in declared_symbols() if not hasattr(lib, n)]
    assert missing == []


def test_binding_covers_every_declared_symbol():
    assert set(declared_symbols()) <= set(_lib.exported_symbols())


def test_version_and_argument_checks_fail_before_any_launch():
    lib = _lib.load()
    assert b"gfx950" in lib.wm_version()
    with pytest.raises(_lib.WhallmError, match="experts must be in"):
        _lib.call("wm_route_softmax_topk", None, 1, 0, 1, 1, None, None, None, None)
    with pytest.raises(_lib.WhallmError, match="k must be"):
        _lib.call("wm_route_softmax_topk", None, 1, 8, 9, 1, None, None, None, None)
    with pytest.raises(_lib.WhallmError, match="workspace too small"):
        _lib.call("wm_permute", None, 10, 4, 16, None, None, None, None, None, None, 0, None)
    table = _lib.MXFP4ExpertsC()
    with pytest.raises(_lib.WhallmError, match="expert region pointer is null"):
        _lib.call("wm_moe_mxfp4", None, 1, None, None, 2, ctypes.byref(table), None, None, None, None, 0, None)
    with pytest.raises(_lib.WhallmError, match="drafts must be in"):
        _lib.call("wm_mtp_verify_greedy", None, None, 16, 100, None, None, 0, None)
    with pytest.raises(_lib.WhallmError, match="workspace too small"):
        _lib.call("wm_mtp_verify_rejection", 1, 1, 1, 3, 100, 1, 1, 1, 0, None)
    # The error message is per thread and clears on the next good call.
    assert lib.wm_last_error() != b""


def _fake_table(tiled: int, hidden=256, inter=128):
    """A table with aligned non-null (never dereferenced) addresses: argument checks only."""
    t = _lib.MXFP4ExpertsC()
    t.gate_up = t.gate_up_scales = t.down = t.down_scales = 0x10000
    t.experts, t.hidden, t.inter, t.tiled = 8, hidden, inter, tiled
    return t


def test_prefill_tile_layout_argument_checks():
    routed, shared = _fake_table(1), _fake_table(0)
    with pytest.raises(_lib.WhallmError, match="both tiled"):
        _lib.call("wm_moe_mxfp4", 1, 1, 1, 1, 2, ctypes.byref(routed), ctypes.byref(shared), None, 1, 1, 1 << 40, None)
    with pytest.raises(_lib.WhallmError, match="multiples of 128"):
        _lib.call("wm_moe_mxfp4", 1, 1, 1, 1, 2, ctypes.byref(_fake_table(1, hidden=96)), None, None, 1, 1, 1 << 40,
                  None)
    with pytest.raises(_lib.WhallmError, match="prefill tile layout"):
        _lib.call("wm_moe_stack_mxfp4", 1, 1, 1, 2, 1, ctypes.byref(routed), None, None, 1, 1e-6, None, 1, 1 << 40,
                  None, None, None)
    with pytest.raises(_lib.WhallmError, match="already in the prefill tile layout"):
        _lib.call("wm_repack_prefill_mxfp4", ctypes.byref(routed), 16, 16, 16, 16, None)
    # a tiled table always takes the grouped GEMM: its workspace is the prefill one, not the
    # (smaller) decode buffer of a single-token call
    lib = _lib.load()
    assert lib.wm_moe_mxfp4_workspace_size(1, 2, ctypes.byref(routed)) > \
        lib.wm_moe_mxfp4_workspace_size(1, 2, ctypes.byref(_fake_table(0)))


def _fake_fp8_table(tiled: int, hidden=1024, inter=1024):
    """An FP8 table with aligned non-null (never dereferenced) addresses: argument checks only."""
    t = _lib.FP8ExpertsC()
    t.w13 = t.w13_scales = t.w2 = t.w2_scales = 0x10000
    t.experts, t.hidden, t.inter, t.tiled = 8, hidden, inter, tiled
    return t


def test_fp8_prefill_tile_layout_argument_checks():
    routed, shared = _fake_fp8_table(1), _fake_fp8_table(0)
    with pytest.raises(_lib.WhallmError, match="both tiled"):
        _lib.call("wm_moe_fp8", 1, 1, 1, 1, 2, ctypes.byref(routed), ctypes.byref(shared), None, 1, 1, 1 << 40, None)
    with pytest.raises(_lib.WhallmError, match="already in the prefill tile layout"):
        _lib.call("wm_repack_prefill_fp8", ctypes.byref(routed), 16, 16, 16, 16, None)
    with pytest.raises(_lib.WhallmError, match="null destination"):
        _lib.call("wm_repack_prefill_fp8", ctypes.byref(shared), 16, None, 16, 16, None)
    with pytest.raises(_lib.WhallmError, match="16-byte aligned"):
        _lib.call("wm_repack_prefill_fp8", ctypes.byref(shared), 8, 16, 16, 16, None)
    with pytest.raises(_lib.WhallmError, match="multiples of 128"):
        _lib.call("wm_repack_prefill_fp8", ctypes.byref(_fake_fp8_table(0, hidden=96)), 16, 16, 16, 16, None)
    # a tiled table always takes the grouped GEMM, whose workspace exceeds the decode buffer
    lib = _lib.load()
    assert lib.wm_moe_fp8_workspace_size(1, 2, ctypes.byref(routed)) > \
        lib.wm_moe_fp8_workspace_size(1, 2, ctypes.byref(shared))


def test_norm_router_argument_checks():
    """wm_norm_router refuses bad shapes, unpaired gate pointers, an output residual that
    overlaps the input and misaligned tensors before any launch."""
    a, b = 0x10000, 0x20000   # residual at a, everything else elsewhere
    def call(*, tokens=1, hidden=256, experts=8, residual=a, router=b, gate=None, shared=None, x=b + 0x10000, r_out=None,
             logits=b + 0x20000, packed=None, packed_bytes=0):
        _lib.call("wm_norm_router", residual, None, None, tokens, hidden, 1e-6, router, experts, gate, packed,
                  packed_bytes, x, r_out, logits, shared, None)
    for kw, msg in (({"hidden": 260}, "multiple of 8"), ({"hidden": 40000}, "multiple of 8"), ({"experts": 0}, "at least 1"),
                    ({"gate": a}, "go together"), ({"shared": a}, "go together"), ({"x": None}, "null pointer"),
                    ({"r_out": a + 512}, "must not overlap"), ({"x": a + 512}, "x must not overlap"),
                    ({"residual": a + 4}, "16-byte aligned"),
                    ({"tokens": -1}, "negative"), ({"packed": a, "packed_bytes": 4096}, "packed router does not match"),
                    ({"packed": a, "packed_bytes": 8192, "gate": a, "shared": a}, "packed router does not match")):
        with pytest.raises(_lib.WhallmError, match=msg):
            call(**kw)
    call(tokens=0)   # nothing to do
    lib = _lib.load()
    assert lib.wm_router_packed_bytes(8, 256, 0) == 16 * 256 * 2
    assert lib.wm_router_packed_bytes(16, 256, 1) == 48 * 256 * 2 and lib.wm_router_packed_bytes(8, 40, 0) == 0
    for e in range(1, 70):   # with and without the gate row the sizes always differ
        assert lib.wm_router_packed_bytes(e, 256, 1) != lib.wm_router_packed_bytes(e, 256, 0)
    with pytest.raises(_lib.WhallmError, match="multiple of 32"):
        _lib.call("wm_repack_router", a, None, 8, 40, a, None)
