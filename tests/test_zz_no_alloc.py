"""GPU test of the allocation-free entry point (wm_moe_mxfp4_noalloc): through the C ABI,
its output equals wm_moe_mxfp4's bit for bit on two calls in a row (the second smaller,
so stale scratch contents from the first would show), with and without a shared expert,
and a call beyond its scratch or off the decode path fails with a message."""
import ctypes

import numpy as np
import pytest
import torch

from whallm_amd import _lib
from whallm_amd import synthetic as S
from whallm_amd.ops import _ptr, _stream, _workspace

pytestmark = pytest.mark.gpu


def _call_pair(device, table, shared, gate, tokens, k, seed):
    rng = np.random.default_rng(seed)
    E = table.count
    x = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (tokens, table.hidden)), device)
    idx = torch.from_numpy(np.stack([rng.choice(E, k, replace=False) for _ in range(tokens)]).astype(np.int32)).to(device)
    w = torch.from_numpy(rng.random((tokens, k)).astype(np.float32)).to(device)
    c = table.c_struct()
    sc = shared.c_struct() if shared is not None else None
    sref = ctypes.byref(sc) if sc is not None else None
    lib = _lib.load()
    ws_bytes = lib.wm_moe_mxfp4_workspace_size(tokens, k, ctypes.byref(c))
    ws = _workspace(ws_bytes, device)
    y_ref = torch.empty_like(x)
    _lib.call("wm_moe_mxfp4", _ptr(x), tokens, _ptr(idx), _ptr(w), k, ctypes.byref(c), sref, _ptr(gate), _ptr(y_ref),
              _ptr(ws), ws_bytes, _stream(device))
    y = torch.full_like(x, 3.0)
    _lib.call("wm_moe_mxfp4_noalloc", _ptr(x), tokens, _ptr(idx), _ptr(w), k, ctypes.byref(c), sref, _ptr(gate),
              _ptr(y), _stream(device))
    torch.cuda.synchronize()
    return y, y_ref


def test_noalloc_matches_the_workspace_entry_point(device):
    rng = np.random.default_rng(0)
    H, I, E = 2048, 512, 64
    table = S.experts_to_device(S.mxfp4_experts_np(rng, E, H, I), device)
    shared = S.experts_to_device(S.mxfp4_experts_np(rng, 1, H, I), device)
    gate = S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (H,), 0.02), device)
    assert _lib.load().wm_moe_mxfp4_noalloc_max_bytes() == 4 << 20
    for tokens, k, sh, seed in ((16, 10, shared, 1), (1, 10, shared, 2), (8, 4, None, 3), (2, 4, None, 4)):
        y, y_ref = _call_pair(device, table, sh, gate if sh is not None else None, tokens, k, seed)
        assert torch.equal(y, y_ref), (tokens, k)


def test_noalloc_rejects_what_it_cannot_hold(device):
    # a real (small) table, so nothing would read outside it even if a check were missing
    rng = np.random.default_rng(5)
    table = S.experts_to_device(S.mxfp4_experts_np(rng, 2, 256, 8192), device)
    c = table.c_struct()
    x = torch.zeros(32, 256, dtype=torch.bfloat16, device=device)
    idx = torch.zeros(32, 8, dtype=torch.int32, device=device)
    w = torch.zeros(32, 8, dtype=torch.float32, device=device)
    with pytest.raises(_lib.WhallmError, match="bytes of scratch"):   # 4 * 32 * 9 * 8192 > 4 MiB
        _lib.call("wm_moe_mxfp4_noalloc", _ptr(x), 32, _ptr(idx), _ptr(w), 8, ctypes.byref(c), None, None, _ptr(x),
                  _stream(device))
    x = torch.zeros(300, 256, dtype=torch.bfloat16, device=device)
    idx = torch.zeros(300, 1, dtype=torch.int32, device=device)
    w = torch.zeros(300, 1, dtype=torch.float32, device=device)
    with pytest.raises(_lib.WhallmError, match="decode path"):
        _lib.call("wm_moe_mxfp4_noalloc", _ptr(x), 300, _ptr(idx), _ptr(w), 1, ctypes.byref(c), None, None, _ptr(x),
                  _stream(device))
