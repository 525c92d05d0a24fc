"""GPU parity of the fused pre-MoE step (wm_norm_router): residual add, RMSNorm, router
GEMV and shared-gate GEMV in one launch, against oracle.norm_router and against the unfused
library path (wm_residual_rmsnorm + wm_linear_bf16), then routed on the device.

Bar: v = r + y exact (fp32 adds); x within one bf16 step of the oracle, at most 0.1% of
elements off by that step (fp32 vs float64 statistics); logits and the shared logit within
1e-5 of the float64 dot product of the kernel's own x, relative to sum |x| |w|; top-k
indices of the kernel's logits identical to the oracle's top-k of the same logits."""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import moe as M
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu


def bf16_tensor(rng, shape, device, std=1.0):
    return S.bf16_bits_to_tensor(S.bf16_normal_np(rng, shape, std), device)


def check_x(got: np.ndarray, want: np.ndarray):
    diff = got != want
    assert diff.mean() <= 1e-3, diff.mean()
    if diff.any():   # one bf16 step at most
        step = np.abs(want[diff]) * 2.0 ** -7
        assert np.all(np.abs(got[diff] - want[diff]) <= step * 1.01)


def check_dot(got, x, w):
    x64, w64 = x.astype(np.float64), w.astype(np.float64)
    want = x64 @ w64.T
    bound = np.abs(x64) @ np.abs(w64).T
    assert np.all(np.abs(got - want) <= 1e-5 * bound + 1e-30)


@pytest.mark.parametrize("T,H,E,with_y,with_w,with_gate", [
    (1, 2560, 512, True, False, True),       # C2 decode: one token, Qwen router + shared gate
    (3, 2048, 128, True, True, True),        # ragged token block
    (40, 4096, 256, False, True, False),     # DeepSeek width, no y, no gate
    (300, 2560, 512, True, True, True),      # MFMA path, 16-token blocks, ragged last block
    (20, 7168, 256, True, False, True),      # MFMA path, 8-token blocks (C4 width)
    (70, 2048, 512, True, True, True),       # MFMA path, 32-token blocks (two column blocks), ragged tail
    (17, 1000, 64, True, True, True),        # hidden not a multiple of 32: dot-product path, 16 tokens
])
def test_norm_router_matches_oracle(device, T, H, E, with_y, with_w, with_gate):
    rng = np.random.default_rng(T + H + E)
    r = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32) * 3).to(device)
    y = bf16_tensor(rng, (T, H), device) if with_y else None
    router = bf16_tensor(rng, (E, H), device, 0.05)
    gate = bf16_tensor(rng, (H,), device, 0.05) if with_gate else None
    nw = (S.bf16_bits_to_tensor(S.bf16_normal_np(rng, (H,), 0.2), device) + 1.0).to(torch.bfloat16) if with_w else None
    r_out = torch.empty_like(r)
    r_before = r.clone()
    x, logits, shared = wa.norm_router(r, y, router, gate, nw, 1e-6, residual_out=r_out)
    torch.cuda.synchronize()
    assert torch.equal(r, r_before)    # the input residual is left alone
    f = lambda t: None if t is None else t.float().cpu().numpy()
    v, x_want, _, _ = M.norm_router(f(r), f(y), f(router), f(gate), f(nw))
    np.testing.assert_array_equal(f(r_out), v)
    xg = f(x)
    check_x(xg, x_want)
    check_dot(f(logits), xg, f(router))
    if with_gate:
        check_dot(f(shared)[:, None], xg, f(gate)[None, :])
    else:
        assert shared is None
    # routed on the device from the fused logits
    k = 8
    idx, w = wa.route_softmax_topk(logits, k)
    want_idx, want_w = M.route_softmax_topk(f(logits), k)
    np.testing.assert_array_equal(idx.cpu().numpy(), want_idx)
    np.testing.assert_allclose(w.cpu().numpy(), want_w, rtol=1e-5, atol=1e-7)


def test_fused_matches_the_unfused_path(device):
    """Same inputs through wm_residual_rmsnorm + wm_linear_bf16 (x to one bf16 step, logits
    to the dot-product bound)."""
    T, H, E = 16, 2560, 512
    rng = np.random.default_rng(11)
    r = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(device)
    y = bf16_tensor(rng, (T, H), device)
    router = bf16_tensor(rng, (E, H), device, 0.05)
    r_out = torch.empty_like(r)
    x, logits, _ = wa.norm_router(r, y, router, residual_out=r_out)
    r2 = r.clone()
    x2 = wa.ops.residual_rmsnorm(r2, y)
    logits2 = wa.linear_bf16(x2, router)
    torch.cuda.synchronize()
    assert torch.equal(r_out, r2)
    check_x(x.float().cpu().numpy(), x2.float().cpu().numpy())
    same = (x == x2).all(dim=-1).cpu().numpy()
    g, u = logits.cpu().numpy(), logits2.cpu().numpy()
    check_dot(g[same], x.float().cpu().numpy()[same], router.float().cpu().numpy())
    check_dot(u[same], x.float().cpu().numpy()[same], router.float().cpu().numpy())


def test_empty_and_error_paths(device):
    r = torch.zeros((0, 256), dtype=torch.float32, device=device)
    router = torch.zeros((8, 256), dtype=torch.bfloat16, device=device)
    x, logits, shared = wa.norm_router(r, None, router)
    assert x.shape == (0, 256) and logits.shape == (0, 8) and shared is None
    r = torch.zeros((2, 256), dtype=torch.float32, device=device)
    with pytest.raises(Exception, match="overlap"):
        wa.norm_router(r, None, router, residual_out=r)
    with pytest.raises(ValueError, match="router"):
        wa.norm_router(r, None, router[:, :128])


@pytest.mark.parametrize("T,H,E,with_gate", [(300, 2560, 512, True), (20, 7168, 256, True), (64, 2048, 40, False),
                                             (1, 2048, 512, True)])
def test_packed_router_is_bit_identical(device, T, H, E, with_gate):
    """repack_router's fragment order (checked against a torch permute of the zero-padded
    rows) feeds the prefill GEMM the same operands, so logits are bit-identical to the row
    path; at one token (dot-product path) the packed copy is not read."""
    rng = np.random.default_rng(T * 7 + E)
    r = torch.from_numpy(rng.standard_normal((T, H)).astype(np.float32)).to(device)
    y = bf16_tensor(rng, (T, H), device)
    router = bf16_tensor(rng, (E, H), device, 0.05)
    gate = bf16_tensor(rng, (H,), device, 0.05) if with_gate else None
    packed = wa.repack_router(router, gate)
    rows = torch.cat([router, gate[None]]) if with_gate else router
    G = (rows.shape[0] + 15) // 16 + int(with_gate)   # a spare zero group marks a packed gate
    padded = torch.zeros(G * 16, H, dtype=torch.bfloat16, device=device)
    padded[:rows.shape[0]] = rows
    want = padded.view(G, 16, H // 32, 4, 8).permute(0, 2, 3, 1, 4).contiguous()
    assert torch.equal(packed.view(torch.bfloat16).view(want.shape), want)
    a = wa.norm_router(r, y, router, gate)
    b = wa.norm_router(r, y, router, gate, router_packed=packed)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert (u is None and v is None) or torch.equal(u, v)
    if T >= 16:
        with pytest.raises(Exception, match="does not match"):
            wa.norm_router(r, y, router, None if with_gate else bf16_tensor(rng, (H,), device), router_packed=packed)


@pytest.mark.parametrize("T,H,E", [(300, 2048, 512), (70, 7168, 256), (64, 1024, 64), (63, 2048, 128),
                                   (1, 2048, 512), (3, 7168, 1000), (4, 7168, 129280), (16, 1032, 77), (9, 2048, 64)])
def test_linear_bf16_prefill_path(device, T, H, E):
    """wm_linear_bf16 at 64+ tokens runs on the router GEMM's MFMA path (a tile of x as
    given), up to 16 tokens on the row-streaming kernel (every weight row read once for all
    tokens; the C5 LM head at 4 x 129,280), in between on the one-wave-per-output kernel:
    each within the dot-product bound of the float64 product."""
    rng = np.random.default_rng(T + E)
    x = bf16_tensor(rng, (T, H), device)
    w = bf16_tensor(rng, (E, H), device, 0.05)
    got = wa.linear_bf16(x, w)
    torch.cuda.synchronize()
    check_dot(got.cpu().numpy(), x.float().cpu().numpy(), w.float().cpu().numpy())


@pytest.mark.parametrize("T,H,with_y", [(1, 2048, True), (4, 7168, True), (33, 1024, False), (5, 8192, True),
                                        (3, 2560, True), (2, 640, False)])
def test_residual_rmsnorm_matches_oracle(device, T, H, with_y):
    """wm_residual_rmsnorm on both of its kernels (hidden = 1024 n up to 8192 holds a row in
    registers; other widths walk it 256 columns at a time): r += y exact, x within one bf16
    step of oracle.rms_norm on the updated r."""
    rng = np.random.default_rng(T * 131 + H)
    r0 = rng.standard_normal((T, H)).astype(np.float32) * 3
    r = torch.from_numpy(r0).to(device)
    y = bf16_tensor(rng, (T, H), device) if with_y else None
    x = wa.ops.residual_rmsnorm(r, y)
    torch.cuda.synchronize()
    want_r = r0 + (y.float().cpu().numpy() if with_y else 0.0)
    np.testing.assert_array_equal(r.cpu().numpy(), want_r.astype(np.float32))
    check_x(x.float().cpu().numpy(), M.rms_norm(want_r, 1e-6))
