"""GPU parity of the persistent one-token decode kernel against the oracle chain.

Chain (both sides): x_l = bf16(rmsnorm(r_l)); top-10 softmax routing from the
layer's logits; y = sum_k w_k FFN_k(x_l) + sigmoid(x_l . g) FFN_shared(x_l);
r_{l+1} = r_l + bf16(y). Tolerance: relative L2 <= 1e-2 and max |err| <=
2e-2 * max |ref| on the final residual and on the rmsnorm output.
"""
import numpy as np
import pytest
import torch

import whallm_amd as wa
from oracle import formats as F
from oracle import moe as M
from whallm_amd import synthetic as S
from whallm_amd.ops import PersistentDecodeStack, repack_down_slices

pytestmark = pytest.mark.gpu

H, I, K = 2048, 512, 10


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    mx = np.abs(got - want).max() / np.abs(want).max()
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"
    return rel


def test_repack_down_slices_bytes(device):
    rng = np.random.default_rng(0)
    a = S.mxfp4_experts_np(rng, 3, H, I)
    dev = S.experts_to_device(a, device)
    d, ds = repack_down_slices(dev)
    got = d.cpu().numpy().view(np.uint8).reshape(3, 8, H, 32)
    src = a["down"].view(np.uint8).reshape(3, H, 8, 32).transpose(0, 2, 1, 3)
    np.testing.assert_array_equal(got, src)
    got_s = ds.cpu().numpy().reshape(3, 8, H, 2)
    np.testing.assert_array_equal(got_s, a["down_scales"].reshape(3, H, 8, 2).transpose(0, 2, 1, 3))


class Chain:
    def __init__(self, device, layers, experts, seed):
        rng = np.random.default_rng(seed)
        self.L, self.E = layers, experts
        self.arrays = [S.mxfp4_experts_np(rng, experts, H, I) for _ in range(layers)]
        self.shared = [S.mxfp4_experts_np(rng, 1, H, I) for _ in range(layers)]
        self.gates = [S.bf16_normal_np(rng, (H,), 0.02) for _ in range(layers)]
        self.dev = [S.experts_to_device(a, device) for a in self.arrays]
        self.dev_shared = [S.experts_to_device(a, device) for a in self.shared]
        self.dev_gates = [S.bf16_bits_to_tensor(g, device) for g in self.gates]
        self.stack = PersistentDecodeStack(self.dev, self.dev_shared, self.dev_gates, k=K)
        self.rng = rng

    def inputs(self):
        logits = self.rng.standard_normal((self.L, self.E)).astype(np.float32)
        r0 = self.rng.standard_normal(H).astype(np.float32)
        return logits, r0

    def oracle(self, logits, r0):
        r = r0.astype(np.float64)
        for l in range(self.L):
            x = M.rms_norm(r[None])
            idx, w = M.route_softmax_topk(logits[l][None], K)
            a = self.arrays[l]
            experts = {int(e): M.MXFP4Expert(a["gate_up"][e], a["gate_up_scales"][e], a["down"][e],
                                             a["down_scales"][e]) for e in idx[0]}
            routed = np.stack([M.expert_ffn(x, experts[int(e)])[0] for e in idx[0]])[None]
            s = self.shared[l]
            sh = M.expert_ffn(x, M.MXFP4Expert(s["gate_up"][0], s["gate_up_scales"][0], s["down"][0],
                                                s["down_scales"][0]))
            g = x.astype(np.float64) @ S.bf16_bits_to_f32(self.gates[l]).astype(np.float64)
            y = M.combine(routed, w, sh, g)[0]
            r = r + F.bf16_round_f32(y)
        return r.astype(np.float32), M.rms_norm(r[None])[0]


@pytest.mark.parametrize("layers,experts", [(1, 16), (6, 64), (3, 512)])
def test_persistent_decode_matches_oracle_chain(device, layers, experts):
    chain = Chain(device, layers, experts, seed=layers * 7 + experts)
    print(f"xcd_local={chain.stack.xcd_local()}", flush=True)
    for call in range(3):  # successive launches advance the message epochs
        logits, r0 = chain.inputs()
        residual = torch.from_numpy(r0.copy()).to(device)
        x_out = torch.empty(H, dtype=torch.bfloat16, device=device)
        chain.stack(torch.from_numpy(logits).to(device), residual, x_out)
        torch.cuda.synchronize()
        assert chain.stack.status() == 0
        want_r, want_x = chain.oracle(logits, r0)
        close(residual.cpu().numpy(), want_r, f"residual call {call}")
        close(x_out.float().cpu().numpy(), want_x, f"x_out call {call}")


def test_persistent_decode_agrees_with_per_layer_path(device):
    # The same 4-layer chain through the per-layer kernels (wm_moe_stack_mxfp4).
    chain = Chain(device, 4, 128, seed=3)
    logits, r0 = chain.inputs()
    r_a = torch.from_numpy(r0.copy()).to(device)
    chain.stack(torch.from_numpy(logits).to(device), r_a)
    stack = wa.ops.MoEStack(chain.dev, chain.dev_shared, chain.dev_gates, k=K)
    r_b = torch.from_numpy(r0.copy()).to(device)
    stack(torch.from_numpy(logits[:, None, :].copy()).to(device), r_b.view(1, H))
    torch.cuda.synchronize()
    close(r_a.cpu().numpy(), r_b.cpu().numpy(), "persistent vs per-layer")
