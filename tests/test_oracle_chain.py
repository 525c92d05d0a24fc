"""The 48-layer decode chain of the oracle is ill-conditioned: its own result moves by more
than the 1e-2 tolerance under a perturbation of one bf16 ulp per output element and layer.

Chain (the C2 stack, H 2048, 512 experts, I 512, top-10 + gated shared expert, one token):
x_l = bf16(rmsnorm(r_l)) (the norm of layer l > 0 reads the bf16 copy of r_l, as the kernel's
broadcast does), y_l = the oracle's fp32/float64 MoE layer, r_{l+1} = r_l + bf16(y_l). The
perturbed chain rounds y_l toward zero instead of to nearest even: each element of each
layer's output moves by at most one bf16 ulp, a change of the size of the kernel's own
deviation from the oracle per layer (its bf16 output rounding). The end-to-end relative L2
between the two chains is required to exceed 1e-2: a free-running 48-layer comparison at the
1e-2 bar tests the chain's conditioning, not the kernel, which is why the GPU test checks every
layer from the kernel's own input and bounds the free-running drift by twice this spread
(tests/test_gpu_decode_persistent.py). Experts are drawn per (layer, expert) from the
benchmark's distribution (MXFP4 codes uniform, scale bytes 119..125), only the routed ones.
"""
import numpy as np

from oracle import formats as F
from oracle import moe as M
from whallm_amd import synthetic as S

H, I, K, L, E = 2048, 512, 10, 48, 512


def bf16_round_toward_zero(v):
    return (np.asarray(v, np.float32).view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)


def chain_spread(seed: int) -> float:
    experts = {}

    def expert(l, e):
        if (l, e) not in experts:
            a = S.mxfp4_experts_np(np.random.default_rng([seed, l, e]), 1, H, I)
            experts[(l, e)] = M.MXFP4Expert(a["gate_up"][0], a["gate_up_scales"][0], a["down"][0],
                                            a["down_scales"][0])
        return experts[(l, e)]

    rng = np.random.default_rng([seed, 1000])
    gates = [S.bf16_bits_to_f32(S.bf16_normal_np(rng, (H,), 0.02)).astype(np.float64) for _ in range(L)]
    logits = rng.standard_normal((L, E)).astype(np.float32)
    r0 = rng.standard_normal(H).astype(np.float32)

    def chain(rounding):
        r = r0.astype(np.float64)
        for l in range(L):
            x = M.rms_norm((r if l == 0 else F.bf16_round_f32(r))[None])
            idx, w = M.route_softmax_topk(logits[l][None], K)
            routed = np.stack([M.expert_ffn(x, expert(l, int(e)))[0] for e in idx[0]])[None]
            shared = M.expert_ffn(x, expert(l, E))
            y = M.combine(routed, w, shared, x.astype(np.float64) @ gates[l])[0]
            r = r + rounding(y)
        return r

    nearest = chain(F.bf16_round_f32)
    toward_zero = chain(bf16_round_toward_zero)
    return float(np.linalg.norm(toward_zero - nearest) / np.linalg.norm(nearest))


def test_48_layer_chain_spread_exceeds_the_tolerance():
    spread = chain_spread(5)
    print(f"48-layer oracle chain, y rounded toward zero vs to nearest: rel L2 {spread:.3e}")
    assert spread >= 1e-2


def test_bf16_round_toward_zero_moves_at_most_one_ulp():
    v = np.random.default_rng(0).standard_normal(4096).astype(np.float32) * 1e3
    a, b = F.bf16_round_f32(v), bf16_round_toward_zero(v)
    ulp = np.abs(a) * 2.0 ** -7
    assert np.all(np.abs(a - b) <= ulp) and np.all(np.abs(b) <= np.abs(v))
