"""Writes the seeded golden fixtures of tests/golden/ from the oracle (numpy restatement).

    python tests/golden/make_fixtures.py

Fixtures (inputs, expected outputs, and SHA-256 digests of the seeded weights so a
drift in the generator is caught rather than silently re-baselined):

* c1_layer_seed0.npz — BASELINE configs[0] (C1): hidden 1024, 64 experts, moe_intermediate
  512, top-4 softmax routing with a bf16 N(0, 0.02) router weight, MXFP4 weights (codes
  uniform, E8M0 exponents uniform in [-8, -2]), bf16 N(0, 1) activations, 16 tokens, seed 0.
  Holds x, the router logits, top-4 ids / weights and the layer output y (fp32).
* scored_routes.npz — DeepSeek routing (deepseek_v41/moe.py:58-74) at 64 tokens x 64
  experts, top-6: sigmoid with 8 groups / top-3 groups (the C4 selection), sqrt-softplus
  and softmax, each with a selection bias and route_scale 2.5.
* mtp_greedy.npz — greedy acceptance cases (native_qwen.py:395-400) at vocab 4096, with
  integer-valued logits so that rows tie at their maximum.

The weights themselves are not stored: tests regenerate them with
whallm_amd.synthetic from the seed and check the digests.
"""
from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from oracle import moe as M  # noqa: E402
from whallm_amd import synthetic as S  # noqa: E402

C1 = dict(hidden=1024, experts=64, inter=512, k=4, tokens=16, seed=0)


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def c1_inputs():
    """The seeded C1 draws, in order: expert regions, router weight, activations."""
    rng = np.random.default_rng(C1["seed"])
    arrays = S.mxfp4_experts_np(rng, C1["experts"], C1["hidden"], C1["inter"])
    router_bits = S.bf16_normal_np(rng, (C1["experts"], C1["hidden"]), 0.02)
    x_bits = S.bf16_normal_np(rng, (C1["tokens"], C1["hidden"]))
    return arrays, router_bits, x_bits


def c1_fixture() -> dict:
    arrays, router_bits, x_bits = c1_inputs()
    xf = S.bf16_bits_to_f32(x_bits).astype(np.float64)
    logits = (xf @ S.bf16_bits_to_f32(router_bits).astype(np.float64).T).astype(np.float32)
    idx, w = M.route_softmax_topk(logits, C1["k"])
    # The k-th and (k+1)-th logits must be far apart compared with fp32 accumulation
    # error (~1e-6 here), so a device router reproduces the ids bit for bit.
    top = np.sort(logits, axis=1)[:, ::-1]
    assert (top[:, C1["k"] - 1] - top[:, C1["k"]]).min() > 1e-4
    experts = [M.MXFP4Expert(arrays["gate_up"][e], arrays["gate_up_scales"][e], arrays["down"][e],
                             arrays["down_scales"][e]) for e in range(C1["experts"])]
    y = M.combine(M.routed_outputs(xf.astype(np.float32), idx, experts), w)
    out = {f"sha_{name}": np.array(digest(a)) for name, a in arrays.items()}
    out.update(sha_router=np.array(digest(router_bits)), x_bits=x_bits, logits=logits, indices=idx, weights=w,
               y=y.astype(np.float32))
    return out


def scored_fixture() -> dict:
    rng = np.random.default_rng(20261201)
    T, E, K = 64, 64, 6
    out = {"logits": rng.standard_normal((T, E)).astype(np.float32),
           "bias": (rng.standard_normal(E) * 0.1).astype(np.float32)}
    for name, func, groups, top in (("sigmoid_groups", "sigmoid", 8, 3), ("sqrtsoftplus", "sqrtsoftplus", 1, 1),
                                    ("softmax", "softmax", 1, 1)):
        idx, w = M.route_scored(out["logits"], out["bias"], K, func=func, route_scale=2.5, n_groups=groups,
                                topk_groups=top)
        out[f"{name}_indices"], out[f"{name}_weights"] = idx, w.astype(np.float32)
    return out


def mtp_fixture() -> dict:
    rng = np.random.default_rng(4096)
    V, n, cases = 4096, 3, 6
    # integer-valued logits: rows hold ties at their maximum (the lowest index must win)
    logits = rng.integers(-64, 64, size=(cases, n + 1, V)).astype(np.float32)
    drafts = logits[:, :n].argmax(axis=-1).astype(np.int32)
    for c in range(n):                       # case c rejects draft c
        drafts[c, c] = (drafts[c, c] + 7) % V
    logits[4, 0, [11, 2000, 4095]] = 100.0   # a tie across chunks above the row: index 11 wins
    drafts[4, 0] = 11
    drafts[4, 1:] = logits[4, 1:n].argmax(axis=-1)
    expected = np.array([M.verify_greedy(drafts[c], logits[c]) for c in range(cases)], np.int32)
    return {"logits": logits, "drafts": drafts, "expected": expected}


def main() -> None:
    np.savez_compressed(HERE / "c1_layer_seed0.npz", **c1_fixture())
    np.savez_compressed(HERE / "scored_routes.npz", **scored_fixture())
    np.savez_compressed(HERE / "mtp_greedy.npz", **mtp_fixture())
    for f in ("c1_layer_seed0.npz", "scored_routes.npz", "mtp_greedy.npz"):
        print(f, (HERE / f).stat().st_size, "bytes")


if __name__ == "__main__":
    main()
