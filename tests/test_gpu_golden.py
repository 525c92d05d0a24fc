"""The HIP path against the committed fixtures (tests/golden/): C1's layer (BASELINE
configs[0], seed 0), DeepSeek scored routing and greedy MTP acceptance.

Top-k ids and acceptance results must match bit for bit; the layer output is held to
relative L2 <= 1e-2 and max |err| <= 2e-2 * max |ref| of the fixture's fp32 oracle output."""
from types import SimpleNamespace

import numpy as np
import pytest
import torch

import whallm_amd as wa
from golden_data import c1_inputs, load
from whallm_amd import operators as O
from whallm_amd import synthetic as S

pytestmark = pytest.mark.gpu


def close(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    assert np.all(np.isfinite(got)), what
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    mx = np.abs(got - want).max() / np.abs(want).max()
    assert rel <= 1e-2 and mx <= 2e-2, f"{what}: rel L2 {rel:.3e} max {mx:.3e}"


def test_c1_layer_matches_fixture(device):
    arrays, router_bits, x_bits, fx = c1_inputs()
    table = S.experts_to_device(arrays, device)
    x = S.bf16_bits_to_tensor(x_bits, device)
    router = S.bf16_bits_to_tensor(router_bits, device)
    logits = wa.linear_bf16(x, router)
    idx, w = wa.route_softmax_topk(logits, 4)
    y = wa.moe_mxfp4(x, idx, w, table)
    torch.cuda.synchronize()
    np.testing.assert_allclose(logits.cpu().numpy(), fx["logits"], rtol=1e-5, atol=1e-5)
    assert np.array_equal(idx.cpu().numpy(), fx["indices"])
    np.testing.assert_allclose(w.cpu().numpy(), fx["weights"], rtol=1e-5, atol=1e-6)
    close(y.float().cpu().numpy(), fx["y"], "C1 layer")


def test_c1_sparse_moe_operator_matches_fixture(device):
    arrays, router_bits, x_bits, fx = c1_inputs()
    table = S.experts_to_device(arrays, device)
    args = SimpleNamespace(hidden_size=1024, num_experts=64, shared_expert_intermediate_size=512,
                           num_experts_per_tok=4, norm_topk_prob=True)
    moe = O.SparseMoE(args, 0, SimpleNamespace(current_batched=lambda _l: table), device=device)
    moe.gate.weight = S.bf16_bits_to_tensor(router_bits, device)
    moe.shared_expert = None
    x = S.bf16_bits_to_tensor(x_bits, device).view(1, 16, 1024)
    probabilities, indices = moe.route(x)
    y = moe(x, (probabilities, indices))
    torch.cuda.synchronize()
    assert np.array_equal(indices.cpu().numpy().reshape(16, 4), fx["indices"])
    close(y.float().cpu().numpy().reshape(16, 1024), fx["y"], "C1 SparseMoE")


@pytest.mark.parametrize("name,func,groups,top", [("sigmoid_groups", "sigmoid", 8, 3),
                                                  ("sqrtsoftplus", "sqrtsoftplus", 1, 1),
                                                  ("softmax", "softmax", 1, 1)])
def test_scored_routes_match_fixture(device, name, func, groups, top):
    fx = load("scored_routes.npz")
    idx, w = wa.route_scored(torch.from_numpy(fx["logits"]).to(device), torch.from_numpy(fx["bias"]).to(device), 6,
                             func=func, route_scale=2.5, n_groups=groups, topk_groups=top)
    torch.cuda.synchronize()
    assert np.array_equal(idx.cpu().numpy(), fx[f"{name}_indices"])
    np.testing.assert_allclose(w.cpu().numpy(), fx[f"{name}_weights"], rtol=1e-5, atol=1e-6)


def test_mtp_greedy_matches_fixture(device):
    fx = load("mtp_greedy.npz")
    for c in range(fx["logits"].shape[0]):
        out = wa.mtp_verify_greedy(torch.from_numpy(fx["logits"][c]).to(device),
                                   torch.from_numpy(fx["drafts"][c]).to(device))
        assert out.cpu().tolist() == fx["expected"][c].tolist(), c
