"""The oracle against the committed fixtures (tests/golden/), CPU only.

reference_kats.json holds vectors transcribed from the reference's own tests; the .npz
fixtures were written by tests/golden/make_fixtures.py from the oracle and pin it
against drift (a change to the oracle or to the seeded generators fails here)."""
import numpy as np

from golden_data import c1_inputs, kats, load, make_fixtures
from oracle import c_oracle as C
from oracle import formats as F
from oracle import moe as M


def test_stable_topk_kat():
    kat = kats()["stable_topk"]
    s = np.array(kat["scores"], np.float32)
    assert M.topk_desc(s, kat["k"]).tolist() == kat["indices"]
    assert C.topk(s, kat["k"]).tolist() == kat["indices"]


def test_constant_experts_kat_through_the_oracle_formats():
    # test_runtime.py:2509-2745: mx.quantize of constant 32x32 matrices, activation = up,
    # x = ones: expert outputs 1024 * w3 * w2, stacked in router order [1, 0].
    kat = kats()["constant_experts"]
    n = kat["size"]

    def restore(value):
        bits = (np.full(n * n, np.float32(value)).view(np.uint32) >> 16).astype(np.uint16)
        w, s = F.quantize_mxfp4_bf16(bits, n, n)
        return F.dequant_mxfp4(np.ascontiguousarray(w).view(np.uint32).reshape(n, -1), s)

    x = np.ones((1, n), np.float32)
    out = []
    for e in kat["selected"]:
        ex = kat["experts"][e]
        out.append(((x @ restore(ex["w3"]).T) @ restore(ex["w2"]).T)[0])
    for row, want in zip(out, kat["outputs"]):
        assert np.all(row == want)


def test_c1_fixture_reproduces():
    c1_inputs()  # digests of the seeded weights
    want = load("c1_layer_seed0.npz")
    got = make_fixtures.c1_fixture()
    for key in ("logits", "indices", "weights", "y"):
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)


def test_scored_routes_fixture_reproduces():
    want = load("scored_routes.npz")
    got = make_fixtures.scored_fixture()
    for key in want:
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)


def test_mtp_fixture_reproduces():
    want = load("mtp_greedy.npz")
    got = make_fixtures.mtp_fixture()
    for key in want:
        np.testing.assert_array_equal(got[key], want[key], err_msg=key)
    assert want["expected"][4].tolist() == [3, int(np.argmax(want["logits"][4, 3]))]
