"""Loads the committed fixtures of tests/golden/ and the seeded inputs they were made from."""
import importlib.util
import json
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"

_spec = importlib.util.spec_from_file_location("make_fixtures", GOLDEN / "make_fixtures.py")
make_fixtures = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(make_fixtures)


def kats() -> dict:
    return json.loads((GOLDEN / "reference_kats.json").read_text())


def load(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def c1_inputs():
    """(expert arrays, router bf16 bits, x bf16 bits) of the C1 fixture, checked against
    the digests stored with it."""
    arrays, router_bits, x_bits = make_fixtures.c1_inputs()
    fx = load("c1_layer_seed0.npz")
    for name, a in arrays.items():
        assert make_fixtures.digest(a) == str(fx[f"sha_{name}"]), f"seeded {name} drifted from the fixture"
    assert make_fixtures.digest(router_bits) == str(fx["sha_router"]), "seeded router weight drifted"
    assert np.array_equal(x_bits, fx["x_bits"])
    return arrays, router_bits, x_bits, fx
