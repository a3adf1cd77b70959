"""The committed golden fixtures (tests/golden/*.npz) through the HIP path.

Each fixture holds seeded inputs and the oracle's outputs (written by
tests/golden/make_golden.py; tests/test_oracle.py checks that the oracle
still reproduces them). Here the GPU entry points get the stored inputs and
are compared with the stored outputs, without the oracle in the loop:
router fixtures through both C entry points (`topk_softmax` and the host
`apply_topk_softmax_inplace`), indices bit-exact and weights within 1e-6
relative; MoE fixtures through `FusedMoE::forward` and the raw `fused_moe`
symbol into a zeroed output, against both stored oracle outputs (f64 and
f32 accumulation) at the dtype's tolerance (rtol 1e-4 f32, 1e-2 f16,
2e-2 bf16, atol = rtol * RMS).
"""
import os

import numpy as np
import pytest

from helpers import RTOL, assert_close
from test_gpu_moe import run_moe, run_raw
from test_gpu_topk import run_router

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")
FILES = sorted(f for f in os.listdir(GOLDEN) if f.endswith(".npz"))
ROUTER = [f for f in FILES if f.startswith("router_")]
MOE = [f for f in FILES if f.startswith("moe_")]


def _load(name):
    return np.load(os.path.join(GOLDEN, name), allow_pickle=False)


def test_fixture_set_is_complete():
    assert ROUTER and MOE and len(ROUTER) + len(MOE) == len(FILES)


@pytest.mark.parametrize("name", ROUTER)
@pytest.mark.parametrize("api", ["host", "raw"])
def test_router_fixture(name, api):
    z = _load(name)
    assert str(z["kind"]) == "router"
    w, i, ei = run_router(z["logits"], int(z["k"]), api)
    assert np.array_equal(i, z["topk_indices"]), name
    assert np.array_equal(ei, z["token_expert_indices"]), name
    want = z["topk_weight"]
    rel = np.abs(w - want) / np.maximum(np.abs(want), 1e-30)
    assert rel.max() <= 1e-6, f"{name}: weights differ by {rel.max():.3g} relative"


@pytest.mark.parametrize("name", MOE)
@pytest.mark.parametrize("entry", ["forward", "raw"])
def test_moe_fixture(name, entry):
    z = _load(name)
    assert str(z["kind"]) == "moe"
    dt, E, k = int(z["dtype"]), int(z["E"]), int(z["k"])
    act, mt = int(z["act"]), int(z["moe_type"])
    down = z["down"] if z["down"].size else None
    args = (z["x"], z["gate"], z["up"], down, z["routing_weights"], z["expert_indices"], E, k, act, mt, dt)
    got = run_moe(*args) if entry == "forward" else run_raw(*args)
    assert np.isfinite(got).all(), name
    assert_close(got, z["out_exact"], RTOL[dt], f"{name} vs stored f64 oracle output")
    assert_close(got, z["out_f32acc"], RTOL[dt], f"{name} vs stored f32-accumulation output")
