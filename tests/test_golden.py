"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py): integrity and
oracle reproduction on the CPU.

The fixtures hold seeded inputs and the outputs of the f32 CPU oracle at generation time,
cross-checked there against an independent numpy float64 restatement (manifest.json records the
distance). These tests pin the oracle against drift: every fixture must still hash to its
manifest entry and the oracle must reproduce its expected outputs bit for bit.
"""
import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"
MANIFEST = json.loads((GOLDEN / "manifest.json").read_text())


def load(name):
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_fixture_integrity(name):
    entry = MANIFEST[name]
    data = (GOLDEN / f"{name}.npz").read_bytes()
    assert hashlib.sha256(data).hexdigest() == entry["sha256"]
    a = load(name)
    assert {k: list(v.shape) for k, v in a.items()} == entry["arrays"]
    assert all(v.dtype == (np.float64 if k.endswith("_f64") else np.float32) for k, v in a.items())
    if "numpy_norm_err" in entry:
        assert entry["numpy_norm_err"] <= 1e-5


def oracle_outputs(name, a):
    """The oracle's outputs for fixture `name` (dict of array name -> array)."""
    if name.startswith("kat_matmul") or name == "matmul_small":
        return {"expected": oracle.matmul(a["A"], a["B"])}
    if name == "mamba_mlp_c1":
        return {"expected": oracle.mamba_mlp(a["X"], a["Wg"], a["bg"], a["Wo"], a["bo"])}
    if name.startswith("s4_ref"):
        return {"expected": oracle.s4_ref_fwd(a["x"], a["a_real"], a["a_imag"], a["B"], a["C"], a["D"])}
    if name.startswith("scan"):
        out, last = oracle.selective_scan(
            a["u"], a["delta"], a["A"], a["B"], a["C"], a.get("D"), a.get("z"), a.get("dt_bias"),
            delta_softplus=MANIFEST[name]["delta_softplus"], return_last_state=True)
        return {"expected": out, "expected_last_state": last}
    if name == "s4d_small":
        keys = ("x", "dt", "a_re", "a_im", "B_re", "B_im", "C_re", "C_im", "D")
        return {"expected": oracle.s4d_complex(*(a[k] for k in keys)).astype(np.float32)}
    if name == "rmsnorm_small":
        return {"expected": oracle.rmsnorm(a["X"], a["w"], 1e-5)}
    if name == "conv1d_small":
        return {"expected": oracle.conv1d_silu(a["x"], a["w"], a["bias"])}
    raise KeyError(name)


@pytest.mark.parametrize("name", [n for n in sorted(MANIFEST) if n.startswith("scan")])
def test_oracle_state_within_bar_of_float64(name):
    """The f32 oracle's final state against the float64 one the GPU state is held to."""
    from tests.util import rel_err
    a = load(name)
    assert rel_err(a["expected_last_state"], a["expected_last_state_f64"]) <= 1e-4


@pytest.mark.parametrize("name", sorted(MANIFEST))
def test_oracle_reproduces_fixture(name):
    a = load(name)
    for k, v in oracle_outputs(name, a).items():
        assert np.array_equal(v, a[k]), (name, k, float(np.abs(v - a[k]).max()))


def test_reference_kat_fixture_values():
    """The reference's own known answer: ones[2,3] . ones[3,4] == 3 everywhere."""
    a = load("kat_matmul_ones")
    assert np.all(a["expected"] == 3.0)
