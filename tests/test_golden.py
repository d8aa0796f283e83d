"""The committed golden fixtures (tests/golden/attn_golden.npz, written by tests/golden/make_golden.py): the
seeded inputs still hash to what the fixtures were made from, and the oracle still reproduces the stored outputs.
A change to a generator, to the rounding or to the oracle's arithmetic shows up here."""
import os

import numpy as np
import pytest

import cases

FIX = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "attn_golden.npz"))


@pytest.mark.parametrize("mk", cases.CASES, ids=lambda f: f.__name__)
def test_fixture_inputs_and_oracle(mk):
    c = mk()
    assert str(FIX[c["name"] + ".hash"]) == c["hash"], "inputs changed"
    o, lse = cases.oracle_of(c)
    eo = FIX[c["name"] + ".o"].astype(np.float64); el = FIX[c["name"] + ".lse"].astype(np.float64)
    assert np.abs(o - eo).max() <= 1e-6 * max(1.0, np.abs(eo).max())
    assert np.abs(lse - el).max() <= 1e-6 * max(1.0, np.abs(el).max())
