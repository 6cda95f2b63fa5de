"""The committed fixtures of tests/golden/ are what the oracle produces (CPU).

Regenerates every case of tests/golden/make_golden.py and compares: the input
hash and the shader-order outputs must match bit for bit, the double-precision
outputs to 1e-12.  A drift in the RNG, RoPE tables, cache write or either
attention oracle shows up here before any GPU comparison uses the fixtures.
"""
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN

sys.path.insert(0, GOLDEN)
import make_golden  # noqa: E402


@pytest.mark.parametrize("name", sorted(make_golden.CASES))
def test_fixture_reproduces(name):
    ref = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    new = make_golden.CASES[name]()
    assert str(ref["input_sha"]) == new["input_sha"]
    np.testing.assert_array_equal(ref["out_wgsl"], new["out_wgsl"])
    np.testing.assert_allclose(ref["out_f64"], new["out_f64"], rtol=0, atol=1e-12)
    if name.startswith("q4k"):
        np.testing.assert_array_equal(ref["blocks"], new["blocks"])
        np.testing.assert_array_equal(ref["dequant"], new["dequant"])
        # f32 rounding of a K-term sum, relative to the terms' magnitude
        # (|x| <= 4 for these seeds)
        mag = np.abs(ref["dequant"]).sum(axis=1).max() * 4.0
        assert np.abs(ref["out_wgsl"] - ref["out_f64"]).max() < 1e-5 * mag
    elif name.startswith("depformer_chain"):
        np.testing.assert_array_equal(ref["tokens"], new["tokens"])
        # f32 through 2 layers x 4 steps of GEMMs, norms and attention
        assert np.abs(ref["out_wgsl"] - ref["out_f64"]).max() < 2e-5 * np.abs(ref["out_f64"]).max()
    else:
        # The two oracles agree with each other within f32 rounding.
        assert np.abs(ref["out_wgsl"] - ref["out_f64"]).max() < 2e-6
