"""CPU: the closed-form chunk decomposition the HIP kernels evaluate
(tests/chunk_algebra.py: momentum via c[t,i] coefficients, slice partial sums
L_j, per-slice read-out) reproduces the oracle's sequential chunk loop."""

import numpy as np
import pytest

import chunk_algebra as CA
import scan_cases as SC
from oracle import atlas_ref as R


@pytest.mark.parametrize("w,gamma,n_slices", [(1, False, 1), (3, True, 2), (8, True, 4), (20, True, 2),
                                              (4, False, 4)])
def test_decomposition_matches_oracle(w, gamma, n_slices):
    inp = SC.make_inputs(1, 32, 2, 8, 16, seed=w * 10 + n_slices, with_gamma=gamma, s_scale=0.01)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"], inp["state"],
            8, w, 5)
    y, st = R.memory_scan(*args)
    y2, st2 = CA.scan(*args[:8], 8, w, 5, n_slices)
    assert SC.rel_l2(y2, y) < 1e-11
    for a, b in zip(st2, st):
        assert SC.rel_l2(a, b) < 1e-11


def test_coefficients_closed_form():
    """c[t,i] from the suffix-sum form equals the direct double sum."""
    rng = np.random.default_rng(0)
    cs, w, D = 12, 5, 8
    th, et, ga = rng.uniform(0.2, 0.9, cs), rng.uniform(0, 0.1, cs), rng.uniform(0, 1, cs)
    c, Theta, A, a = CA.chunk_coefficients(rng.uniform(0.2, 0.9, cs), et, th, ga, w, D)
    for t in range(cs):
        for i in range(cs):
            ref = 0.0
            if i <= t:
                for s in range(i, min(t, i + w - 1) + 1):
                    ref += np.prod(th[s + 1:t + 1]) * (-et[s])
                ref *= ga[i] * 2.0 / D
            assert abs(c[t, i] - ref) < 1e-15
