"""CPU: the NumPy float32 evaluation used in the fp32 ensembles computes the
oracle's function: within fp32 rounding of the float64 oracle on one chunk
(windowed, without a window, ragged T), and far from it when the Omega window
is dropped (a planted mistake)."""

import numpy as np
import pytest

import fp32_eval as FE
import scan_cases as SC
from oracle import atlas_ref as R


@pytest.mark.parametrize("T,w,gamma", [(64, 16, True), (64, 1, False), (40, 8, True)])
def test_fp32_evaluation_matches_oracle(T, w, gamma):
    cs, ns = 64, 5
    inp = SC.make_inputs(1, T, 2, 32, 64, seed=21, with_gamma=gamma, s_scale=0.01)
    args = [inp[k] for k in ("q", "k", "v", "alpha", "eta", "theta", "gamma")]
    y_ref, st_ref = R.memory_scan(*args, inp["state"], cs, w, ns)
    y, st = FE.memory_scan(*args, inp["state"], cs, w, ns)
    assert SC.rel_l2(y, y_ref) <= 1e-4
    for a, b in zip(st, st_ref):
        assert SC.rel_l2(a, b) <= 1e-4


def test_fp32_evaluation_sees_a_dropped_window():
    cs, ns = 64, 5
    inp = SC.make_inputs(1, 64, 2, 32, 64, seed=22)
    args = [inp[k] for k in ("q", "k", "v", "alpha", "eta", "theta", "gamma")]
    y_ref, _ = R.memory_scan(*args, inp["state"], cs, 16, ns)
    y, _ = FE.memory_scan(*args, inp["state"], cs, 1, ns)
    assert SC.rel_l2(y, y_ref) > 1e-3
