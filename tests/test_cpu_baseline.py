"""CPU: the benchmark's CPU baseline (oracle/cpu_baseline.py, the torch-CPU
restatement of the reference's non-fused chunk loop that bench.py times)
computes the same function as the float64 oracle (oracle/atlas_ref.py), so
the reported speed-up divides by the same work.  Evaluated in float64 the two
agree to rounding (1e-10 rel-L2) on a two-chunk scan with an Omega window,
without a window, and on a ragged-free D != E shape; in float32, as bench.py
runs it, within the fp32 bar 1e-4 on one chunk."""

import numpy as np
import pytest
import torch

import scan_cases as SC
from oracle import atlas_ref as R
from oracle import cpu_baseline as CB


def _run(inp, cs, w, ns, dtype):
    def t(a):
        return None if a is None else torch.tensor(np.asarray(a), dtype=dtype)
    st = tuple(t(s) for s in inp["state"])
    y, fin = CB.memory_scan(t(inp["q"]), t(inp["k"]), t(inp["v"]), t(inp["alpha"]), t(inp["eta"]),
                            t(inp["theta"]), t(inp["gamma"]), st, cs, w, ns)
    return y.double().numpy(), [s.double().numpy() for s in fin]


@pytest.mark.parametrize("D,E,w,gamma", [(32, 64, 8, True), (32, 32, 1, False), (16, 48, 16, True)])
def test_cpu_baseline_equals_oracle_float64(D, E, w, gamma):
    cs, ns = 16, 5
    inp = SC.make_inputs(1, 2 * cs, 2, D, E, seed=13, with_gamma=gamma, s_scale=0.01)
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = _run(inp, cs, w, ns, torch.float64)
    assert SC.rel_l2(y, y_ref) <= 1e-10
    for a, b in zip(st, st_ref):
        assert SC.rel_l2(a, b) <= 1e-10


def test_cpu_baseline_float32_within_fp32_bar():
    cs, w, ns = 64, 32, 5
    inp = SC.make_inputs(1, cs, 2, 64, 128, seed=14, io="bf16")
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = _run(inp, cs, w, ns, torch.float32)
    assert SC.rel_l2(y, y_ref) <= 1e-4
    for a, b in zip(st, st_ref):
        assert SC.rel_l2(a, b) <= 1e-4


def test_cpu_baseline_catches_a_planted_mistake(monkeypatch):
    """The float64 comparison is tight enough to see a dropped Omega window."""
    cs, w, ns = 16, 8, 5
    inp = SC.make_inputs(1, cs, 2, 32, 64, seed=15)
    y_ref, _ = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                             inp["gamma"], inp["state"], cs, w, ns)
    y, _ = _run(inp, cs, 1, ns, torch.float64)   # window 1: no Omega aggregation
    assert SC.rel_l2(y, y_ref) > 1e-6
