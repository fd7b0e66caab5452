"""CPU: the committed golden fixtures (tests/golden/) against their recipe and
the oracle.  The inputs regenerate bit for bit from the recorded recipe
(sha256 in golden.json), the float64 oracle reproduces every stored output
to float32 storage precision, and the fixtures discriminate: an oracle with
a planted mistake (Omega window dropped, one Newton-Schulz step fewer, a
transposed weight) misses them by far more than any tolerance."""

import json
import os

import numpy as np
import pytest

import __graft_entry__  # noqa: F401  (sets sys.path)
import scan_cases as SC
from oracle import atlas_ref as R
from golden import make_golden as MG

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _meta():
    with open(os.path.join(GOLD, "golden.json")) as f:
        return json.load(f)


def _scan_case(z, name):
    inp = {k: (z[f"{name}/{k}"].astype(np.float64) if f"{name}/{k}" in z else None) for k in MG.INPUT_KEYS}
    inp["state"] = tuple(z[f"{name}/{m}"].astype(np.float64) for m in ("W1_0", "W2_0", "S1_0", "S2_0"))
    T = inp["q"].shape[1]
    out = (z[f"{name}/traj_y"][:, :T], tuple(z[f"{name}/traj_{m}"][-1] for m in ("W1", "W2", "S1", "S2")))
    return inp, out


def test_c1_inputs_regenerate_from_recipe():
    assert MG.input_digest(MG.c1_inputs()) == _meta()["c1_trajectory"]["input_sha256"]


def test_c1_oracle_reproduces_trajectory():
    c = MG.C1
    z = np.load(os.path.join(GOLD, "c1_trajectory.npz"))
    y, states = SC.oracle_trajectory(MG.c1_inputs(), c["cs"], c["w"], c["ns"])
    assert SC.rel_l2(z["y"], y) <= 1e-6
    for m, name in enumerate(("W1", "W2", "S1", "S2")):
        for j, s in enumerate(states):
            assert SC.rel_l2(z[name][j], s[m]) <= 1e-6, (name, j)


@pytest.mark.parametrize("name", list(MG.SCAN_CASES))
def test_scan_case_inputs_and_outputs(name):
    meta = _meta()["scan_cases"][name]
    z = np.load(os.path.join(GOLD, "scan_cases.npz"))
    inp, (y_g, st_g) = _scan_case(z, name)
    regen = MG.scan_case_inputs(name)
    assert MG.input_digest(regen) == meta["input_sha256"]
    for k in MG.INPUT_KEYS:
        if regen[k] is not None:
            np.testing.assert_array_equal(inp[k], regen[k])
    y, st = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"],
                          inp["state"], meta["cs"], meta["w"], meta["ns"])
    assert SC.rel_l2(y_g, y) <= 1e-6
    for a, b in zip(st_g, st):
        assert SC.rel_l2(a, b) <= 1e-6
    # every stored chunk-boundary state is the oracle's
    padded = dict(zip(MG.INPUT_KEYS, R._pad_inputs(*(inp[k] for k in MG.INPUT_KEYS), meta["cs"])),
                  state=inp["state"])
    y_p, states = SC.oracle_trajectory(padded, meta["cs"], meta["w"], meta["ns"])
    assert SC.rel_l2(z[f"{name}/traj_y"], y_p) <= 1e-6
    for j, m in enumerate(("W1", "W2", "S1", "S2")):
        for c, s in enumerate(states):
            assert SC.rel_l2(z[f"{name}/traj_{m}"][c], s[j]) <= 1e-6, (m, c)


@pytest.mark.parametrize("name", list(MG.PE_CASES))
def test_pe_case(name):
    shape, ns, seed = MG.PE_CASES[name]
    z = np.load(os.path.join(GOLD, "pe_cases.npz"))
    np.testing.assert_array_equal(z[f"{name}/X"], MG.pe_case_input(name))
    assert SC.rel_l2(z[f"{name}/P"], R.polar_express(z[f"{name}/X"].astype(np.float64), ns)) <= 1e-6
    # and the SVD closed form U p(S/s) V^T agrees with the stored output
    assert SC.rel_l2(z[f"{name}/P"], R.polar_express_svd(z[f"{name}/X"].astype(np.float64), ns)) <= 1e-6


def test_fixtures_catch_planted_mistakes():
    name = "d32e64_ragged"
    meta = _meta()["scan_cases"][name]
    z = np.load(os.path.join(GOLD, "scan_cases.npz"))
    inp, (y_g, _) = _scan_case(z, name)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"])
    cs, w, ns = meta["cs"], meta["w"], meta["ns"]
    wrong = [
        R.memory_scan(*args, inp["state"], cs, 1, ns)[0],                       # Omega window dropped
        R.memory_scan(*args, inp["state"], cs, w, ns - 1)[0],                   # one NS step fewer
        R.memory_scan(*args, (inp["state"][0], np.swapaxes(inp["state"][0], -1, -2), *inp["state"][2:]),
                      cs, w, ns)[0],                                            # W2 := W1^T
    ]
    for y in wrong:
        assert SC.rel_l2(y, y_g) > 1e-3
