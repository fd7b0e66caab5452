"""GPU: the HIP path (through the C ABI) against the committed golden
fixtures (tests/golden/, float64 oracle outputs stored as float32).

  - small scans (1-3 chunks), every chunk teacher-forced from the stored
    chunk-start state: fp32 compute within rel-L2 1e-4, the E = 256 case in
    the fp16-MFMA mode within 2e-2 (E = 256 has no fp32 kernel); and end to
    end from the initial state, where the recurrence's amplification of
    rounding is allowed for: 1e-3 in fp32 (the oracle itself evaluated in
    fp32 is already up to 1e-4 off float64 after three chunks), 2e-2 in
    fp16 mode;
  - config 1 over all 16 chunks, teacher-forced from the stored chunk-start
    states (every chunk an independent stream of one call): each chunk's y
    and end state within 1e-4 (fp32) / 2e-2 (fp16 mode);
  - Polar-Express alone (wide, tall, square): fp32 within 1e-4.
Every expected value comes from the stored fixtures; the oracle is not run."""

import os

import numpy as np
import pytest

import scan_cases as SC
from golden import make_golden as MG

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TOL = {"f32": 1e-4, "f16": 2e-2}


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _scan(inp, cs, w, ns, precision):
    torch = _torch()
    from atlas_amd import DeepMemoryState, memory_scan

    def t(a):
        return None if a is None else torch.tensor(np.asarray(a, np.float32), device="cuda")

    y, st = memory_scan(t(inp["q"]), t(inp["k"]), t(inp["v"]), t(inp["alpha"]), t(inp["eta"]), t(inp["theta"]),
                        t(inp["gamma"]), DeepMemoryState(*(t(s) for s in inp["state"])), cs, w, ns,
                        precision=precision)
    torch.cuda.synchronize()
    return y.cpu().numpy(), [s.cpu().numpy() for s in st]


E2E_TOL = {"f32": 1e-3, "f16": 2e-2}
MATS = ("W1", "W2", "S1", "S2")


def _pad(a, T_pad, val):
    if a is None or a.shape[1] == T_pad:
        return a
    fill = np.full((a.shape[0], T_pad - a.shape[1], *a.shape[2:]), val, a.dtype)
    return np.concatenate([a, fill], axis=1)


@pytest.mark.parametrize("name", list(MG.SCAN_CASES))
def test_scan_case(name):
    B, T, H, D, E, cs, w, ns, seed, init, wg, prec = MG.SCAN_CASES[name]
    z = np.load(os.path.join(GOLD, "scan_cases.npz"))
    inp = {k: (z[f"{name}/{k}"] if f"{name}/{k}" in z else None) for k in MG.INPUT_KEYS}
    inp["state"] = tuple(z[f"{name}/{m}"] for m in ("W1_0", "W2_0", "S1_0", "S2_0"))
    y_traj = z[f"{name}/traj_y"]
    traj = [z[f"{name}/traj_{m}"] for m in MATS]
    nc = y_traj.shape[1] // cs
    states = [tuple(t[c].astype(np.float64) for t in traj) for c in range(nc + 1)]

    print(f"golden scan case {name} ({prec}), teacher-forced", flush=True)
    T_pad = nc * cs
    padded = {k: _pad(inp[k], T_pad, 1.0 if k == "alpha" else 0.0) for k in MG.INPUT_KEYS}
    tf = SC.teacher_forced_inputs(padded, states, cs)
    y, st = _scan(tf, cs, w, ns, prec)
    errs = SC.worst_chunk_errors(y, st, y_traj, states, B, nc, cs)
    print(name, "per chunk", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= TOL[prec], f"{name}: chunk {k} rel-L2 {v:.3e}"

    print(f"golden scan case {name} ({prec}), end to end", flush=True)
    y, st = _scan(inp, cs, w, ns, prec)
    errs = {"y": SC.rel_l2(y, y_traj[:, :T])}
    for m, s, t in zip(MATS, st, traj):
        errs[m] = SC.rel_l2(s, t[-1])
    print(name, "end to end", {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= E2E_TOL[prec], f"{name}: {k} rel-L2 {v:.3e}"


@pytest.mark.parametrize("precision", ["f32", "f16"])
def test_c1_teacher_forced_against_fixture(precision):
    c = MG.C1
    z = np.load(os.path.join(GOLD, "c1_trajectory.npz"))
    inp = MG.c1_inputs()
    nc = c["T"] // c["cs"]
    states = [tuple(z[m][j].astype(np.float64) for m in ("W1", "W2", "S1", "S2")) for j in range(nc + 1)]
    tf = SC.teacher_forced_inputs(inp, states, c["cs"])
    print(f"golden C1 teacher-forced ({precision})", flush=True)
    y, st = _scan(tf, c["cs"], c["w"], c["ns"], precision)
    errs = SC.worst_chunk_errors(y, st, z["y"], states, c["B"], nc, c["cs"])
    print("C1", precision, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= TOL[precision], f"{k} rel-L2 {v:.3e}"


@pytest.mark.parametrize("name", list(MG.PE_CASES))
def test_pe_case(name):
    torch = _torch()
    from atlas_amd import polar_express
    shape, ns, seed = MG.PE_CASES[name]
    z = np.load(os.path.join(GOLD, "pe_cases.npz"))
    X = torch.tensor(z[f"{name}/X"], device="cuda")
    print(f"golden PE case {name}", flush=True)
    P = polar_express(X, ns, precision="f32")
    torch.cuda.synchronize()
    e = SC.rel_l2(P.cpu().numpy(), z[f"{name}/P"])
    print(f"PE {name}: rel-L2 {e:.2e}", flush=True)
    assert e <= 1e-4
