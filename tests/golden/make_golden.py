"""Writes the golden fixtures of this directory from the float64 oracle.

The reference holds no golden data files (no .npy/.npz/.json) and its JAX
stack is not installed, so the fixtures are the outputs of the oracle
(oracle/atlas_ref.py, itself pinned by closed forms, the per-token brute
force and the reference's known-answer tests), frozen here so that the HIP
path is checked against fixed data and any later change of the oracle is
caught.  Inputs follow the BASELINE config-1 recipe (tests/scan_cases.py:
numpy PCG64(seed); q, k, v ~ N(0,1) with q, k L2-normalised over D; gates =
sigmoid of N(0,1) logits, eta times max_lr 0.1; W1, W2 ~ N(0, 1/D), or the
model initial state W1=0, W2=[I;0]) and are stored with the outputs.

  c1_trajectory.npz  config 1 (B1 T1024 H4 D32 E32 cs64 w16 ns5, seed 0):
                     y and the state at every chunk boundary (float32);
                     the inputs are regenerated from the recipe and checked
                     against the sha256 recorded in golden.json
  scan_cases.npz     small scans (1-3 chunks): D != E, window longer than
                     the chunk, no window, ns 0/1/5, ragged T, the model
                     initial state, E = 256; inputs (rounded to float32
                     before the oracle runs) and the trajectory over the
                     padded length: y and the state at every chunk boundary
                     (float32).  The layer's outputs are its first T rows of
                     y and the last state.
  pe_cases.npz       Polar-Express alone: wide, tall and square, ns 3/5
                     (float32-rounded inputs, float32 outputs)
  golden.json        recipe, semantic choices, shapes and input checksums

Run from the repository root:  python tests/golden/make_golden.py
"""

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
for _p in (ROOT, os.path.join(ROOT, "tests")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import scan_cases as SC  # noqa: E402
from oracle import atlas_ref as R  # noqa: E402

C1 = dict(B=1, T=1024, H=4, D=32, E=32, cs=64, w=16, ns=5, seed=0)

# name: (B, T, H, D, E, cs, w, ns, seed, init, with_gamma, precision the GPU check runs in)
SCAN_CASES = {
    "d32e64_ragged": (1, 40, 2, 32, 64, 16, 4, 5, 11, "rand", True, "f32"),
    "d32e32_w_gt_cs_ns1": (2, 32, 1, 32, 32, 16, 24, 1, 12, "rand", True, "f32"),
    "d64e128_nowindow_ns0": (1, 24, 1, 64, 128, 8, 1, 0, 13, "rand", False, "f32"),
    "d64e64_model_init": (1, 48, 2, 64, 64, 16, 8, 5, 14, "model", True, "f32"),
    "d64e256_c3_shape": (1, 64, 1, 64, 256, 64, 64, 5, 15, "rand", True, "f16"),
}

# name: (shape, ns, seed)
PE_CASES = {
    "wide_64x128": ((2, 64, 128), 5, 21),
    "tall_128x64": ((2, 128, 64), 5, 22),
    "square_64": ((2, 64, 64), 5, 23),
    "wide_32x64_ns3": ((4, 32, 64), 3, 24),
}

INPUT_KEYS = ("q", "k", "v", "alpha", "eta", "theta", "gamma")


def input_digest(inp):
    """sha256 over the float64 bytes of the inputs and initial state."""
    h = hashlib.sha256()
    for k in INPUT_KEYS:
        if inp[k] is not None:
            h.update(np.ascontiguousarray(inp[k], np.float64).tobytes())
    for s in inp["state"]:
        h.update(np.ascontiguousarray(s, np.float64).tobytes())
    return h.hexdigest()


def c1_inputs():
    c = C1
    return SC.make_inputs(c["B"], c["T"], c["H"], c["D"], c["E"], seed=c["seed"])


def _f32(a):
    return None if a is None else np.asarray(a, np.float32).astype(np.float64)


def scan_case_inputs(name):
    """The recipe's inputs rounded to float32 (what is stored and what the
    oracle consumes)."""
    B, T, H, D, E, cs, w, ns, seed, init, wg, _ = SCAN_CASES[name]
    inp = SC.make_inputs(B, T, H, D, E, seed=seed, init=init, with_gamma=wg, s_scale=0.05)
    out = {k: _f32(inp[k]) for k in INPUT_KEYS}
    out["state"] = tuple(_f32(s) for s in inp["state"])
    return out


def pe_case_input(name):
    shape, ns, seed = PE_CASES[name]
    return _f32(np.random.Generator(np.random.PCG64(seed)).standard_normal(shape))


def main():
    meta = {
        "generator": "tests/golden/make_golden.py from oracle/atlas_ref.py (float64)",
        "recipe": "tests/scan_cases.py make_inputs: numpy PCG64(seed); q,k,v ~ N(0,1), q,k L2-normalised over D; "
                  "alpha,theta,gamma = sigmoid(N(0,1)), eta = sigmoid(N(0,1))*0.1; W ~ N(0,1/D) ('rand', "
                  "S ~ 0.05 N(0,1) for the small cases, S = 0 for config 1) or W1=0, W2=[I;0], S=0 ('model'); "
                  "gates and state rounded to float32",
        "semantics": "memory forward with the tanh GELU, u_W2 with the erf GELU derivative, scale 2/D, Omega "
                     "window within the chunk, padding alpha=1 eta=theta=gamma=0 q=k=v=0, read-out with the tanh "
                     "GELU, Polar-Express coefficients memory_layer.py:34-40 with 1e-12 / 1.01 / 1e-6",
    }
    c = C1
    inp = c1_inputs()
    y, states = SC.oracle_trajectory(inp, c["cs"], c["w"], c["ns"])
    st = [np.stack([s[m] for s in states]).astype(np.float32) for m in range(4)]
    np.savez_compressed(os.path.join(HERE, "c1_trajectory.npz"), y=y.astype(np.float32),
                        W1=st[0], W2=st[1], S1=st[2], S2=st[3])
    meta["c1_trajectory"] = dict(C1, input_sha256=input_digest(inp),
                                 arrays="y (B,T,H,D); W1,W2,S1,S2 (n_chunks+1, B, H, ...) at every chunk boundary")

    arrays = {}
    meta["scan_cases"] = {}
    for name, (B, T, H, D, E, cs, w, ns, seed, init, wg, prec) in SCAN_CASES.items():
        inp = scan_case_inputs(name)
        padded = dict(zip(INPUT_KEYS, R._pad_inputs(*(inp[k] for k in INPUT_KEYS), cs)), state=inp["state"])
        y, states = SC.oracle_trajectory(padded, cs, w, ns)
        for k in INPUT_KEYS:
            if inp[k] is not None:
                arrays[f"{name}/{k}"] = inp[k].astype(np.float32)
        for m, s in zip(("W1_0", "W2_0", "S1_0", "S2_0"), inp["state"]):
            arrays[f"{name}/{m}"] = s.astype(np.float32)
        arrays[f"{name}/traj_y"] = y.astype(np.float32)
        for j, m in enumerate(("W1", "W2", "S1", "S2")):
            arrays[f"{name}/traj_{m}"] = np.stack([s[j] for s in states]).astype(np.float32)
        meta["scan_cases"][name] = dict(B=B, T=T, H=H, D=D, E=E, cs=cs, w=w, ns=ns, seed=seed, init=init,
                                        with_gamma=wg, gpu_precision=prec, input_sha256=input_digest(inp))
    np.savez_compressed(os.path.join(HERE, "scan_cases.npz"), **arrays)

    arrays = {}
    meta["pe_cases"] = {}
    for name, (shape, ns, seed) in PE_CASES.items():
        X = pe_case_input(name)
        arrays[f"{name}/X"] = X.astype(np.float32)
        arrays[f"{name}/P"] = R.polar_express(X, ns).astype(np.float32)
        meta["pe_cases"][name] = dict(shape=list(shape), ns=ns, seed=seed)
    np.savez_compressed(os.path.join(HERE, "pe_cases.npz"), **arrays)

    with open(os.path.join(HERE, "golden.json"), "w") as f:
        json.dump(meta, f, indent=1)
        f.write("\n")


if __name__ == "__main__":
    main()
