"""CPU: why the fp16 compute mode uses fp16 (not bf16) matrix-core operands.

The float64 oracle's chunk body is run with a Polar-Express whose products
take their operands rounded to bf16 or to fp16 (fp32 accumulation, fp32
master X, the b*A term kept in fp32 -- the rounding points of the HIP
kernel's Polar-Express).  On the C2 shape (D=64, E=128, chunk 64, window
32) Polar-Express alone costs about 1e-2 relative L2 per chunk with bf16
operands, half of the 2e-2 budget before any other rounding, and about
8x less with fp16 operands, which run at the same MFMA rate.
"""

import numpy as np
import pytest

import scan_cases as SC
from oracle import atlas_ref as R


def _round(x, kind):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32))
    t = t.to(torch.bfloat16) if kind == "bf16" else t.to(torch.float16)
    return t.float().numpy().astype(np.float64)


def _f32(a):
    return np.asarray(a, np.float32).astype(np.float64)


def _pe_rounded(kind):
    def pe(X, steps=5):
        X = _f32(X)
        X = _f32(X / (np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True) + 1e-12) * 1.01 + 1e-6))
        tall = X.shape[-2] > X.shape[-1]
        if tall:
            X = np.swapaxes(X, -1, -2)
        for a, b, c in R.PE_COEFFS[:steps]:
            Xr = _round(X, kind)
            A = _f32(Xr @ np.swapaxes(Xr, -1, -2))
            Ar = _round(A, kind)
            Bm = _f32(b * A + c * _f32(Ar @ Ar))
            X = _f32(a * X + _f32(_round(Bm, kind) @ Xr))
        return np.swapaxes(X, -1, -2) if tall else X
    return pe


def _chunk_errors(monkeypatch, state, args, kind):
    ref = R.process_chunk_deep(state, *args)
    with monkeypatch.context() as m:
        m.setattr(R, "polar_express", _pe_rounded(kind))
        out = R.process_chunk_deep(state, *args)
    return max([SC.rel_l2(out[0], ref[0])] + [SC.rel_l2(a, b) for a, b in zip(out[1][:2], ref[1][:2])])


@pytest.mark.parametrize("init,chunk", [("rand", 0), ("model", 1), ("model", 3)])
def test_fp16_operands_are_needed_in_polar_express(monkeypatch, init, chunk):
    cs, w, ns = 64, 32, 5
    inp = SC.make_inputs(1, cs * (chunk + 1), 2, 64, 128, seed=3, init=init, io="bf16")
    _, states = SC.oracle_trajectory(inp, cs, w, ns)
    sl = slice(chunk * cs, (chunk + 1) * cs)
    args = [inp[k][:, sl] for k in ("q", "k", "v", "alpha", "eta", "theta")] + [inp["gamma"][:, sl], w, ns]
    e16 = _chunk_errors(monkeypatch, states[chunk], args, "f16")
    ebf = _chunk_errors(monkeypatch, states[chunk], args, "bf16")
    print(f"{init} chunk {chunk}: fp16 {e16:.2e}, bf16 {ebf:.2e}")
    assert e16 < 3e-3
    assert ebf > 1e-2 and ebf > 5 * e16
