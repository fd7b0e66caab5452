"""A float32 evaluation of the reference semantics in NumPy, token by token:
one more member of the fp32 ensembles that bound the end-to-end tests.

The chunk body of atlas_jax/memory_layer.py:496-597 (inner gradient :505-520,
Omega window as a cumulative sum minus the sum w tokens back :233-253 /
:522-527, momentum and memory scans :529-533 / :566-590, Polar-Express
:43-71, read-out :592-595) with every array operation in float32 and the
scans run sequentially per token, as the reference's lax.scan does; batched
over (B, H) with NumPy's float32 matmul.  Its summation orders differ from
those of the torch evaluation (oracle/atlas_ref_torch.py in float32): over
the 16 chunks of config 1 its end-to-end error against float64 is 2-3x the
torch evaluation's, while both are valid fp32 arithmetic of the same
function -- an fp32 bound has to cover such orders."""

import numpy as np

from oracle import atlas_ref as R

F = np.float32


def _pe(X, ns):
    """Polar-Express (memory_layer.py:43-71) in float32 on (..., d1, d2)."""
    X = X.astype(F)
    nrm = np.sqrt((X * X).sum(axis=(-2, -1), keepdims=True, dtype=F) + F(1e-12)) * F(1.01) + F(1e-6)
    X = (X / nrm).astype(F)
    tall = X.shape[-2] > X.shape[-1]
    if tall:
        X = np.swapaxes(X, -1, -2)
    for a, b, c in R.PE_COEFFS[:ns]:
        A = np.matmul(X, np.swapaxes(X, -1, -2)).astype(F)
        B = (F(b) * A + F(c) * np.matmul(A, A)).astype(F)
        X = (F(a) * X + np.matmul(B, X)).astype(F)
    return np.swapaxes(X, -1, -2) if tall else X


def _gelu_tanh(x):
    return (F(0.5) * x * (F(1) + np.tanh(F(0.7978845608028654) * (x + F(0.044715) * x * x * x)))).astype(F)


def chunk(state, q, k, v, alpha, eta, theta, gamma, w, ns):
    """One chunk: q, k, v (B, cs, H, D); gates (B, cs, H); state (W1, W2,
    S1, S2) as (B, H, ...).  Returns (y (B, cs, H, D), state), float32."""
    W1, W2, S1, S2 = (np.asarray(s, F) for s in state)
    q, k, v = (np.asarray(x, F) for x in (q, k, v))
    D = q.shape[-1]
    cs = q.shape[1]
    kt = np.transpose(k, (0, 2, 1, 3))                       # (B, H, cs, D)
    vt = np.transpose(v, (0, 2, 1, 3))
    h = np.matmul(kt, np.swapaxes(W2, -1, -2)).astype(F)    # (B, H, cs, E)
    act = _gelu_tanh(h)
    gp = R.gelu_derivative(h.astype(np.float64)).astype(F)
    err = (kt + np.matmul(act, np.swapaxes(W1, -1, -2)) - vt).astype(F)   # (B, H, cs, D)
    chain = (np.matmul(err, W1) * gp).astype(F)                            # (B, H, cs, E)
    sc = F(2.0 / D)
    u1 = (sc * err[..., :, None] * act[..., None, :]).astype(F)           # (B, H, cs, D, E)
    u2 = (sc * chain[..., :, None] * kt[..., None, :]).astype(F)          # (B, H, cs, E, D)
    if w > 1 and gamma is not None:
        g = np.transpose(np.asarray(gamma, F), (0, 2, 1))[..., None, None]
        c1 = np.cumsum((g * u1).astype(F), axis=2, dtype=F)
        c2 = np.cumsum((g * u2).astype(F), axis=2, dtype=F)
        if w < cs:
            c1[:, :, w:] = (c1[:, :, w:] - c1[:, :, :-w]).astype(F)
            c2[:, :, w:] = (c2[:, :, w:] - c2[:, :, :-w]).astype(F)
        u1, u2 = c1, c2
    al, et, th = (np.transpose(np.asarray(x, F), (0, 2, 1)) for x in (alpha, eta, theta))
    y = np.zeros(q.shape, F)
    for t in range(cs):
        S1 = (th[..., t, None, None] * S1 - et[..., t, None, None] * u1[:, :, t]).astype(F)
        S2 = (th[..., t, None, None] * S2 - et[..., t, None, None] * u2[:, :, t]).astype(F)
        W1 = (al[..., t, None, None] * W1 + _pe(S1, ns)).astype(F)
        W2 = (al[..., t, None, None] * W2 + _pe(S2, ns)).astype(F)
        qt = q[:, t]                                                        # (B, H, D)
        hq = np.matmul(W2, qt[..., None])[..., 0].astype(F)
        y[:, t] = (qt + np.matmul(W1, _gelu_tanh(hq)[..., None])[..., 0]).astype(F)
    return y, (W1, W2, S1, S2)


def memory_scan(q, k, v, alpha, eta, theta, gamma, state, cs, w, ns):
    """The chunk loop (memory_layer.py:649-716) with the reference padding
    (alpha 1, eta = theta = gamma = 0, q = k = v = 0 past T)."""
    T = q.shape[1]
    q, k, v, alpha, eta, theta, gamma = R._pad_inputs(q, k, v, alpha, eta, theta, gamma, cs)
    ys = []
    for c0 in range(0, q.shape[1], cs):
        sl = slice(c0, c0 + cs)
        y, state = chunk(state, q[:, sl], k[:, sl], v[:, sl], alpha[:, sl], eta[:, sl], theta[:, sl],
                         None if gamma is None else gamma[:, sl], w, ns)
        ys.append(y)
    return np.concatenate(ys, axis=1)[:, :T], state
