"""Seeded inputs and oracle trajectories shared by the scan tests.

Inputs follow the BASELINE config-1 recipe (numpy PCG64(seed)): q, k, v ~
N(0,1) with q, k L2-normalised over D; gate logits ~ N(0,1); alpha, theta,
gamma = sigmoid(logit), eta = sigmoid(logit) * max_lr; W1 (D,E) and W2 (E,D)
~ N(0, 1/D) (or the model initial state W1=0, W2=[I;0]); S = 0.

Because the Atlas recurrence amplifies rounding differences from chunk to
chunk, long-horizon parity is checked "teacher-forced": every chunk of the
oracle's own float64 trajectory becomes an independent stream (batch row) of
one GPU call, started from the oracle's state at that chunk's start.
"""

import numpy as np

from oracle import atlas_ref as R

MAX_LR = 0.1


def bf16_round(x):
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).to(torch.bfloat16).float().numpy() \
        .astype(np.float64)


def f16_round(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def make_inputs(B, T, H, D, E, seed=0, init="rand", io="f32", with_gamma=True, s_scale=0.0):
    rng = np.random.Generator(np.random.PCG64(seed))
    q = rng.standard_normal((B, T, H, D))
    k = rng.standard_normal((B, T, H, D))
    v = rng.standard_normal((B, T, H, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    k /= np.linalg.norm(k, axis=-1, keepdims=True)
    sig = lambda z: 1.0 / (1.0 + np.exp(-z))  # noqa: E731
    alpha = sig(rng.standard_normal((B, T, H)))
    eta = sig(rng.standard_normal((B, T, H))) * MAX_LR
    theta = sig(rng.standard_normal((B, T, H)))
    gamma = sig(rng.standard_normal((B, T, H))) if with_gamma else None
    if init == "model":
        state = R.initial_model_state(B, H, D, E)
    else:
        W1 = rng.standard_normal((B, H, D, E)) / np.sqrt(D)
        W2 = rng.standard_normal((B, H, E, D)) / np.sqrt(D)
        S1 = rng.standard_normal((B, H, D, E)) * s_scale
        S2 = rng.standard_normal((B, H, E, D)) * s_scale
        state = (W1, W2, S1, S2)
    if io == "bf16":
        q, k, v = bf16_round(q), bf16_round(k), bf16_round(v)
    elif io == "f16":
        q, k, v = f16_round(q), f16_round(k), f16_round(v)
    # the GPU consumes fp32 gates/state: round them once so both sides agree
    f32 = lambda a: None if a is None else np.asarray(a, np.float32).astype(np.float64)  # noqa: E731
    return dict(q=q, k=k, v=v, alpha=f32(alpha), eta=f32(eta), theta=f32(theta), gamma=f32(gamma),
                state=tuple(f32(s) for s in state))


def oracle_trajectory(inp, cs, w, ns):
    """Sequential float64 oracle; returns y (B,T,H,D) and the list of states at
    every chunk boundary (n_chunks + 1 entries)."""
    q, k, v = inp["q"], inp["k"], inp["v"]
    T = q.shape[1]
    assert T % cs == 0
    st = inp["state"]
    states = [st]
    ys = []
    for c0 in range(0, T, cs):
        sl = slice(c0, c0 + cs)
        g = None if inp["gamma"] is None else inp["gamma"][:, sl]
        y, st = R.process_chunk_deep(st, q[:, sl], k[:, sl], v[:, sl], inp["alpha"][:, sl], inp["eta"][:, sl],
                                     inp["theta"][:, sl], g, w, ns)
        ys.append(y)
        states.append(st)
    return np.concatenate(ys, axis=1), states


def teacher_forced_inputs(inp, states, cs):
    """Rearrange (B, T, ...) inputs into (B*nc, cs, ...) streams whose start
    states are the oracle's chunk-start states (fp32-rounded)."""
    B, T, H, D = inp["q"].shape
    nc = T // cs

    def seq(a):
        return None if a is None else a.reshape(B, nc, cs, *a.shape[2:]).reshape(B * nc, cs, *a.shape[2:])

    start = []
    for m in range(4):
        s = np.stack([states[c][m] for c in range(nc)], axis=1)   # (B, nc, H, ...)
        start.append(np.asarray(s.reshape(B * nc, *s.shape[2:]), np.float32).astype(np.float64))
    out = {k_: seq(inp[k_]) for k_ in ("q", "k", "v", "alpha", "eta", "theta", "gamma")}
    out["state"] = tuple(start)
    return out


def permuted_pe(seed):
    """Polar-Express of the row- and column-permuted matrix, permuted back:
    the same mathematics with every summation order changed (a member of the
    fp32 ensembles that set the end-to-end and gradient bounds)."""
    import torch
    from oracle import atlas_ref_torch as RT
    pe, g = RT.polar_express_t, torch.Generator().manual_seed(seed)

    def f(X, steps=5, norm_eps=1e-12):
        r, c = torch.randperm(X.shape[-2], generator=g), torch.randperm(X.shape[-1], generator=g)
        return pe(X[..., r, :][..., :, c], steps, norm_eps)[..., torch.argsort(r), :][..., :, torch.argsort(c)]
    return f


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    nb = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / nb) if nb > 0 else float(np.linalg.norm(a - b))


def worst_chunk_errors(y_gpu, states_gpu, y_ref, states_ref, B, nc, cs):
    """Per-chunk rel-L2 of y and of each end-state matrix; returns the worst."""
    H, D = y_ref.shape[2], y_ref.shape[3]
    yg = np.asarray(y_gpu).reshape(B, nc, cs, H, D)
    yr = np.asarray(y_ref).reshape(B, nc, cs, H, D)
    worst = {"y": 0.0, "W1": 0.0, "W2": 0.0, "S1": 0.0, "S2": 0.0}
    for c in range(nc):
        worst["y"] = max(worst["y"], rel_l2(yg[:, c], yr[:, c]))
        for m, name in enumerate(("W1", "W2", "S1", "S2")):
            g = np.asarray(states_gpu[m]).reshape(B, nc, *states_gpu[m].shape[1:])[:, c]
            worst[name] = max(worst[name], rel_l2(g, states_ref[c + 1][m]))
    return worst
