"""CPU baseline: torch-CPU fp32 restatement of the reference's non-fused JAX
chunk loop.

TEST/MEASUREMENT INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).  JAX is not
installed on these machines, so the reference's own JAX-on-CPU path cannot be
timed; this restates it operation for operation in torch on the host cores:
per chunk the batched inner gradient with materialised (B,cs,H,D,E) tensors,
the cumsum Omega window, sequential linear scans, batched fp32 Polar-Express
over all cs tokens and the read-out (atlas_jax/memory_layer.py:496-597 in the
D != E branch :577-595; the chunk loop :699-716).
"""

import math

import torch

PE = [
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
]


def _pe(X, steps):
    frob = torch.sqrt((X * X).sum(dim=(-2, -1), keepdim=True) + 1e-12)
    X = X / (frob * 1.01 + 1e-6)
    tall = X.shape[-2] > X.shape[-1]
    for a, b, c in PE[:steps]:
        if tall:
            A = X.transpose(-1, -2) @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ X.transpose(-1, -2)
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


def _gelu_tanh(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def _gelu_prime(x):
    return 0.5 * (1.0 + torch.erf(x * 0.7071067811865476)) + x * torch.exp(-0.5 * x * x) * 0.3989422804014327


def _scan(h, g, x):
    out = torch.empty_like(x)
    shape = (g.shape[0], g.shape[2]) + (1,) * (x.dim() - 3)
    for t in range(x.shape[1]):
        h = g[:, t].reshape(shape) * h + x[:, t]
        out[:, t] = h
    return out, h


def chunk(state, q, k, v, a, e, t, g, w, ns):
    W1, W2, S1, S2 = state
    D = k.shape[-1]
    h = torch.einsum('bhed,bchd->bche', W2, k)
    act = _gelu_tanh(h)
    err = k + torch.einsum('bhde,bche->bchd', W1, act) - v
    u1 = (2.0 / D) * torch.einsum('bchd,bche->bchde', err, act)
    chain = torch.einsum('bhde,bchd->bche', W1, err) * _gelu_prime(h)
    u2 = (2.0 / D) * torch.einsum('bche,bchd->bched', chain, k)
    if w > 1 and g is not None:
        cs = u1.shape[1]
        gg = g[..., None, None]

        def omega(u):
            cum = torch.cumsum(gg * u, dim=1)
            if w >= cs:
                return cum
            return cum - torch.cat([torch.zeros_like(cum[:, :w]), cum[:, :-w]], dim=1)
        u1, u2 = omega(u1), omega(u2)
    ee = e[..., None, None]
    S1a, S1 = _scan(S1, t, -ee * u1)
    S2a, S2 = _scan(S2, t, -ee * u2)
    W1a, W1 = _scan(W1, a, _pe(S1a, ns))
    W2a, W2 = _scan(W2, a, _pe(S2a, ns))
    hq = torch.einsum('bched,bchd->bche', W2a, q)
    y = q + torch.einsum('bchde,bche->bchd', W1a, _gelu_tanh(hq))
    return y, (W1, W2, S1, S2)


def memory_scan(q, k, v, a, e, t, g, state, cs, w, ns):
    ys = []
    for c0 in range(0, q.shape[1], cs):
        sl = slice(c0, c0 + cs)
        y, state = chunk(state, q[:, sl], k[:, sl], v[:, sl], a[:, sl], e[:, sl], t[:, sl],
                         None if g is None else g[:, sl], w, ns)
        ys.append(y)
    return torch.cat(ys, dim=1), state
