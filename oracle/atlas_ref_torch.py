"""torch float64 restatement of the fused-chunk operator, for its gradients.

TEST INFRASTRUCTURE ONLY -- imported by tests/ as the checker of the
backward passes, never by the product path.

fused_chunk_regular_t follows kernels/fused_chunk.py:279-314 (_regular_fwd)
with polar_express (memory_layer.py:43-71) or its straight-through variant
(:74-76), linear_scan (memory_layer.py:256-296) and the tanh GELU of the
read-out; its gradients come from torch autograd in float64, which is what
the reference's custom VJP (fused_chunk.py:357-376, jax.vjp of
_regular_fwd) computes.

Pinning: the forward equals oracle.atlas_ref.fused_chunk_regular (itself
pinned by the per-token brute force) to 1e-12, and torch.autograd.gradcheck
(finite differences) checks the gradients on small inputs
(tests/test_oracle_grad.py).
"""

import math

import torch

from .atlas_ref import PE_COEFFS


def polar_express_t(X, steps=5, norm_eps=1e-12):
    """memory_layer.py:43-71 in torch float64 (differentiable)."""
    frob = torch.sqrt((X * X).sum(dim=(-2, -1), keepdim=True) + norm_eps)
    X = X / (frob * 1.01 + 1e-6)
    tall = X.shape[-2] > X.shape[-1]
    for a, b, c in PE_COEFFS[:steps].tolist():
        if tall:
            A = X.mT @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ X.mT
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


def polar_express_ste_t(X, steps=5):
    """memory_layer.py:74-76: forward PE(X), backward identity."""
    return X + (polar_express_t(X, steps) - X).detach()


def linear_scan_t(h0, gates, x):
    """memory_layer.py:256-296: h_t = g_t h_{t-1} + x_t along axis 1."""
    hs = []
    h = h0
    extra = (1,) * (x.dim() - 3)
    for t in range(x.shape[1]):
        h = gates[:, t].reshape(*gates[:, t].shape, *extra) * h + x[:, t]
        hs.append(h)
    return torch.stack(hs, dim=1), h


def gelu_tanh_t(x):
    return 0.5 * x * (1.0 + torch.tanh(math.sqrt(2.0 / math.pi) * (x + 0.044715 * x ** 3)))


def fused_chunk_regular_t(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste=False):
    """kernels/fused_chunk.py:279-314 -> (y, W1_end, W2_end, S1_end, S2_end)."""
    pe = polar_express_ste_t if pe_ste else polar_express_t
    S1_all, S1 = linear_scan_t(SW1, theta, momW1)
    S2_all, S2 = linear_scan_t(SW2, theta, momW2)
    W1_all, W1e = linear_scan_t(W1, alpha, pe(S1_all, ns_steps))
    W2_all, W2e = linear_scan_t(W2, alpha, pe(S2_all, ns_steps))
    h = torch.einsum("bched,bchd->bche", W2_all, q)
    y = q + torch.einsum("bchde,bche->bchd", W1_all, gelu_tanh_t(h))
    return y, W1e, W2e, S1, S2


def fused_chunk_vjp_t(inputs, cotangents, ns_steps, pe_ste=False):
    """float64 gradients of fused_chunk_regular_t's five outputs, contracted
    with `cotangents` (gy, gW1, gW2, gS1, gS2), with respect to the nine
    array inputs (W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q)."""
    xs = [torch.as_tensor(a, dtype=torch.float64).clone().requires_grad_(True) for a in inputs]
    outs = fused_chunk_regular_t(*xs, ns_steps, pe_ste)
    cts = [torch.as_tensor(c, dtype=torch.float64) for c in cotangents]
    grads = torch.autograd.grad(outs, xs, grad_outputs=cts, allow_unused=True)
    return [torch.zeros_like(x) if g is None else g for x, g in zip(xs, grads)]


def gelu_erf_derivative_t(x):
    """memory_layer.py:225-230: Phi(x) + x phi(x)."""
    return 0.5 * (1.0 + torch.erf(x / math.sqrt(2.0))) + x * torch.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def omega_aggregate_t(u, gamma, w):
    """memory_layer.py:233-253, written as the window sum it equals:
    G_t = sum_{i=max(0,t-w+1)}^{t} gamma_i u_i along axis 1."""
    gu = gamma.reshape(*gamma.shape, *(1,) * (u.dim() - 3)) * u
    return torch.stack([gu[:, max(0, t - w + 1):t + 1].sum(dim=1) for t in range(u.shape[1])], dim=1)


def memory_scan_t(q, k, v, alpha, eta, theta, gamma, state, cs, w, ns_steps, pe_ste=False,
                  stop_grad_chunks=False):
    """The whole layer's chunk loop (memory_layer.py:649-711) with
    _process_chunk_deep's fused branch (:496-541) in torch float64:
    padding, memory forward, inner gradient, Omega window, momentum input and
    fused_chunk_regular_t per chunk -> (y (B,T,H,D), (W1, W2, S1, S2)).
    stop_grad_chunks detaches the carry at every chunk start (:665)."""
    B, T, H, D = q.shape
    W1, W2, S1, S2 = state
    if T % cs:
        pad = cs - T % cs

        def _p(t, val):
            return torch.cat([t, torch.full((B, pad, *t.shape[2:]), val, dtype=t.dtype)], dim=1)
        q, k, v = _p(q, 0.0), _p(k, 0.0), _p(v, 0.0)
        alpha, eta, theta = _p(alpha, 1.0), _p(eta, 0.0), _p(theta, 0.0)
        gamma = None if gamma is None else _p(gamma, 0.0)
    ys = []
    for c in range(q.shape[1] // cs):
        sl = slice(c * cs, (c + 1) * cs)
        if stop_grad_chunks:
            W1, W2, S1, S2 = (t.detach() for t in (W1, W2, S1, S2))
        kc, vc = k[:, sl], v[:, sl]
        h = torch.einsum("bhed,bchd->bche", W2, kc)
        act = gelu_tanh_t(h)
        err = kc + torch.einsum("bhde,bche->bchd", W1, act) - vc
        u1 = (2.0 / D) * torch.einsum("bchd,bche->bchde", err, act)
        chain = torch.einsum("bhde,bchd->bche", W1, err) * gelu_erf_derivative_t(h)
        u2 = (2.0 / D) * torch.einsum("bche,bchd->bched", chain, kc)
        if w > 1 and gamma is not None:
            u1 = omega_aggregate_t(u1, gamma[:, sl], w)
            u2 = omega_aggregate_t(u2, gamma[:, sl], w)
        e = eta[:, sl, :, None, None]
        y, W1, W2, S1, S2 = fused_chunk_regular_t(W1, W2, S1, S2, -(e * u1), -(e * u2), theta[:, sl],
                                                  alpha[:, sl], q[:, sl], ns_steps, pe_ste)
        ys.append(y)
    return torch.cat(ys, dim=1)[:, :T], (W1, W2, S1, S2)
