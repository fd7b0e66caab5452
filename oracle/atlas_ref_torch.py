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


# ---------------------------------------------------------------------------
# Layer and model forwards in torch (float64), for whole-model gradients.
# Each follows the NumPy oracle function of the same name (oracle/atlas_ref.py,
# itself pinned in tests/test_oracle_model.py) and is checked against it to
# 1e-12 in tests/test_oracle_grad.py; gradients come from torch autograd.
# Parameters are dicts of tensors with the NumPy oracle's keys.
# ---------------------------------------------------------------------------

def rms_norm_t(x):
    """memory_layer.py:211-216."""
    return x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6)


def short_conv_t(x, weight, bias):
    """memory_layer.py:303-329: out[t] = bias + sum_j w[j] x[t-(K-1)+j]."""
    B, T, C = x.shape
    K = weight.shape[-1]
    xp = torch.cat([torch.zeros(B, K - 1, C, dtype=x.dtype), x], dim=1)
    out = bias.reshape(1, 1, C).expand(B, T, C)
    for j in range(K):
        out = out + xp[:, j:j + T, :] * weight[:, 0, j].reshape(1, 1, C)
    return out


def poly_features_t(x, coeffs):
    """memory_layer.py:459-466."""
    out, xp = coeffs[0] * x, x
    for i in range(1, coeffs.shape[0]):
        xp = xp * x
        out = out + coeffs[i] * xp
    return out


def memory_layer_forward_t(x, p, cfg, state=None):
    """memory_layer.py:599-727 (prologue :606-633, default state :635-643,
    chunk loop, retrieve gate :720-722, output projection :724-725)."""
    B, T, C = x.shape
    H, D, E = cfg['n_head'], cfg['head_dim'], cfg['expand_dim']
    q = short_conv_t(x @ p['c_q'].T, p['conv_q_w'], p['conv_q_b']).reshape(B, T, H, D)
    k = short_conv_t(x @ p['c_k'].T, p['conv_k_w'], p['conv_k_b']).reshape(B, T, H, D)
    v = short_conv_t(x @ p['c_v'].T, p['conv_v_w'], p['conv_v_b']).reshape(B, T, H, D)
    if cfg['poly_degree'] > 0:
        q = poly_features_t(rms_norm_t(q), p['poly_coeffs'])
        k = rms_norm_t(poly_features_t(k, p['poly_coeffs']))
    else:
        q, k = rms_norm_t(q), rms_norm_t(k)

    def gate(name):
        return torch.sigmoid(x @ p[name + '_w'].T + p[name + '_b'])

    alpha, eta, theta = gate('gate_alpha'), gate('gate_eta') * cfg['max_lr'], gate('gate_theta')
    gamma = gate('gate_gamma') if cfg['omega_window'] > 1 else None
    if state is None:
        W1 = p['W1_init'].unsqueeze(0).expand(B, H, D, E)
        W2 = p['W2_init'].unsqueeze(0).expand(B, H, E, D)
        state = (W1, W2, torch.zeros(B, H, D, E, dtype=x.dtype), torch.zeros(B, H, E, D, dtype=x.dtype))
    y, state = memory_scan_t(q, k, v, alpha, eta, theta, gamma, state, cfg['chunk_size'], cfg['omega_window'],
                             cfg['ns_steps'], cfg.get('pe_ste', False), cfg.get('stop_grad_chunks', False))
    if p.get('retrieve_w') is not None:
        y = y * torch.sigmoid(x @ p['retrieve_w'].T).unsqueeze(-1)
    return y.reshape(B, T, H * D) @ p['c_proj'].T, state


def mlp_geglu_t(x, p):
    """model.py:142-167 (GEGLU)."""
    h = x @ p['mlp_fc'].T
    half = h.shape[-1] // 2
    return (torch.nn.functional.silu(h[..., half:]) * h[..., :half]) @ p['mlp_proj'].T


def initial_model_state_t(B, H, D, E, dtype=torch.float64):
    """model.py:251-264: W1 = 0, W2 = [I; 0], S = 0."""
    W2 = torch.zeros(B, H, E, D, dtype=dtype)
    m = min(D, E)
    W2[:, :, :m, :m] = torch.eye(m, dtype=dtype)
    return (torch.zeros(B, H, D, E, dtype=dtype), W2, torch.zeros(B, H, D, E, dtype=dtype),
            torch.zeros(B, H, E, D, dtype=dtype))


def atlas_forward_t(idx, params, cfg, states=None):
    """model.py:305-374 (no dropout); persistent memory tokens
    (params['persist_mem']) prepended (:316-320) and dropped after the final
    norm (:359-360)."""
    B, T = idx.shape
    H, D, E = cfg['n_head'], cfg['head_dim'], cfg['expand_dim']
    x = params['wte'][idx]
    pm = params.get('persist_mem')
    n_persist = 0 if pm is None else pm.shape[0]
    if n_persist:
        x = torch.cat([pm.unsqueeze(0).expand(B, -1, -1), x], dim=1)
    new_states = []
    for li, p in enumerate(params['layers']):
        st = initial_model_state_t(B, H, D, E, x.dtype) if states is None else states[li]
        mem, st = memory_layer_forward_t(rms_norm_t(x), p, cfg, st)
        x = x + mem
        x = x + mlp_geglu_t(rms_norm_t(x), p)
        new_states.append(st)
    logits = (rms_norm_t(x)[:, n_persist:] @ params['lm_head'].T)[..., :cfg['vocab_size']]
    sc = cfg.get('logit_softcap', 0.0)
    if sc > 0:
        logits = sc * torch.tanh(logits / sc)
    return logits, new_states


def swa_core_t(q, k, v, window):
    """model.py:109-129 after the projection (rotary rotation, banded causal
    softmax, value sum), on (B, T, H, D)."""
    B, T, H, D = q.shape
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    ang = torch.outer(torch.arange(T, dtype=torch.float64), inv)
    c, s = torch.cos(ang).to(q.dtype)[None, :, None], torch.sin(ang).to(q.dtype)[None, :, None]

    def rot(x):
        x1, x2 = x[..., :D // 2], x[..., D // 2:]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1)

    sc = torch.einsum('bthd,bshd->bhts', rot(q), rot(k)) / math.sqrt(D)
    t = torch.arange(T)[:, None]
    s_ = torch.arange(T)[None, :]
    mask = (t >= s_) & ((t - s_) <= window)
    p = torch.softmax(sc.masked_fill(~mask, float('-inf')), dim=-1)
    return torch.einsum('bhts,bshd->bthd', p, v)


def mag_forward_t(idx, params, cfg, states=None):
    """mag_transformer.py:128-166 (no dropout), attention model.py:100-133,
    MemoryGate mag_transformer.py:22-32."""
    B, T = idx.shape
    H, D = cfg['n_head'], cfg['head_dim']
    x = params['wte'][idx]
    new_states = []
    for li, p in enumerate(params['layers']):
        qkv = rms_norm_t(x) @ p['to_qkv'].T
        q, k, v = (qkv[..., i * H * D:(i + 1) * H * D].reshape(B, T, H, D) for i in range(3))
        attn = swa_core_t(q, k, v, cfg['window_size']).reshape(B, T, H * D) @ p['to_out'].T
        st = None
        if p.get('c_q') is not None:
            mem, st = memory_layer_forward_t(rms_norm_t(x), p, cfg, None if states is None else states[li])
            g = torch.sigmoid(rms_norm_t(mem) @ p['gate_w'].T + p['gate_b'])
            x = x + attn + g * mem
        else:
            x = x + attn
        x = x + mlp_geglu_t(rms_norm_t(x), p)
        new_states.append(st)
    return rms_norm_t(x) @ params['lm_head'].T, new_states
