"""NumPy float64 restatement of the Atlas memory-layer path (the oracle).

TEST INFRASTRUCTURE ONLY -- imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product path.

Every function follows a named span of the reference (rkstgr/atlas-jax,
paths relative to the repository root) and computes in float64 whatever
dtype the inputs have.  Inputs that the GPU path takes in bf16 are rounded to
bf16 by the caller before they reach the oracle, so both sides see the same
values.

Pinning (what checks each function beyond restating it; see tests/):
  polar_express         SVD closed form U p(S/s) V^T (polar_express_svd),
                        diagonal inputs, ns=0, zero input, orthogonality and
                        batch invariants of tests/test_polar_express.py.
  muon_polar_express    same SVD closed form with the eps-free norm.
  muon_leaf_update      momentum=0 reduces to the polar factor of the
                        gradient; with beta2=0 NorMuon equalises every row's
                        (column's) mean square and keeps the Frobenius norm;
                        cautious decay only acts where update and weight agree.
  linear_scan           manual loop of tests/test_memory_layer.py:17-34 and the
                        closed form h_t = prod(g) h0 + sum prod(g) x.
  omega_aggregate       naive O(cs*w) double loop (tests/test_omega.py:34-51),
                        w=1 => gamma*u, w>=cs => cumsum, gamma mask [1,1,2,2].
  gelu_tanh/gelu_erf    closed forms; gelu_derivative by finite differences.
  inner_gradient        u_W1 equals autograd of (1/D)||k+W1 gelu(W2 k)-v||^2
                        (torch float64); u_W2 equals (2/D) times the W2-autograd
                        of <sg(err), W1 gelu_erf(W2 k)> (the erf surrogate;
                        tests/test_oracle_model.py, with planted W1/W1^T, tanh
                        derivative and v-for-k mistakes rejected).
  process_chunk_deep /  per-token brute force (memory_scan_bruteforce) that
  memory_scan           uses the SVD form of PE and scalar recurrences.
  short_conv, rms_norm, closed forms on small inputs (tests/test_oracle.py).
  poly_features
  memory_layer_prologue k leaves with unit RMS, q does not unless the map is
                        linear (norm/map order, a swapped order rejected).
  memory_layer_forward  zero retrieve weight halves the output; chunk-aligned
                        continuation from the carried state equals one call.
  atlas_forward         zero block outputs reduce it to rms_norm(wte) lm_head
                        (+ softcap); causal bit for bit (a right-padded conv
                        rejected); padding zeroes S; chunk-aligned continuation
                        from carried per-layer states equals one call (the
                        layers' states swapped rejected); persistent tokens
                        equal to embedding rows z give the forward on [z, idx]
                        without its first positions (appended tokens or the
                        wrong positions dropped rejected).
  mlp_geglu             a saturated gate (silu(50) = 50) makes it the linear
                        value path; the swapped split rejected.
  rope_tables,          angle-by-angle loop (swa_bruteforce); the rotation
  apply_rope            keeps each (d, d + D/2) pair's norm and makes q'.k'
                        depend on t - s only.
  swa_core              per-query brute force with explicit angles and a
                        max-shifted softmax over the allowed keys only;
                        window = 0 returns v exactly; window >= T is plain
                        causal attention.
  swa_forward           window 0 makes it (rms_norm(x) W_v^T) W_out^T with W_v
                        the last third of to_qkv (q/v thirds swapped rejected).
  memory_gate           zero weight gives sigmoid(b); with W = cI the logit is
                        c rms_norm(x) (unit RMS; a gate without the norm
                        rejected).
  mag_forward           zero outputs reduce it to rms_norm(wte) lm_head; causal
                        bit for bit; the memory branch adds gate(mem) * mem
                        (an ungated add rejected).
"""

import numpy as np
from scipy.special import erf as _erf

# memory_layer.py:34-40 -- the five (a, b, c) odd-quintic Polar-Express
# coefficient rows.  The values are data fixed by the reference (the same
# table is in the HIP library), not something to re-derive.
PE_COEFFS = np.array([
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
], dtype=np.float64)

MAX_NS_STEPS = 5


def _f64(x):
    return np.asarray(x, dtype=np.float64)


def _mT(x):
    return np.swapaxes(x, -2, -1)


# ---------------------------------------------------------------------------
# Polar-Express
# ---------------------------------------------------------------------------

def polar_express(X, steps=5):
    """memory_layer.py:43-71 and kernels/triton_pe.py:26-69 (identical for
    steps <= 5).  Frobenius-normalise with sqrt(sum X^2 + 1e-12)*1.01 + 1e-6,
    then `steps` odd-quintic iterations; tall inputs (rows > cols) use the
    X^T X Gram, square and wide inputs use X X^T."""
    if not 0 <= steps <= MAX_NS_STEPS:
        raise ValueError(f"steps must be in [0, {MAX_NS_STEPS}], got {steps}")
    X = _f64(X)
    frob = np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True) + 1e-12)
    X = X / (frob * 1.01 + 1e-6)
    d1, d2 = X.shape[-2], X.shape[-1]
    for a, b, c in PE_COEFFS[:steps]:
        if d1 > d2:
            A = _mT(X) @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ _mT(X)
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


def pe_scalar_map(sigma, steps):
    """The scalar odd polynomial that Polar-Express applies to each singular
    value: s -> a s + b s^3 + c s^5 per coefficient row."""
    s = _f64(sigma)
    for a, b, c in PE_COEFFS[:steps]:
        s = a * s + b * s ** 3 + c * s ** 5
    return s


def polar_express_svd(X, steps=5, norm_eps=1e-12):
    """Independent closed form of polar_express: with X = U diag(s) V^T and
    scale = sqrt(sum s^2 + eps)*1.01 + 1e-6, PE(X) = U diag(p(s/scale)) V^T.
    (X X^T)^j X = X (X^T X)^j, so the tall and wide branches agree exactly."""
    X = _f64(X)
    U, s, Vt = np.linalg.svd(X, full_matrices=False)
    scale = np.sqrt(np.sum(s * s, axis=-1, keepdims=True) + norm_eps) * 1.01 + 1e-6
    p = pe_scalar_map(s / scale, steps)
    return (U * p[..., None, :]) @ Vt


def muon_polar_express(G, steps=5):
    """optim.py:69-83: Muon's Polar-Express on a (stacked) 2-D update.  Same
    iteration as polar_express but the Frobenius norm has no 1e-12 term and the
    branch is chosen on the parameter's own shape (tall iff rows > cols)."""
    if not 0 <= steps <= MAX_NS_STEPS:
        raise ValueError(f"steps must be in [0, {MAX_NS_STEPS}], got {steps}")
    X = _f64(G)
    frob = np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True))
    X = X / (frob * 1.01 + 1e-6)
    for a, b, c in PE_COEFFS[:steps]:
        if X.shape[-2] > X.shape[-1]:
            A = _mT(X) @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ _mT(X)
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


def muon_leaf_update(grad, momentum_buf, second_moment, param, learning_rate, momentum, beta2,
                     weight_decay, ns_steps):
    """optim.py:56-108 (_muon_leaf_update): Nesterov momentum, Polar-Express
    on the Nesterov direction, NorMuon per-row (or per-column) variance
    reduction, cautious weight decay.  Arrays are float64; returns
    (update, new_momentum, new_second_moment)."""
    grad = _f64(grad)
    shape = grad.shape
    lr_scale = max(1.0, shape[-2] / shape[-1]) ** 0.5
    new_momentum = _f64(momentum_buf) * momentum + grad * (1 - momentum)
    g = grad * (1 - momentum) + new_momentum * momentum
    g = muon_polar_express(g, ns_steps)
    red = -1 if shape[-2] >= shape[-1] else -2
    n_red = shape[red]
    v_mean = np.mean(g * g, axis=red, keepdims=True)
    v_norm = np.sqrt(np.sum(v_mean, axis=(-2, -1), keepdims=True) * n_red)
    new_second = _f64(second_moment) * beta2 + v_mean * (1 - beta2)
    step = 1.0 / np.sqrt(np.maximum(new_second, 1e-10))
    v_norm_new = np.sqrt(np.sum(v_mean * n_red * step ** 2, axis=(-2, -1), keepdims=True))
    g = g * (step * (v_norm / np.maximum(v_norm_new, 1e-10)))
    if param is not None and weight_decay > 0:
        mask = (g * _f64(param)) >= 0
        update = -(learning_rate * lr_scale * g + learning_rate * lr_scale * weight_decay * _f64(param) * mask)
    else:
        update = -learning_rate * lr_scale * g
    return update, new_momentum, new_second


# ---------------------------------------------------------------------------
# Elementwise pieces
# ---------------------------------------------------------------------------

def rms_norm(x):
    """memory_layer.py:211-216: x * rsqrt(mean(x^2) + 1e-6) over the last axis."""
    x = _f64(x)
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + 1e-6)


def gelu_tanh(x):
    """jax.nn.gelu with its default approximate=True, as called at
    memory_layer.py:506,594: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))."""
    x = _f64(x)
    return 0.5 * x * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (x + 0.044715 * x ** 3)))


def gelu_erf(x):
    """Exact GELU x * Phi(x)."""
    x = _f64(x)
    return 0.5 * x * (1.0 + _erf(x / np.sqrt(2.0)))


def gelu_derivative(x):
    """memory_layer.py:225-230: derivative of the exact (erf) GELU,
    Phi(x) + x phi(x)."""
    x = _f64(x)
    cdf = 0.5 * (1.0 + _erf(x * 0.7071067811865476))
    pdf = np.exp(-0.5 * x * x) * 0.3989422804014327
    return cdf + x * pdf


def poly_features(x, coeffs):
    """memory_layer.py:459-466: sum_{i=1..p} coeffs[i-1] * x^i."""
    x = _f64(x)
    out = coeffs[0] * x
    xp = x
    for c in coeffs[1:]:
        xp = xp * x
        out = out + c * xp
    return out


def sigmoid(x):
    x = _f64(x)
    return 1.0 / (1.0 + np.exp(-x))


def silu(x):
    x = _f64(x)
    return x * sigmoid(x)


def short_conv(x, weight, bias):
    """memory_layer.py:303-329: causal depthwise conv over time.
    x (B,T,C), weight (C,1,K), bias (C,).  lax.conv_general_dilated is a
    cross-correlation over the left-padded input, so
    out[t,c] = bias[c] + sum_j weight[c,0,j] * x[t-(K-1)+j, c]."""
    x = _f64(x)
    B, T, C = x.shape
    K = weight.shape[-1]
    xp = np.concatenate([np.zeros((B, K - 1, C)), x], axis=1)
    out = np.zeros_like(x)
    for j in range(K):
        out += xp[:, j:j + T, :] * _f64(weight)[:, 0, j][None, None, :]
    return out + _f64(bias)[None, None, :]


# ---------------------------------------------------------------------------
# Scans and the Omega window
# ---------------------------------------------------------------------------

def omega_aggregate(u, gamma, omega_window):
    """memory_layer.py:233-253: G_t = sum_{i=max(0,t-w+1)}^{t} gamma_i u_i along
    axis 1 (the in-chunk token axis); the window restarts every chunk."""
    u = _f64(u)
    cs = u.shape[1]
    cum = np.cumsum(_f64(gamma) * u, axis=1)
    if omega_window >= cs:
        return cum
    shifted = np.concatenate(
        [np.zeros_like(cum[:, :omega_window]), cum[:, :-omega_window]], axis=1)
    return cum - shifted


def linear_scan(h_init, gates, inputs):
    """memory_layer.py:256-296 (and kernels/triton_scan.py): h_t = g_t h_{t-1}
    + x_t along axis 1.  gates (B,T,H) broadcast over trailing state dims.
    Returns (all h_t (B,T,H,...), final h (B,H,...))."""
    h = _f64(h_init).copy()
    g = _f64(gates)
    x = _f64(inputs)
    extra = x.ndim - g.ndim
    out = np.empty_like(x)
    for t in range(x.shape[1]):
        gt = g[:, t].reshape(g.shape[0], g.shape[2], *([1] * extra))
        h = gt * h + x[:, t]
        out[:, t] = h
    return out, h


# ---------------------------------------------------------------------------
# The chunk body and the chunk loop
# ---------------------------------------------------------------------------

def inner_gradient(W1, W2, k, v):
    """memory_layer.py:505-520: memory forward at the chunk-start weights
    (h = W2 k, act = gelu_tanh(h), err = k + W1 act - v) and the per-token
    inner gradients with scale 2/D:
      u_W1 = (2/D) err (x) act                                  (B,cs,H,D,E)
      u_W2 = (2/D) ((W1^T err) * gelu_derivative(h)) (x) k       (B,cs,H,E,D)
    W1 (B,H,D,E), W2 (B,H,E,D); k, v (B,cs,H,D)."""
    W1, W2, k, v = _f64(W1), _f64(W2), _f64(k), _f64(v)
    D = k.shape[-1]
    h = np.einsum('bhed,bchd->bche', W2, k)
    act = gelu_tanh(h)
    err = k + np.einsum('bhde,bche->bchd', W1, act) - v
    scale = 2.0 / D
    u1 = scale * np.einsum('bchd,bche->bchde', err, act)
    chain = np.einsum('bhde,bchd->bche', W1, err) * gelu_derivative(h)
    u2 = scale * np.einsum('bche,bchd->bched', chain, k)
    return u1, u2


def process_chunk_deep(state, q, k, v, alpha, eta, theta, gamma, omega_window, ns_steps):
    """memory_layer.py:496-597 (non-fused path).  q,k,v (B,cs,H,D); gates
    (B,cs,H); state = (W1 (B,H,D,E), W2 (B,H,E,D), S1, S2).  The reference's
    D==E branch (:544-576) stacks W1/W2 for batching; it is the same
    arithmetic as the D!=E branch (:577-590) followed here.
    Returns (y (B,cs,H,D), new state)."""
    W1, W2, S1, S2 = (_f64(s) for s in state)
    q = _f64(q)
    u1, u2 = inner_gradient(W1, W2, k, v)
    # omega :522-527 (only with a window > 1 and a gamma gate)
    if omega_window > 1 and gamma is not None:
        g = _f64(gamma)[..., None, None]
        u1 = omega_aggregate(u1, g, omega_window)
        u2 = omega_aggregate(u2, g, omega_window)
    # :529-533
    e = _f64(eta)[..., None, None]
    S1_all, S1 = linear_scan(S1, theta, -e * u1)
    S2_all, S2 = linear_scan(S2, theta, -e * u2)
    P1 = polar_express(S1_all, ns_steps)
    P2 = polar_express(S2_all, ns_steps)
    W1_all, W1 = linear_scan(W1, alpha, P1)
    W2_all, W2 = linear_scan(W2, alpha, P2)
    # mem_output :592-595
    hq = np.einsum('bched,bchd->bche', W2_all, q)
    y = q + np.einsum('bchde,bche->bchd', W1_all, gelu_tanh(hq))
    return y, (W1, W2, S1, S2)


def _pad_inputs(q, k, v, alpha, eta, theta, gamma, cs):
    """memory_layer.py:649-660: pad T up to a multiple of cs with q=k=v=0,
    alpha=1, eta=0, theta=0, gamma=0 (theta=0 zeroes the carried momentum)."""
    T = q.shape[1]
    if T % cs == 0:
        return (_f64(q), _f64(k), _f64(v), _f64(alpha), _f64(eta), _f64(theta),
                None if gamma is None else _f64(gamma))
    pad = cs - T % cs

    def p(x, val):
        widths = [(0, 0)] * x.ndim
        widths[1] = (0, pad)
        return np.pad(_f64(x), widths, constant_values=val)

    return (p(q, 0.0), p(k, 0.0), p(v, 0.0), p(alpha, 1.0), p(eta, 0.0),
            p(theta, 0.0), None if gamma is None else p(gamma, 0.0))


def memory_scan(q, k, v, alpha, eta, theta, gamma, state, chunk_size,
                omega_window, ns_steps):
    """The chunk loop of memory_layer.py:649-718 from already-prepared q,k,v
    (B,T,H,D) and post-sigmoid gates (B,T,H) (eta already times max_lr).
    Returns (y (B,T,H,D), final state (W1, W2, S1, S2))."""
    T_orig = q.shape[1]
    q, k, v, alpha, eta, theta, gamma = _pad_inputs(
        q, k, v, alpha, eta, theta, gamma, chunk_size)
    n_chunks = q.shape[1] // chunk_size
    ys = []
    for c in range(n_chunks):
        sl = slice(c * chunk_size, (c + 1) * chunk_size)
        y_c, state = process_chunk_deep(
            state, q[:, sl], k[:, sl], v[:, sl], alpha[:, sl], eta[:, sl],
            theta[:, sl], None if gamma is None else gamma[:, sl],
            omega_window, ns_steps)
        ys.append(y_c)
    y = np.concatenate(ys, axis=1)[:, :T_orig]
    return y, state


def memory_scan_bruteforce(q, k, v, alpha, eta, theta, gamma, state, chunk_size,
                           omega_window, ns_steps):
    """Per-token restatement of the same recurrence, written independently of
    the batched form: for each (b,h) and token, the inner gradient at the
    chunk-start weights, an explicit window sum, scalar momentum/memory
    recurrences, Polar-Express via the SVD closed form, then the read-out.
    Used only to pin memory_scan."""
    T_orig = q.shape[1]
    q, k, v, alpha, eta, theta, gamma = _pad_inputs(
        q, k, v, alpha, eta, theta, gamma, chunk_size)
    B, T, H, D = q.shape
    W1s, W2s, S1s, S2s = (_f64(s).copy() for s in state)
    y = np.zeros((B, T, H, D))
    use_omega = omega_window > 1 and gamma is not None
    for b in range(B):
        for hh in range(H):
            W1, W2, S1, S2 = W1s[b, hh], W2s[b, hh], S1s[b, hh], S2s[b, hh]
            for c0 in range(0, T, chunk_size):
                W1c, W2c = W1.copy(), W2.copy()
                u1s, u2s = [], []
                for t in range(c0, c0 + chunk_size):
                    kt, vt = k[b, t, hh], v[b, t, hh]
                    pre = W2c @ kt
                    a = gelu_tanh(pre)
                    er = kt + W1c @ a - vt
                    u1s.append((2.0 / D) * np.outer(er, a))
                    ch = (W1c.T @ er) * gelu_derivative(pre)
                    u2s.append((2.0 / D) * np.outer(ch, kt))
                for i, t in enumerate(range(c0, c0 + chunk_size)):
                    if use_omega:
                        lo = max(0, i - omega_window + 1)
                        G1 = sum(gamma[b, c0 + j, hh] * u1s[j] for j in range(lo, i + 1))
                        G2 = sum(gamma[b, c0 + j, hh] * u2s[j] for j in range(lo, i + 1))
                    else:
                        G1, G2 = u1s[i], u2s[i]
                    S1 = theta[b, t, hh] * S1 - eta[b, t, hh] * G1
                    S2 = theta[b, t, hh] * S2 - eta[b, t, hh] * G2
                    W1 = alpha[b, t, hh] * W1 + polar_express_svd(S1, ns_steps)
                    W2 = alpha[b, t, hh] * W2 + polar_express_svd(S2, ns_steps)
                    y[b, t, hh] = q[b, t, hh] + W1 @ gelu_tanh(W2 @ q[b, t, hh])
            W1s[b, hh], W2s[b, hh], S1s[b, hh], S2s[b, hh] = W1, W2, S1, S2
    return y[:, :T_orig], (W1s, W2s, S1s, S2s)


def fused_chunk_regular(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps):
    """kernels/fused_chunk.py:279-314 (_regular_fwd, the operator semantics of
    fused_chunk_scan): momentum scans over precomputed momentum inputs, PE,
    memory scans, read-out y = q + W1_t gelu_tanh(W2_t q)."""
    S1_all, S1 = linear_scan(SW1, theta, momW1)
    S2_all, S2 = linear_scan(SW2, theta, momW2)
    W1_all, W1n = linear_scan(W1, alpha, polar_express(S1_all, ns_steps))
    W2_all, W2n = linear_scan(W2, alpha, polar_express(S2_all, ns_steps))
    q = _f64(q)
    hq = np.einsum('bched,bchd->bche', W2_all, q)
    y = q + np.einsum('bchde,bche->bchd', W1_all, gelu_tanh(hq))
    return y, (W1n, W2n, S1, S2)


# ---------------------------------------------------------------------------
# Layer and model forwards (composition of the above with dense matmuls)
# ---------------------------------------------------------------------------

def initial_model_state(B, H, D, E):
    """model.py:251-264 for one layer: W1=0, W2=[I;0], S=0."""
    W1 = np.zeros((B, H, D, E))
    W2 = np.zeros((B, H, E, D))
    m = min(D, E)
    W2[:, :, :m, :m] = np.eye(m)
    return W1, W2, np.zeros((B, H, D, E)), np.zeros((B, H, E, D))


def memory_layer_prologue(x, p, cfg):
    """memory_layer.py:606-633: projections, causal convs, q/k norm + poly
    (q: norm then poly; k: poly then norm), sigmoid gates with eta*max_lr.
    p holds the layer weights (see atlas_amd.memory_layer for the names)."""
    B, T, C = x.shape
    H, D = cfg['n_head'], cfg['head_dim']
    x = _f64(x)
    q = short_conv(x @ _f64(p['c_q']).T, p['conv_q_w'], p['conv_q_b']).reshape(B, T, H, D)
    k = short_conv(x @ _f64(p['c_k']).T, p['conv_k_w'], p['conv_k_b']).reshape(B, T, H, D)
    v = short_conv(x @ _f64(p['c_v']).T, p['conv_v_w'], p['conv_v_b']).reshape(B, T, H, D)
    if cfg['poly_degree'] > 0:
        q = poly_features(rms_norm(q), p['poly_coeffs'])
        k = rms_norm(poly_features(k, p['poly_coeffs']))
    else:
        q, k = rms_norm(q), rms_norm(k)

    def gate(name):
        return sigmoid(x @ _f64(p[name + '_w']).T + _f64(p[name + '_b']))

    alpha = gate('gate_alpha')
    eta = gate('gate_eta') * cfg['max_lr']
    theta = gate('gate_theta')
    gamma = gate('gate_gamma') if cfg['omega_window'] > 1 else None
    return q, k, v, alpha, eta, theta, gamma


def memory_layer_forward(x, p, cfg, state=None):
    """memory_layer.py:599-727: prologue, default state from W1_init/W2_init
    when none is given (:635-643), the chunk loop, retrieve gate (:720-722)
    and the output projection (:724-725)."""
    B, T, C = x.shape
    H, D, E = cfg['n_head'], cfg['head_dim'], cfg['expand_dim']
    q, k, v, alpha, eta, theta, gamma = memory_layer_prologue(x, p, cfg)
    if state is None:
        W1 = np.broadcast_to(_f64(p['W1_init'])[None], (B, H, D, E)).copy()
        W2 = np.broadcast_to(_f64(p['W2_init'])[None], (B, H, E, D)).copy()
        state = (W1, W2, np.zeros((B, H, D, E)), np.zeros((B, H, E, D)))
    y, state = memory_scan(q, k, v, alpha, eta, theta, gamma, state,
                           cfg['chunk_size'], cfg['omega_window'], cfg['ns_steps'])
    if p.get('retrieve_w') is not None:
        y = y * sigmoid(_f64(x) @ _f64(p['retrieve_w']).T)[..., None]
    y = y.reshape(B, T, H * D) @ _f64(p['c_proj']).T
    return y, state


def mlp_geglu(x, p):
    """model.py:142-167 with geglu_ff=True: h = x W_fc^T, (v, gate) = split(h),
    silu(gate) * v, then the output projection."""
    h = _f64(x) @ _f64(p['mlp_fc']).T
    half = h.shape[-1] // 2
    return (silu(h[..., half:]) * h[..., :half]) @ _f64(p['mlp_proj']).T


def atlas_forward(idx, params, cfg, states=None):
    """model.py:305-374 (no dropout): embedding; persistent memory tokens
    (params['persist_mem'], (n, C), when present) prepended to every row
    (:316-320); per layer x += memory(rms_norm(x), state); x +=
    mlp(rms_norm(x)); final norm, the persistent positions dropped (:359-360),
    lm_head, float logits (optional softcap).  States default to
    initial_model_state.  Returns (logits, per-layer states)."""
    B, T = idx.shape
    H, D, E = cfg['n_head'], cfg['head_dim'], cfg['expand_dim']
    x = _f64(params['wte'])[idx]
    pm = params.get('persist_mem')
    n_persist = 0 if pm is None else pm.shape[0]
    if n_persist:
        x = np.concatenate([np.broadcast_to(_f64(pm)[None], (B,) + pm.shape), x], axis=1)
    new_states = []
    for li, p in enumerate(params['layers']):
        st = initial_model_state(B, H, D, E) if states is None else states[li]
        mem, st = memory_layer_forward(rms_norm(x), p, cfg, st)
        x = x + mem
        x = x + mlp_geglu(rms_norm(x), p)
        new_states.append(st)
    x = rms_norm(x)[:, n_persist:]
    logits = (x @ _f64(params['lm_head']).T)[..., :cfg['vocab_size']]
    if cfg.get('logit_softcap', 0.0) > 0:
        sc = cfg['logit_softcap']
        logits = sc * np.tanh(logits / sc)
    return logits, new_states


# ---------------------------------------------------------------------------
# Sliding-window attention and the MAG model
# ---------------------------------------------------------------------------

def rope_tables(T, D):
    """model.py:49-62: inv_freq = 1/10000^(arange(0, D, 2)/D), angle
    t * inv_freq -> (cos, sin), each (T, D/2)."""
    inv = 1.0 / (10000.0 ** (np.arange(0, D, 2, dtype=np.float64) / D))
    ang = np.outer(np.arange(T, dtype=np.float64), inv)
    return np.cos(ang), np.sin(ang)


def apply_rope(x, cos, sin):
    """model.py:64-73 on (B, T, H, D): halves x1 = x[..., :D/2], x2 = x[..., D/2:]
    -> [x1 cos - x2 sin, x2 cos + x1 sin]."""
    x = _f64(x)
    d2 = x.shape[-1] // 2
    x1, x2 = x[..., :d2], x[..., d2:]
    c = _f64(cos)[None, :, None, :]
    s = _f64(sin)[None, :, None, :]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def swa_core(q, k, v, window, cos=None, sin=None):
    """model.py:109-129 after the qkv projection, on (B, T, H, D): rotate q
    and k, scores q'.k'/sqrt(D), mask causal and t - s <= window (masked
    scores -1e9), softmax over s, weighted sum of v."""
    B, T, H, D = q.shape
    if cos is None:
        cos, sin = rope_tables(T, D)
    qr, kr = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
    sc = np.einsum('bthd,bshd->bhts', qr, kr) / np.sqrt(D)
    t = np.arange(T)[:, None]
    s_ = np.arange(T)[None, :]
    mask = (t >= s_) & ((t - s_) <= window)
    sc = np.where(mask[None, None], sc, -1e9)
    sc = sc - sc.max(axis=-1, keepdims=True)
    p = np.exp(sc)
    p = p / p.sum(axis=-1, keepdims=True)
    return np.einsum('bhts,bshd->bthd', p, _f64(v))


def swa_bruteforce(q, k, v, window):
    """Independent restatement of swa_core for pinning: per (b, h, t), the
    allowed keys s in [max(0, t - window), t] only, each rotation from its own
    angle, softmax shifted by the maximum allowed score."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, T, H, D = q.shape
    d2 = D // 2
    out = np.zeros((B, T, H, D))

    def rot(x, pos):
        y = np.empty(D)
        for i in range(d2):
            a = pos / (10000.0 ** (2.0 * i / D))
            y[i] = x[i] * np.cos(a) - x[i + d2] * np.sin(a)
            y[i + d2] = x[i + d2] * np.cos(a) + x[i] * np.sin(a)
        return y

    for b in range(B):
        for hh in range(H):
            kr = [rot(k[b, s, hh], s) for s in range(T)]
            for t in range(T):
                qt = rot(q[b, t, hh], t)
                keys = range(max(0, t - window), t + 1)
                sc = np.array([qt @ kr[s] for s in keys]) / np.sqrt(D)
                w = np.exp(sc - sc.max())
                w = w / w.sum()
                out[b, t, hh] = sum(wi * v[b, s, hh] for wi, s in zip(w, keys))
    return out


def swa_forward(x, p, cfg):
    """model.py:100-133: rms_norm, qkv projection (split in thirds, heads of
    dim D), swa_core with window_size, output projection."""
    B, T, C = x.shape
    H = cfg['n_head']
    D = cfg['head_dim']
    qkv = rms_norm(x) @ _f64(p['to_qkv']).T
    q, k, v = (qkv[..., i * H * D:(i + 1) * H * D].reshape(B, T, H, D) for i in range(3))
    out = swa_core(q, k, v, cfg['window_size'])
    return out.reshape(B, T, H * D) @ _f64(p['to_out']).T


def memory_gate(x, p):
    """mag_transformer.py:22-32: sigmoid(rms_norm(x) W_g^T + b_g)."""
    return sigmoid(rms_norm(x) @ _f64(p['gate_w']).T + _f64(p['gate_b']))


def mag_forward(idx, params, cfg, states=None):
    """mag_transformer.py:128-166 (no dropout): embedding; per block
    attn = swa_forward(x); with memory mem, st = memory_layer_forward(
    rms_norm(x)) (default state from the layer's W_init when none is given)
    and x = x + attn + memory_gate(mem) * mem, else x = x + attn; then
    x += mlp(rms_norm(x)); final norm and LM head.  Returns (logits, states)."""
    x = _f64(params['wte'])[idx]
    new_states = []
    for li, p in enumerate(params['layers']):
        attn = swa_forward(x, p, cfg)
        st = None
        if p.get('c_q') is not None:
            mem, st = memory_layer_forward(rms_norm(x), p, cfg, None if states is None else states[li])
            x = x + attn + memory_gate(mem, p) * mem
        else:
            x = x + attn
        x = x + mlp_geglu(rms_norm(x), p)
        new_states.append(st)
    x = rms_norm(x)
    return x @ _f64(params['lm_head']).T, new_states

