"""NumPy model of the chunk decomposition the HIP scan kernels implement.

This is a CPU statement of the product's algorithm (not of the reference): it
lets the CPU test-suite check the decomposition against the oracle without a
GPU.  Per (batch, head) stream and chunk of cs tokens, with the chunk-start
state (W1, W2, S1, S2):

  prep    H = K W2^T, Act = gelu_tanh(H), Gp = gelu'(H), Err = K + Act W1^T - V,
          Chain = (Err W1) * Gp                      (all at chunk-start weights)
  coeffs  Theta_t = prod_{r<=t} theta_r
          c[t,i]  = (2/D) g_i sum_{s=i}^{min(t,i+w-1)} theta(s->t) (-eta_s), i<=t
                    (g_i = gamma_i with an Omega window, else 1 and w = 1)
          A_t = prod_{r<=t} alpha_r,  a(s->t) = prod_{s<r<=t} alpha_r
  S_t     S1_t   = Theta_t S1 + Err^T diag(c[t]) Act        (D x E)
          S2_t^T = Theta_t S2^T + K^T diag(c[t]) Chain      (D x E)
  PE      P1_t = PE(S1_t), P2_t^T = PE(S2_t^T) (wide form)
  slices  tokens split in n_slices slices T_j with last token end_j
          L_j   = sum_{s in T_j} a(s->end_j) P_s
          h_t   = A_t W2 q_t + sum_{i<j} a(end_i->t) L2_i^T q_t + sum_{s in T_j,s<=t} a(s->t) P2_s q_t
          y_t   = q_t + A_t W1 g_t + sum_{i<j} a(end_i->t) L1_i g_t + sum_{s in T_j,s<=t} a(s->t) P1_s g_t
          W_end = A_{cs-1} W + sum_j a(end_j->cs-1) L_j,   S_end = S_{cs-1}
"""

import numpy as np

from oracle import atlas_ref as R


def chunk_coefficients(alpha, eta, theta, gamma, omega_window, D):
    cs = len(theta)
    use_omega = omega_window > 1 and gamma is not None
    w = omega_window if use_omega else 1
    c = np.zeros((cs, cs))
    Theta = np.cumprod(theta)
    for t in range(cs):
        m = np.zeros(cs)
        prod = 1.0
        for s in range(t, -1, -1):
            m[s] = prod * (-eta[s])
            prod *= theta[s]
        for i in range(t + 1):
            c[t, i] = m[i:min(t, i + w - 1) + 1].sum() * (gamma[i] if use_omega else 1.0)
    c *= 2.0 / D
    A = np.cumprod(alpha)

    def a(s, t):  # prod_{s<r<=t} alpha_r
        return np.prod(alpha[s + 1:t + 1])

    return c, Theta, A, a


def chunk_step(state, q, k, v, alpha, eta, theta, gamma, omega_window, ns_steps, n_slices):
    """One chunk for one stream.  q,k,v (cs,D); gates (cs,).  state fp64
    (W1 (D,E), W2 (E,D), S1 (D,E), S2 (E,D)).  Returns (y (cs,D), state)."""
    W1, W2, S1, S2 = state
    cs, D = q.shape
    H = k @ W2.T
    act, gp = R.gelu_tanh(H), R.gelu_derivative(H)
    err = k + act @ W1.T - v
    chain = (err @ W1) * gp
    c, Theta, A, a = chunk_coefficients(alpha, eta, theta, gamma, omega_window, D)
    P1, P2T = [], []
    for t in range(cs):
        S1t = Theta[t] * S1 + err.T @ (c[t][:, None] * act)
        S2Tt = Theta[t] * S2.T + k.T @ (c[t][:, None] * chain)
        P1.append(R.polar_express(S1t, ns_steps))
        P2T.append(R.polar_express(S2Tt, ns_steps))   # wide D x E form
    TS = cs // n_slices
    ends = [(j + 1) * TS - 1 for j in range(n_slices)]
    L1 = [sum(a(s, ends[j]) * P1[s] for s in range(j * TS, ends[j] + 1)) for j in range(n_slices)]
    L2 = [sum(a(s, ends[j]) * P2T[s] for s in range(j * TS, ends[j] + 1)) for j in range(n_slices)]
    y = np.zeros((cs, D))
    for j in range(n_slices):
        for t in range(j * TS, ends[j] + 1):
            h = A[t] * (W2 @ q[t]) + sum(a(ends[i], t) * (L2[i].T @ q[t]) for i in range(j))
            h = h + sum(a(s, t) * (P2T[s].T @ q[t]) for s in range(j * TS, t + 1))
            g = R.gelu_tanh(h)
            yt = A[t] * (W1 @ g) + sum(a(ends[i], t) * (L1[i] @ g) for i in range(j))
            yt = yt + sum(a(s, t) * (P1[s] @ g) for s in range(j * TS, t + 1))
            y[t] = q[t] + yt
    W1n = A[-1] * W1 + sum(a(ends[j], cs - 1) * L1[j] for j in range(n_slices))
    W2n = A[-1] * W2 + sum(a(ends[j], cs - 1) * L2[j].T for j in range(n_slices))
    S1n = Theta[-1] * S1 + err.T @ (c[-1][:, None] * act)
    S2n = (Theta[-1] * S2.T + k.T @ (c[-1][:, None] * chain)).T
    return y, (W1n, W2n, S1n, S2n)


def scan(q, k, v, alpha, eta, theta, gamma, state, cs, omega_window, ns_steps, n_slices):
    """Whole-sequence driver over (B,T,H,...) inputs with T % cs == 0."""
    B, T, H, D = q.shape
    W1, W2, S1, S2 = (np.array(s, dtype=np.float64) for s in state)
    y = np.zeros((B, T, H, D))
    for b in range(B):
        for h in range(H):
            st = (W1[b, h], W2[b, h], S1[b, h], S2[b, h])
            for c0 in range(0, T, cs):
                sl = slice(c0, c0 + cs)
                g = None if gamma is None else gamma[b, sl, h]
                y[b, sl, h], st = chunk_step(st, q[b, sl, h], k[b, sl, h], v[b, sl, h],
                                             alpha[b, sl, h], eta[b, sl, h], theta[b, sl, h],
                                             g, omega_window, ns_steps, n_slices)
            W1[b, h], W2[b, h], S1[b, h], S2[b, h] = st
    return y, (W1, W2, S1, S2)
