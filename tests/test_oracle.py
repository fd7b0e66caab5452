"""CPU: pin the float64 oracle (oracle/atlas_ref.py) against known answers,
closed forms and brute force, so that a plausible slip (dropped term, wrong
sign or index, transposed operand) fails here before it can bless a kernel."""

import numpy as np
import pytest
import torch

from oracle import atlas_ref as R
import scan_cases as SC

rng = np.random.default_rng(12345)


# ---------------------------------------------------------------------------
# Polar-Express
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("shape", [(4, 16, 16), (3, 16, 40), (3, 40, 16), (2, 64, 128), (2, 128, 64)])
@pytest.mark.parametrize("ns", [0, 1, 3, 5])
def test_pe_equals_svd_closed_form(shape, ns):
    X = rng.standard_normal(shape)
    assert SC.rel_l2(R.polar_express(X, ns), R.polar_express_svd(X, ns)) < 1e-11


def test_pe_diagonal_acts_elementwise():
    d = np.array([3.0, -1.0, 0.5, 0.0, 2.0])
    X = np.diag(d)[None]
    s = np.sqrt(np.sum(d * d) + 1e-12) * 1.01 + 1e-6
    expect = np.diag(np.sign(d) * R.pe_scalar_map(np.abs(d) / s, 5))
    np.testing.assert_allclose(R.polar_express(X, 5)[0], expect, atol=1e-13)


def test_pe_ns0_is_normalisation_and_zero_maps_to_zero():
    X = rng.standard_normal((2, 8, 12))
    s = np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True) + 1e-12) * 1.01 + 1e-6
    np.testing.assert_allclose(R.polar_express(X, 0), X / s, rtol=1e-14)
    assert np.abs(R.polar_express(np.zeros((1, 8, 8)), 5)).max() == 0.0


def test_pe_reference_invariants():
    """tests/test_polar_express.py:23-95 of the reference."""
    X = rng.standard_normal((4, 32, 32))
    Y = R.polar_express(X, 5)
    for i in range(4):
        YtY = Y[i].T @ Y[i]
        diag = np.diag(YtY)
        assert np.max(np.abs(YtY - np.diag(diag))) < 0.5 * np.mean(np.abs(diag))
    big = R.polar_express(rng.standard_normal((2, 16, 16)) * 100.0, 5)
    assert np.all(np.isfinite(big)) and np.max(np.abs(big)) < 100.0
    Xb = rng.standard_normal((4, 16, 16))
    Yb = R.polar_express(Xb, 5)
    for i in range(4):
        np.testing.assert_allclose(Yb[i], R.polar_express(Xb[i:i + 1], 5)[0], atol=1e-12)
    eye = R.polar_express(np.eye(16)[None], 5)[0]
    assert np.std(np.diag(eye.T @ eye)) < 0.1


def test_muon_pe_uses_eps_free_norm():
    X = rng.standard_normal((2, 24, 40))
    assert SC.rel_l2(R.muon_polar_express(X, 5), R.polar_express_svd(X, 5, norm_eps=0.0)) < 1e-11


def test_pe_pin_detects_planted_mistakes():
    """Copies of polar_express with a dropped c-term, a flipped b sign, the
    coefficient rows in reverse order, or the 1.01 safety factor missing must
    all disagree with the SVD closed form."""
    X = rng.standard_normal((2, 16, 24))
    ref = R.polar_express_svd(X, 5)

    def variant(kind):
        safety = 1.0 if kind == "no_safety" else 1.01
        Y = X / (np.sqrt(np.sum(X * X, axis=(-2, -1), keepdims=True) + 1e-12) * safety + 1e-6)
        rows = R.PE_COEFFS[::-1] if kind == "reversed" else R.PE_COEFFS
        for a, b, c in rows[:5]:
            A = Y @ np.swapaxes(Y, -1, -2)
            if kind == "drop_c":
                Y = a * Y + (b * A) @ Y
            elif kind == "sign_b":
                Y = a * Y + (-b * A + c * A @ A) @ Y
            else:
                Y = a * Y + (b * A + c * A @ A) @ Y
        return Y

    with np.errstate(over="ignore", invalid="ignore"):
        for kind in ("drop_c", "sign_b", "reversed", "no_safety"):
            err = SC.rel_l2(variant(kind), ref)
            assert not np.isfinite(err) or err > 1e-4, kind


# ---------------------------------------------------------------------------
# Elementwise pieces
# ---------------------------------------------------------------------------

def test_gelus_and_derivative():
    x = np.linspace(-6, 6, 2001)
    tx = torch.tensor(x, dtype=torch.float64)
    np.testing.assert_allclose(R.gelu_tanh(x), torch.nn.functional.gelu(tx, approximate="tanh").numpy(),
                               atol=1e-14)
    np.testing.assert_allclose(R.gelu_erf(x), torch.nn.functional.gelu(tx).numpy(), atol=1e-14)
    h = 1e-5
    fd = (R.gelu_erf(x + h) - R.gelu_erf(x - h)) / (2 * h)
    np.testing.assert_allclose(R.gelu_derivative(x), fd, atol=1e-8)
    # the tanh form differs from the erf form (mixing them is the reference's choice)
    assert np.max(np.abs(R.gelu_tanh(x) - R.gelu_erf(x))) > 1e-4


def test_rms_norm_poly_short_conv():
    x = rng.standard_normal((2, 5, 7))
    np.testing.assert_allclose(R.rms_norm(x), x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6))
    np.testing.assert_allclose(R.poly_features(x, [1.0, 1.0]), x + x * x)
    np.testing.assert_allclose(R.poly_features(x, [2.0, 0.5, -1.0]), 2 * x + 0.5 * x ** 2 - x ** 3)
    B, T, C, K = 2, 9, 4, 4
    x = rng.standard_normal((B, T, C))
    w = rng.standard_normal((C, 1, K))
    b = rng.standard_normal(C)
    got = R.short_conv(x, w, b)
    ref = torch.nn.functional.conv1d(torch.nn.functional.pad(torch.tensor(x).transpose(1, 2), (K - 1, 0)),
                                     torch.tensor(w), torch.tensor(b), groups=C).transpose(1, 2).numpy()
    np.testing.assert_allclose(got, ref, atol=1e-12)
    # causality: output at t only depends on x[<= t]
    x2 = x.copy()
    x2[:, 5:] += 1.0
    np.testing.assert_allclose(R.short_conv(x2, w, b)[:, :5], got[:, :5])


# ---------------------------------------------------------------------------
# Scans and the Omega window (reference tests/test_omega.py, test_memory_layer.py)
# ---------------------------------------------------------------------------

def test_linear_scan_known_answer():
    B, T, H, D = 2, 4, 2, 3
    h0 = rng.standard_normal((B, H, D))
    g = 1 / (1 + np.exp(-rng.standard_normal((B, T, H))))
    x = rng.standard_normal((B, T, H, D))
    h_all, h_fin = R.linear_scan(h0, g, x)
    h = h0
    for t in range(T):
        h = g[:, t, :, None] * h + x[:, t]
        np.testing.assert_allclose(h_all[:, t], h, atol=1e-14)
    np.testing.assert_allclose(h_fin, h)
    # closed form: h_T = prod g h0 + sum_s prod_{r>s} g x_s
    cf = np.prod(g, axis=1)[..., None] * h0
    for s in range(T):
        cf = cf + np.prod(g[:, s + 1:], axis=1)[..., None] * x[:, s]
    np.testing.assert_allclose(h_fin, cf, atol=1e-13)


def test_omega_known_answers():
    u = rng.standard_normal((2, 8, 4, 16))
    ones = np.ones((2, 8, 4, 1))
    np.testing.assert_allclose(R.omega_aggregate(u, ones, 1), u)
    np.testing.assert_allclose(R.omega_aggregate(u, ones, 8), np.cumsum(u, axis=1))
    u2 = rng.standard_normal((1, 8, 2, 4))
    g = 1 / (1 + np.exp(-rng.standard_normal((1, 8, 2, 1))))
    naive = np.zeros_like(u2)
    for t in range(8):
        for i in range(max(0, t - 3 + 1), t + 1):
            naive[:, t] += g[:, i] * u2[:, i]
    np.testing.assert_allclose(R.omega_aggregate(u2, g, 3), naive, atol=1e-14)
    mask = np.array([1.0, 0.0, 1.0, 0.0]).reshape(1, 4, 1, 1)
    res = R.omega_aggregate(np.ones((1, 4, 1, 2)), mask, 4)
    np.testing.assert_allclose(res[0, :, 0, 0], [1.0, 1.0, 2.0, 2.0])


def test_inner_gradient_u_w1_is_autograd():
    """u_W1 (memory_layer.py:516) = d/dW1 of (1/D)||k + W1 gelu_tanh(W2 k) - v||^2."""
    D, E = 6, 10
    W1 = torch.tensor(rng.standard_normal((D, E)), requires_grad=True)
    W2 = torch.tensor(rng.standard_normal((E, D)))
    k = torch.tensor(rng.standard_normal(D))
    v = torch.tensor(rng.standard_normal(D))
    act = torch.nn.functional.gelu(W2 @ k, approximate="tanh")
    loss = ((k + W1 @ act - v) ** 2).sum() / D
    loss.backward()
    err = (k + W1 @ act - v).detach().numpy()
    np.testing.assert_allclose(W1.grad.numpy(), (2.0 / D) * np.outer(err, act.detach().numpy()), atol=1e-13)


# ---------------------------------------------------------------------------
# Whole chunk loop: batched restatement vs per-token brute force (SVD-form PE)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T,w,gamma,ns", [(32, 4, True, 5), (32, 1, False, 3), (27, 16, True, 5),
                                          (24, 8, False, 0), (16, 3, True, 1)])
def test_memory_scan_matches_bruteforce(T, w, gamma, ns):
    inp = SC.make_inputs(1, T, 2, 8, 16, seed=T + w, with_gamma=gamma, s_scale=0.01)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"], inp["state"],
            8, w, ns)
    y, st = R.memory_scan(*args)
    yb, sb = R.memory_scan_bruteforce(*args)
    assert SC.rel_l2(y, yb) < 1e-11
    for a, b in zip(st, sb):
        if np.linalg.norm(b) == 0:
            assert np.abs(a).max() == 0
        else:
            assert SC.rel_l2(a, b) < 1e-11


def test_padding_zeroes_momentum_keeps_memory():
    inp = SC.make_inputs(1, 20, 2, 8, 16, seed=3, s_scale=0.01)
    y, st = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"],
                          inp["state"], 8, 4, 5)
    assert y.shape == (1, 20, 2, 8)
    assert np.abs(st[2]).max() == 0 and np.abs(st[3]).max() == 0
    assert np.linalg.norm(st[0]) > 0


def test_fused_chunk_regular_consistent_with_chunk_body():
    """fused_chunk.py:279-314 semantics: feeding the chunk body's own momentum
    inputs reproduces process_chunk_deep."""
    inp = SC.make_inputs(2, 8, 2, 8, 16, seed=5, s_scale=0.01)
    q, k, v = inp["q"], inp["k"], inp["v"]
    W1, W2, S1, S2 = inp["state"]
    y, st = R.process_chunk_deep(inp["state"], q, k, v, inp["alpha"], inp["eta"], inp["theta"], inp["gamma"], 4, 5)
    # recompute the momentum inputs exactly as :505-533
    h = np.einsum('bhed,bchd->bche', W2, k)
    act = R.gelu_tanh(h)
    err = k + np.einsum('bhde,bche->bchd', W1, act) - v
    u1 = (2 / 8) * np.einsum('bchd,bche->bchde', err, act)
    u2 = (2 / 8) * np.einsum('bche,bchd->bched',
                             np.einsum('bhde,bchd->bche', W1, err) * R.gelu_derivative(h), k)
    g = inp["gamma"][..., None, None]
    u1, u2 = R.omega_aggregate(u1, g, 4), R.omega_aggregate(u2, g, 4)
    e = inp["eta"][..., None, None]
    yf, sf = R.fused_chunk_regular(W1, W2, S1, S2, -e * u1, -e * u2, inp["theta"], inp["alpha"], q, 5)
    assert SC.rel_l2(yf, y) < 1e-12
    for a, b in zip(sf, st):
        assert SC.rel_l2(a, b) < 1e-12


# ---------------------------------------------------------------------------
# Muon leaf update (optim.py:56-108)
# ---------------------------------------------------------------------------

def test_muon_leaf_update_known_answers():
    rng = np.random.default_rng(3)
    for shape in [(24, 40), (40, 24)]:
        G = rng.standard_normal(shape)
        zeros = np.zeros(shape)
        sm_shape = (shape[0], 1) if shape[0] >= shape[1] else (1, shape[1])
        # momentum 0, beta2 0, no decay: the update is -lr * lr_scale * NorMuon(PE(G))
        upd, mom, sec = R.muon_leaf_update(G, zeros, np.zeros(sm_shape), None, 0.1, 0.0, 0.0, 0.0, 5)
        assert np.allclose(mom, G)
        P = R.muon_polar_express(G, 5)
        lr_scale = max(1.0, shape[0] / shape[1]) ** 0.5
        g = -upd / (0.1 * lr_scale)
        red = -1 if shape[0] >= shape[1] else -2
        ms = np.mean(g * g, axis=red)
        # NorMuon with beta2 = 0 equalises the mean squares along the kept axis ...
        assert np.allclose(ms, ms.mean(), rtol=1e-9)
        # ... and keeps the Frobenius norm of the orthogonalised direction
        assert abs(np.linalg.norm(g) - np.linalg.norm(P)) < 1e-9 * np.linalg.norm(P)
        # Nesterov: with momentum m, g = (1-m) grad + m * new_momentum
        upd2, mom2, _ = R.muon_leaf_update(G, G, np.ones(sm_shape), None, 0.1, 0.5, 0.9, 0.0, 0)
        assert np.allclose(mom2, G)
        # cautious weight decay acts only where sign(update direction) == sign(param)
        W = rng.standard_normal(shape)
        u0, _, _ = R.muon_leaf_update(G, zeros, np.zeros(sm_shape), None, 0.1, 0.0, 0.0, 0.0, 5)
        u1, _, _ = R.muon_leaf_update(G, zeros, np.zeros(sm_shape), W, 0.1, 0.0, 0.0, 0.5, 5)
        mask = ((-u0) * W) >= 0
        assert np.allclose(u1 - u0, -0.1 * lr_scale * 0.5 * W * mask)
