"""CPU: pins of the gradient oracle (oracle/atlas_ref_torch.py) -- its
forward against the NumPy oracle and its autograd gradients against finite
differences -- and the product's fp32 Polar-Express VJP helper
(atlas_amd.autograd.polar_express_vjp, pure torch) against it."""

import numpy as np
import pytest
import torch

import __graft_entry__  # noqa: F401  (sets sys.path)
from oracle import atlas_ref as R
from oracle import atlas_ref_torch as RT


def _inputs(B, cs, H, D, E, seed):
    rng = np.random.default_rng(seed)
    W1 = rng.standard_normal((B, H, D, E)) / np.sqrt(D)
    W2 = rng.standard_normal((B, H, E, D)) / np.sqrt(D)
    SW1 = rng.standard_normal((B, H, D, E)) * 0.1
    SW2 = rng.standard_normal((B, H, E, D)) * 0.1
    m1 = rng.standard_normal((B, cs, H, D, E)) * 0.1
    m2 = rng.standard_normal((B, cs, H, E, D)) * 0.1
    theta = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, cs, H))))
    alpha = 1.0 / (1.0 + np.exp(-rng.standard_normal((B, cs, H))))
    q = rng.standard_normal((B, cs, H, D))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    return [W1, W2, SW1, SW2, m1, m2, theta, alpha, q]


def test_torch_oracle_forward_matches_numpy_oracle():
    xs = _inputs(2, 5, 2, 4, 8, seed=0)
    out_t = RT.fused_chunk_regular_t(*(torch.tensor(a) for a in xs), 5)
    y, st = R.fused_chunk_regular(*xs, 5)
    np.testing.assert_allclose(out_t[0].numpy(), y, rtol=1e-12, atol=1e-12)
    for a, b in zip(out_t[1:], st):
        np.testing.assert_allclose(a.numpy(), b, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("pe_ste", [False, True])
def test_torch_oracle_gradients_match_finite_differences(pe_ste):
    xs = [torch.tensor(a).requires_grad_(True) for a in _inputs(1, 3, 1, 2, 4, seed=1)]

    def f(*args):
        return RT.fused_chunk_regular_t(*args, 3, pe_ste)

    if pe_ste:
        # the straight-through backward is not the derivative of the forward;
        # it is the derivative of the surrogate with P = S + C, C = PE(S) - S
        # frozen at the base point: finite differences check that surrogate,
        # and the STE gradients must equal its gradients at the base point
        W1, W2, SW1, SW2, m1, m2, th, al, q = (x.detach() for x in xs)
        C1 = RT.polar_express_t(RT.linear_scan_t(SW1, th, m1)[0], 3) - RT.linear_scan_t(SW1, th, m1)[0]
        C2 = RT.polar_express_t(RT.linear_scan_t(SW2, th, m2)[0], 3) - RT.linear_scan_t(SW2, th, m2)[0]

        def f_lin(*args):
            W1, W2, SW1, SW2, m1, m2, th, al, q = args
            S1_all, S1 = RT.linear_scan_t(SW1, th, m1)
            S2_all, S2 = RT.linear_scan_t(SW2, th, m2)
            W1_all, W1e = RT.linear_scan_t(W1, al, S1_all + C1)
            W2_all, W2e = RT.linear_scan_t(W2, al, S2_all + C2)
            h = torch.einsum("bched,bchd->bche", W2_all, q)
            y = q + torch.einsum("bchde,bche->bchd", W1_all, RT.gelu_tanh_t(h))
            return y, W1e, W2e, S1, S2
        assert torch.autograd.gradcheck(f_lin, xs, eps=1e-6, atol=1e-6, rtol=1e-5)
        cts = [torch.randn_like(o) for o in f(*xs)]
        g1 = torch.autograd.grad(f(*xs), xs, cts)
        g2 = torch.autograd.grad(f_lin(*xs), xs, cts)
        for a, b in zip(g1, g2):
            torch.testing.assert_close(a, b, rtol=1e-10, atol=1e-12)
    else:
        assert torch.autograd.gradcheck(f, xs, eps=1e-6, atol=1e-6, rtol=1e-5)


@pytest.mark.parametrize("shape,steps", [((3, 8, 16), 5), ((2, 16, 8), 5), ((2, 6, 6), 3), ((1, 4, 12), 0)])
def test_polar_express_vjp_helper(shape, steps):
    from atlas_amd.autograd import polar_express_vjp
    g = torch.Generator().manual_seed(7)
    X = torch.randn(*shape, generator=g, dtype=torch.float64)
    G = torch.randn(*shape, generator=g, dtype=torch.float64)
    Xr = X.clone().requires_grad_(True)
    ref, = torch.autograd.grad(RT.polar_express_t(Xr, steps), Xr, G)
    got = polar_express_vjp(X.float(), G.float(), steps).double()
    err = ((got - ref).norm() / ref.norm()).item()
    assert err < 1e-4, err


def _layer_inputs(B, T, H, D, E, seed, with_gamma=True):
    import scan_cases as SC
    inp = SC.make_inputs(B, T, H, D, E, seed=seed, with_gamma=with_gamma, s_scale=0.1)
    return inp, [torch.tensor(inp[n]) for n in ("q", "k", "v", "alpha", "eta", "theta")]


@pytest.mark.parametrize("T,cs,w,with_gamma", [(11, 4, 3, True), (8, 4, 8, True), (9, 3, 1, False)])
def test_layer_oracle_forward_matches_numpy_oracle(T, cs, w, with_gamma):
    """memory_scan_t (the whole-layer gradient oracle) computes the same
    values as the NumPy chunk loop and as its per-token brute force."""
    inp, ts = _layer_inputs(1, T, 2, 4, 8, seed=T + w, with_gamma=with_gamma)
    gam = None if inp["gamma"] is None else torch.tensor(inp["gamma"])
    st = [torch.tensor(s) for s in inp["state"]]
    y_t, st_t = RT.memory_scan_t(*ts, gam, st, cs, w, 5)
    args = (inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"], inp["gamma"], inp["state"],
            cs, w, 5)
    for y_r, st_r in (R.memory_scan(*args), R.memory_scan_bruteforce(*args)):
        np.testing.assert_allclose(y_t.numpy(), y_r, rtol=1e-10, atol=1e-12)
        for a, b in zip(st_t, st_r):
            np.testing.assert_allclose(a.numpy(), b, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("pe_ste", [False, True])
def test_layer_oracle_gradients_match_finite_differences(pe_ste):
    """Gradients of the whole-layer oracle (through the inner gradient, the
    Omega window, padding and three chunks) against finite differences.
    With pe_ste the backward is that of the surrogate whose Polar-Express
    correction is frozen, so only the plain form is checked by finite
    differences; the STE form must differ from it (the identity backward is
    really taken) and agree with it when ns=0 turns PE into a pure scaling
    whose own derivative is dropped."""
    inp, ts = _layer_inputs(1, 5, 1, 2, 4, seed=3)
    xs = [t.clone().requires_grad_(True) for t in ts + [torch.tensor(inp["gamma"])]
          + [torch.tensor(s) for s in inp["state"]]]

    def f(ns, ste):
        def g(q, k, v, a, e, th, ga, W1, W2, S1, S2):
            y, st = RT.memory_scan_t(q, k, v, a, e, th, ga, (W1, W2, S1, S2), 2, 2, ns, ste)
            return (y, *st)
        return g

    if not pe_ste:
        # Polar-Express of a 2x4 iterate is strongly curved here (Jacobian
        # entries ~1e3): a central difference needs eps=1e-7 to reach the
        # analytic value to ~1e-6 (at eps=1e-6 its own truncation error is ~1 %)
        assert torch.autograd.gradcheck(f(3, False), xs, eps=1e-7, atol=1e-5, rtol=1e-5)
    else:
        outs = f(3, False)(*xs)
        cts = [torch.randn_like(o) for o in outs]
        g_plain = torch.autograd.grad(outs, xs, cts)
        g_ste = torch.autograd.grad(f(3, True)(*xs), xs, cts)
        assert any((a - b).abs().max() > 1e-6 for a, b in zip(g_plain, g_ste))


def test_product_omega_aggregate_matches_window_sum():
    """autograd._omega_aggregate (cumsum minus shifted cumsum, as
    memory_layer.py:233-253) equals the oracle's explicit window sum, for a
    window shorter than, equal to and longer than the chunk."""
    from atlas_amd.autograd import _omega_aggregate
    g = torch.Generator().manual_seed(5)
    u = torch.randn(2, 7, 3, 4, 5, generator=g, dtype=torch.float64)
    gam = torch.rand(2, 7, 3, generator=g, dtype=torch.float64)
    for w in (1, 3, 7, 9):
        torch.testing.assert_close(_omega_aggregate(u, gam, w), RT.omega_aggregate_t(u, gam, w),
                                   rtol=1e-12, atol=1e-12)


def test_layer_oracle_stop_grad_chunks_equals_independent_chunks():
    """With stop_grad_chunks the carry is detached at every chunk start,
    the first included (memory_layer.py:664-665 applies stop_gradient inside
    chunk_body): the gradients of chunk c's inputs must equal those of a
    one-chunk call started from chunk c's state taken as a constant, and the
    initial state receives no gradient."""
    import scan_cases as SC
    inp, ts = _layer_inputs(1, 12, 2, 4, 8, seed=9)
    gam = torch.tensor(inp["gamma"])
    cs, w = 4, 3
    xs = [t.clone().requires_grad_(True) for t in ts + [gam]]
    s0 = [torch.tensor(s).requires_grad_(True) for s in inp["state"]]
    y, fin = RT.memory_scan_t(*xs[:6], xs[6], tuple(s0), cs, w, 5, stop_grad_chunks=True)
    g = torch.Generator().manual_seed(2)
    cts = [torch.randn(o.shape, generator=g, dtype=torch.float64) for o in (y, *fin)]
    grads = torch.autograd.grad((y, *fin), xs + s0, cts, allow_unused=True)
    assert all(gs is None for gs in grads[7:])
    _, starts = SC.oracle_trajectory(inp, cs, w, 5)
    for c in range(3):
        sl = slice(c * cs, (c + 1) * cs)
        xc = [t[:, sl].detach().clone().requires_grad_(True) for t in ts + [gam]]
        yc, fc = RT.memory_scan_t(*xc[:6], xc[6], tuple(torch.tensor(s) for s in starts[c]), cs, w, 5)
        outs, cc = [yc], [cts[0][:, sl]]
        if c == 2:
            outs += list(fc)
            cc += cts[1:]
        gc = torch.autograd.grad(outs, xc, cc)
        for a, b in zip(grads[:7], gc):
            torch.testing.assert_close(a[:, sl], b, rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------------------
# Whole-model gradient oracle: torch float64 Atlas / MAG forwards
# ---------------------------------------------------------------------------

def _model_cfg(**kw):
    c = dict(n_head=2, head_dim=4, expand_dim=8, poly_degree=2, max_lr=0.1, omega_window=3, chunk_size=4,
             ns_steps=3, vocab_size=20, logit_softcap=15.0, window_size=3)
    c.update(kw)
    return c


def _model_params(cfg, C, n_layer=2, mag=False, seed=0):
    import test_oracle_model as TOM
    TOM.rng = np.random.default_rng(seed)
    return TOM._model_params(cfg, C, n_layer=n_layer, conv_k=2, mag=mag, mem_layers=(1,) if mag else None)


def _to_t(params, requires_grad=False):
    def conv(a):
        return None if a is None else torch.tensor(a, dtype=torch.float64, requires_grad=requires_grad)
    out = {"wte": conv(params["wte"]), "lm_head": conv(params["lm_head"]),
           "layers": [{k: conv(v) for k, v in p.items()} for p in params["layers"]]}
    if params.get("persist_mem") is not None:
        out["persist_mem"] = conv(params["persist_mem"])
    return out


def test_torch_model_forwards_match_numpy_oracle():
    """atlas_forward_t / mag_forward_t equal the pinned NumPy atlas_forward /
    mag_forward (ragged T, carried states) to 1e-12."""
    cfg = _model_cfg()
    params = _model_params(cfg, 8)
    idx = np.random.default_rng(1).integers(0, cfg["vocab_size"], (2, 10))
    lt, st_t = RT.atlas_forward_t(torch.tensor(idx), _to_t(params), cfg)
    ln, st_n = R.atlas_forward(idx, params, cfg)
    np.testing.assert_allclose(lt.numpy(), ln, rtol=1e-10, atol=1e-10)
    for a, b in zip(st_t, st_n):
        for x, y in zip(a, b):
            np.testing.assert_allclose(x.numpy(), y, rtol=1e-10, atol=1e-10)
    lt2, _ = RT.atlas_forward_t(torch.tensor(idx[:, :3]), _to_t(params), cfg, st_t)
    ln2, _ = R.atlas_forward(idx[:, :3], params, cfg, st_n)
    np.testing.assert_allclose(lt2.numpy(), ln2, rtol=1e-10, atol=1e-10)
    mparams = _model_params(cfg, 8, mag=True, seed=3)
    lm_t, _ = RT.mag_forward_t(torch.tensor(idx), _to_t(mparams), cfg)
    lm_n, _ = R.mag_forward(idx, mparams, cfg)
    np.testing.assert_allclose(lm_t.numpy(), lm_n, rtol=1e-10, atol=1e-10)
    # persistent memory tokens (model.py:316-320, 359-360)
    pparams = dict(params, persist_mem=np.random.default_rng(6).standard_normal((3, 8)) * 0.5)
    lp_t, _ = RT.atlas_forward_t(torch.tensor(idx), _to_t(pparams), cfg)
    lp_n, _ = R.atlas_forward(idx, pparams, cfg)
    assert lp_t.shape == (2, 10, cfg["vocab_size"])
    np.testing.assert_allclose(lp_t.numpy(), lp_n, rtol=1e-10, atol=1e-10)


@pytest.mark.parametrize("mag", [False, True])
def test_torch_model_gradients_match_finite_differences(mag):
    """Autograd of the float64 model forwards against central differences on
    random coordinates of every parameter tensor (loss = sum(logits * R))."""
    cfg = _model_cfg()
    params = _model_params(cfg, 8, mag=mag, seed=5)
    idx = torch.tensor(np.random.default_rng(2).integers(0, cfg["vocab_size"], (1, 7)))
    Rw = torch.tensor(np.random.default_rng(4).standard_normal((1, 7, cfg["vocab_size"])))
    fwd = RT.mag_forward_t if mag else RT.atlas_forward_t
    pt = _to_t(params, requires_grad=True)
    (fwd(idx, pt, cfg)[0] * Rw).sum().backward()
    leaves = [("wte", pt["wte"]), ("lm_head", pt["lm_head"])] + [
        (f"{li}.{k}", v) for li, p in enumerate(pt["layers"]) for k, v in p.items() if v is not None]
    rng = np.random.default_rng(6)
    h = 1e-6
    for name, t in leaves:
        for _ in range(2):
            i = int(rng.integers(t.numel()))
            with torch.no_grad():
                flat = t.view(-1)
                old = flat[i].item()
                flat[i] = old + h
                up = (fwd(idx, pt, cfg)[0] * Rw).sum().item()
                flat[i] = old - h
                dn = (fwd(idx, pt, cfg)[0] * Rw).sum().item()
                flat[i] = old
            fd = (up - dn) / (2 * h)
            # W1_init / W2_init are unused by the Atlas forward (it passes the
            # model initial state, model.py:322-326): no gradient at all
            g = 0.0 if t.grad is None else t.grad.view(-1)[i].item()
            assert abs(fd - g) <= 1e-6 + 1e-5 * abs(fd), (name, i, fd, g)
