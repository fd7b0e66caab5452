"""CPU: pins for the oracle's compositions (oracle/atlas_ref.py) -- the inner
gradient u_W2, the layer prologue, the GEGLU MLP, the MAG memory gate, the
attention block, and the Atlas / MAG model forwards.

None of these has reference vectors, so each is pinned by an identity that
the mathematics fixes (an autograd identity, an invariant, a special case
that reduces to a closed form, causality, state carry), and each test also
plants a plausible mistake in a copy of the oracle and checks that the same
identity rejects it.  Reference spans: memory_layer.py:505-520 (inner
gradient), :606-633 (prologue), :649-660 (padding), :720-725 (retrieve gate
and output projection); model.py:160-163 (GEGLU), :100-133 (attention),
:305-374 (Atlas forward); mag_transformer.py:22-32 (MemoryGate), :63-79
(MAGBlock), :128-166 (MAG forward); tests/test_model.py:74-97 and
tests/test_memory_layer.py:161-172 (padding, continuation, persistence)."""

import copy

import numpy as np
import pytest
import torch

from oracle import atlas_ref as R
import scan_cases as SC

rng = np.random.default_rng(2024)


def _cfg(**kw):
    c = dict(n_head=2, head_dim=8, expand_dim=16, poly_degree=2, max_lr=0.1, omega_window=4, chunk_size=8,
             ns_steps=3, vocab_size=50, logit_softcap=0.0, window_size=5)
    c.update(kw)
    return c


def _layer_params(cfg, C, conv_k=4, mlp=True, attn=False, gate=False, retrieve=True):
    H, D, E = cfg["n_head"], cfg["head_dim"], cfg["expand_dim"]
    g = lambda *s, sd=1.0: rng.standard_normal(s) * sd  # noqa: E731
    p = {"c_q": g(H * D, C, sd=C ** -0.5), "c_k": g(H * D, C, sd=C ** -0.5), "c_v": g(H * D, C, sd=C ** -0.5),
         "c_proj": g(C, H * D, sd=(H * D) ** -0.5),
         "poly_coeffs": np.linspace(1.0, 0.6, cfg["poly_degree"]) if cfg["poly_degree"] else None,
         "W1_init": g(H, D, E, sd=D ** -0.5), "W2_init": g(H, E, D, sd=D ** -0.5),
         "retrieve_w": g(H, C, sd=0.3) if retrieve else None}
    for c in "qkv":
        p[f"conv_{c}_w"], p[f"conv_{c}_b"] = g(H * D, 1, conv_k, sd=0.5), g(H * D, sd=0.1)
    for name in ("alpha", "eta", "theta", "gamma"):
        p[f"gate_{name}_w"], p[f"gate_{name}_b"] = g(H, C, sd=0.3), g(H, sd=1.0)
    if mlp:
        inner = 12
        p["mlp_fc"], p["mlp_proj"] = g(2 * inner, C, sd=C ** -0.5), g(C, inner, sd=inner ** -0.5)
    if attn:
        p["to_qkv"], p["to_out"] = g(3 * H * D, C, sd=C ** -0.5), g(C, H * D, sd=(H * D) ** -0.5)
    if gate:
        p["gate_w"], p["gate_b"] = g(C, C, sd=C ** -0.5), g(C, sd=0.5)
    return p


def _model_params(cfg, C, n_layer=2, conv_k=4, mag=False, mem_layers=None):
    layers = []
    for li in range(n_layer):
        has_mem = mem_layers is None or li in mem_layers
        p = _layer_params(cfg, C, conv_k=conv_k, attn=mag, gate=mag and has_mem)
        if not has_mem:
            p = {k: v for k, v in p.items() if k in ("mlp_fc", "mlp_proj", "to_qkv", "to_out")}
        layers.append(p)
    return {"wte": rng.standard_normal((cfg["vocab_size"], C)),
            "lm_head": rng.standard_normal((cfg["vocab_size"], C)) * 0.2, "layers": layers}


# ---------------------------------------------------------------------------
# Inner gradient: u_W2 is the autograd gradient of a surrogate
# ---------------------------------------------------------------------------

def _u_w2_autograd(W1, W2, k, v):
    """(2/D) grad_{W2} <sg(err), W1 gelu_erf(W2 k)> with err = k + W1
    gelu_tanh(W2 k) - v held fixed (torch float64 autograd), per token."""
    W1t, kt, vt = (torch.tensor(a) for a in (W1, k, v))
    W2t = torch.tensor(W2, requires_grad=True)
    h = torch.einsum('bhed,bchd->bche', W2t, kt)
    err = (kt + torch.einsum('bhde,bche->bchd', W1t, torch.nn.functional.gelu(h, approximate="tanh")) - vt).detach()
    # one surrogate per token: sum over tokens would merge the per-token
    # gradients, so differentiate each token's term separately
    D = k.shape[-1]
    out = np.zeros(W2.shape[:2] + (k.shape[1],) + W2.shape[2:])   # (B,H,cs,E,D)
    for c in range(k.shape[1]):
        if W2t.grad is not None:
            W2t.grad = None
        hc = torch.einsum('bhed,bhd->bhe', W2t, kt[:, c])
        f = (err[:, c] * torch.einsum('bhde,bhe->bhd', W1t, torch.nn.functional.gelu(hc))).sum()
        f.backward()
        out[:, :, c] = (2.0 / D) * W2t.grad.numpy()
    return np.transpose(out, (0, 2, 1, 3, 4))   # (B,cs,H,E,D)


@pytest.mark.parametrize("D,E", [(6, 10), (8, 8)])
def test_u_w2_is_autograd_of_erf_surrogate(D, E):
    """memory_layer.py:511-520: u_W2 = (2/D)((W1^T err) * gelu_erf'(h)) (x) k
    equals the W2-gradient of <sg(err), W1 gelu_erf(W2 k)>."""
    B, cs, H = 2, 3, 2
    W1, W2 = rng.standard_normal((B, H, D, E)), rng.standard_normal((B, H, E, D))
    k, v = rng.standard_normal((B, cs, H, D)), rng.standard_normal((B, cs, H, D))
    _, u2 = R.inner_gradient(W1, W2, k, v)
    np.testing.assert_allclose(u2, _u_w2_autograd(W1, W2, k, v), atol=1e-12)


def test_u_w2_pin_detects_planted_mistakes():
    """Square D = E so that transposed operands still type-check."""
    D = E = 8
    B, cs, H = 1, 2, 2
    W1, W2 = rng.standard_normal((B, H, D, E)), rng.standard_normal((B, H, E, D))
    k, v = rng.standard_normal((B, cs, H, D)), rng.standard_normal((B, cs, H, D))
    ref = _u_w2_autograd(W1, W2, k, v)

    def variant(kind):
        h = np.einsum('bhed,bchd->bche', W2, k)
        act = R.gelu_tanh(h)
        err = k + np.einsum('bhde,bche->bchd', W1, act) - v
        if kind == "W1_not_transposed":
            back = np.einsum('bhed,bchd->bche', W1, err)
        else:
            back = np.einsum('bhde,bchd->bche', W1, err)
        if kind == "tanh_derivative":
            x = torch.tensor(h, requires_grad=True)
            torch.nn.functional.gelu(x, approximate="tanh").sum().backward()
            deriv = x.grad.numpy()
        else:
            deriv = R.gelu_derivative(h)
        chain = back * deriv
        vec = v if kind == "v_for_k" else k
        return (2.0 / D) * np.einsum('bche,bchd->bched', chain, vec)

    for kind in ("W1_not_transposed", "tanh_derivative", "v_for_k"):
        assert np.max(np.abs(variant(kind) - ref)) > 1e-3, kind
    np.testing.assert_allclose(variant("none"), ref, atol=1e-12)


# ---------------------------------------------------------------------------
# Prologue: q is normalised then mapped, k mapped then normalised
# ---------------------------------------------------------------------------

def test_prologue_norm_poly_order():
    """memory_layer.py:612-616: k = rms_norm(poly(k)) leaves with unit RMS
    per head; q = poly(rms_norm(q)) does not (and rms_norm(q) is recovered
    by inverting the degree-2 map); gates lie in (0, 1), eta in (0, max_lr)."""
    cfg = _cfg()
    C = 16
    p = _layer_params(cfg, C)
    x = rng.standard_normal((2, 11, C))
    q, k, v, al, et, th, ga = R.memory_layer_prologue(x, p, cfg)
    rms = lambda a: np.sqrt(np.mean(a * a, axis=-1))  # noqa: E731
    np.testing.assert_allclose(rms(k), 1.0 / np.sqrt(1.0 + 1e-6 / np.mean(
        R.poly_features(R.short_conv(x @ p["c_k"].T, p["conv_k_w"], p["conv_k_b"]).reshape(2, 11, 2, 8),
                        p["poly_coeffs"]) ** 2, axis=-1)), rtol=1e-12)
    assert np.min(np.abs(rms(q) - 1.0)) > 1e-3
    # with the linear coefficient alone the map is the identity: q leaves
    # with unit RMS as well (norm applied to q before the map)
    q_lin = R.memory_layer_prologue(x, dict(p, poly_coeffs=np.array([1.0, 0.0])), cfg)[0]
    qc = R.short_conv(x @ p["c_q"].T, p["conv_q_w"], p["conv_q_b"]).reshape(2, 11, 2, 8)
    np.testing.assert_allclose(rms(q_lin), 1.0 / np.sqrt(1.0 + 1e-6 / np.mean(qc ** 2, axis=-1)), rtol=1e-12)
    assert 0 < al.min() and al.max() < 1 and 0 < et.min() and et.max() < cfg["max_lr"]
    # planted mistake: swapped order for k breaks the unit RMS
    kc = R.short_conv(x @ p["c_k"].T, p["conv_k_w"], p["conv_k_b"]).reshape(2, 11, 2, 8)
    assert np.max(np.abs(rms(R.poly_features(R.rms_norm(kc), p["poly_coeffs"])) - 1.0)) > 1e-2


# ---------------------------------------------------------------------------
# GEGLU: a saturated gate turns the MLP into its linear value path
# ---------------------------------------------------------------------------

def test_mlp_geglu_split_order():
    """model.py:160-163: v, gate = split(h) and silu(gate) * v.  With the
    input's first coordinate 1 and gate rows (50, 0, ...), silu(gate) = 50 to
    double precision, so the MLP equals 50 * (x W_v^T) W_proj^T; the swapped
    split silu(v) * gate is not linear in x and fails."""
    C, inner = 6, 5
    x = rng.standard_normal((3, 4, C))
    x[..., 0] = 1.0
    Wv = rng.standard_normal((inner, C))
    Wg = np.zeros((inner, C))
    Wg[:, 0] = 50.0
    p = {"mlp_fc": np.concatenate([Wv, Wg], 0), "mlp_proj": rng.standard_normal((C, inner))}
    lin = 50.0 * (x @ Wv.T) @ p["mlp_proj"].T
    np.testing.assert_allclose(R.mlp_geglu(x, p), lin, rtol=1e-12)
    h = x @ p["mlp_fc"].T
    swapped = (R.silu(h[..., :inner]) * h[..., inner:]) @ p["mlp_proj"].T
    assert np.max(np.abs(swapped - lin)) > 1.0


# ---------------------------------------------------------------------------
# MAG memory gate
# ---------------------------------------------------------------------------

def test_memory_gate_zero_weight_and_norm():
    """mag_transformer.py:22-32: zero weights give sigmoid(b) everywhere; with
    W = c I and b = 0 the pre-activation logit(g)/c is rms_norm(x), which has
    unit RMS per row (a gate without the norm fails)."""
    C = 7
    x = rng.standard_normal((2, 5, C)) * 3.0
    b = rng.standard_normal(C)
    g0 = R.memory_gate(x, {"gate_w": np.zeros((C, C)), "gate_b": b})
    np.testing.assert_allclose(g0, np.broadcast_to(R.sigmoid(b), g0.shape), rtol=1e-15)
    c = 0.5
    g = R.memory_gate(x, {"gate_w": c * np.eye(C), "gate_b": np.zeros(C)})
    pre = np.log(g / (1 - g)) / c
    np.testing.assert_allclose(np.sqrt(np.mean(pre * pre, axis=-1)), 1.0, atol=1e-6)
    no_norm = R.sigmoid(x @ (c * np.eye(C)).T)
    pre2 = np.log(no_norm / (1 - no_norm)) / c
    assert np.max(np.abs(np.sqrt(np.mean(pre2 * pre2, axis=-1)) - 1.0)) > 0.1


# ---------------------------------------------------------------------------
# Attention block: window 0 returns v, so the block is linear in rms_norm(x)
# ---------------------------------------------------------------------------

def test_swa_forward_value_third():
    """model.py:100-133 with window 0: every query attends to itself only, so
    the block is (rms_norm(x) W_v^T) W_out^T with W_v the last third of
    to_qkv; taking the first third (q/v swapped) fails."""
    cfg = _cfg(window_size=0)
    H, D, C = cfg["n_head"], cfg["head_dim"], 16
    p = {"to_qkv": rng.standard_normal((3 * H * D, C)), "to_out": rng.standard_normal((C, H * D))}
    x = rng.standard_normal((2, 9, C))
    want = (R.rms_norm(x) @ p["to_qkv"][2 * H * D:].T) @ p["to_out"].T
    np.testing.assert_allclose(R.swa_forward(x, p, cfg), want, rtol=1e-10, atol=1e-12)
    wrong = (R.rms_norm(x) @ p["to_qkv"][:H * D].T) @ p["to_out"].T
    assert np.max(np.abs(wrong - want)) > 1e-2


# ---------------------------------------------------------------------------
# Memory layer: retrieve gate, chunk-aligned continuation, persistence
# ---------------------------------------------------------------------------

def test_retrieve_gate_zero_weight_halves_output():
    """memory_layer.py:720-725: a zero retrieve weight gives sigmoid(0) = 1/2
    per head, applied before the output projection (linear), so the layer
    output is exactly half of the ungated one."""
    cfg = _cfg()
    C = 16
    p = _layer_params(cfg, C)
    x = rng.standard_normal((1, 12, C))
    p0 = dict(p, retrieve_w=np.zeros_like(p["retrieve_w"]))
    pn = dict(p, retrieve_w=None)
    y0, _ = R.memory_layer_forward(x, p0, cfg)
    yn, _ = R.memory_layer_forward(x, pn, cfg)
    np.testing.assert_allclose(y0, 0.5 * yn, rtol=1e-12)


def _split_equals_whole(fwd, first, second, whole):
    """Helper: run fwd on the first part, carry its states into the second."""
    out1, st = fwd(first, None)
    out2, st2 = fwd(second, st)
    out, stw = fwd(whole, None)
    return out1, out2, st2, out, stw


def test_memory_layer_chunk_aligned_continuation():
    """With conv_kernel 1 (no token mixing outside the memory), a layer run on
    a chunk-aligned prefix and then on the rest from the carried state equals
    one call over the whole sequence (y and final state); carrying nothing
    into the second call (the reference's persistence test,
    tests/test_memory_layer.py:161-172) changes the output."""
    cfg = _cfg()
    C = 16
    p = _layer_params(cfg, C, conv_k=1)
    x = rng.standard_normal((2, 24, C))
    y1, st1 = R.memory_layer_forward(x[:, :16], p, cfg)
    y2, st2 = R.memory_layer_forward(x[:, 16:], p, cfg, st1)
    y, st = R.memory_layer_forward(x, p, cfg)
    np.testing.assert_allclose(np.concatenate([y1, y2], 1), y, rtol=1e-10, atol=1e-12)
    for a, b in zip(st2, st):
        np.testing.assert_allclose(a, b, rtol=1e-10, atol=1e-12)
    y2_fresh, _ = R.memory_layer_forward(x[:, 16:], p, cfg)
    assert SC.rel_l2(y2_fresh, y[:, 16:]) > 1e-3


def _atlas(cfg, params):
    return lambda idx, st: R.atlas_forward(idx, params, cfg, st)


def test_atlas_forward_outer_structure():
    """model.py:305-374: with every block's output projections zero
    (memory c_proj and MLP c_proj) the residual stream stays the embedding,
    so the logits are rms_norm(wte[idx]) lm_head^T, softcapped when asked."""
    cfg = _cfg(logit_softcap=3.0)
    C = 16
    params = _model_params(cfg, C)
    for p in params["layers"]:
        p["c_proj"] = np.zeros_like(p["c_proj"])
        p["mlp_proj"] = np.zeros_like(p["mlp_proj"])
    idx = rng.integers(0, cfg["vocab_size"], (2, 10))
    logits, states = R.atlas_forward(idx, params, cfg)
    want = R.rms_norm(params["wte"][idx]) @ params["lm_head"].T
    np.testing.assert_allclose(logits, 3.0 * np.tanh(want / 3.0), rtol=1e-12)
    assert len(states) == 2


def test_atlas_forward_causal_and_padding():
    """The forward is causal: logits at positions < t0 do not depend on
    tokens >= t0 (T = 13 pads to 16 with chunk 8, the reference's
    test_sequence_padding shape), and the padded call returns zero momentum
    (memory_layer.py:650-660).  A non-causal convolution (padding on the
    right) fails the check."""
    cfg = _cfg()
    C = 16
    params = _model_params(cfg, C)
    idx = rng.integers(0, cfg["vocab_size"], (1, 13))
    idx2 = idx.copy()
    idx2[0, 9:] = (idx2[0, 9:] + 7) % cfg["vocab_size"]
    l1, st1 = R.atlas_forward(idx, params, cfg)
    l2, _ = R.atlas_forward(idx2, params, cfg)
    assert l1.shape == (1, 13, cfg["vocab_size"])
    np.testing.assert_array_equal(l1[:, :9], l2[:, :9])
    assert np.max(np.abs(l1[:, 9:] - l2[:, 9:])) > 1e-6
    for st in st1:
        assert np.abs(st[2]).max() == 0 and np.abs(st[3]).max() == 0
        assert np.linalg.norm(st[0]) > 0

    orig = R.short_conv

    def right_padded(x, weight, bias):
        x = R._f64(x)
        B, T, Cc = x.shape
        K = weight.shape[-1]
        xp = np.concatenate([x, np.zeros((B, K - 1, Cc))], axis=1)
        out = np.zeros_like(x)
        for j in range(K):
            out += xp[:, j:j + T, :] * R._f64(weight)[:, 0, j][None, None, :]
        return out + R._f64(bias)[None, None, :]

    try:
        R.short_conv = right_padded
        m1, _ = R.atlas_forward(idx, params, cfg)
        m2, _ = R.atlas_forward(idx2, params, cfg)
    finally:
        R.short_conv = orig
    assert np.max(np.abs(m1[:, :9] - m2[:, :9])) > 1e-6


def test_atlas_forward_state_continuation():
    """tests/test_model.py:84-97 made exact: with conv_kernel 1, the model run
    on a chunk-aligned prefix and then on the remaining tokens from the
    carried per-layer states equals one call (logits and states).  Passing
    the layers' states in the wrong order fails."""
    cfg = _cfg()
    C = 16
    params = _model_params(cfg, C, conv_k=1)
    idx = rng.integers(0, cfg["vocab_size"], (2, 17))
    l1, st1 = R.atlas_forward(idx[:, :8], params, cfg)
    l2, st2 = R.atlas_forward(idx[:, 8:], params, cfg, st1)
    l, st = R.atlas_forward(idx, params, cfg)
    np.testing.assert_allclose(np.concatenate([l1, l2], 1), l, rtol=1e-9, atol=1e-11)
    for a, b in zip(st2, st):
        for x, y in zip(a, b):
            np.testing.assert_allclose(x, y, rtol=1e-9, atol=1e-12)
    l2_swapped, _ = R.atlas_forward(idx[:, 8:], params, cfg, st1[::-1])
    assert SC.rel_l2(l2_swapped, l[:, 8:]) > 1e-4
    # a single token continuing from the carried states (test_model.py:84-97)
    _, st16 = R.atlas_forward(idx[:, :16], params, cfg)
    l3, _ = R.atlas_forward(idx[:, 16:], params, cfg, st16)
    np.testing.assert_allclose(l3, l[:, 16:], rtol=1e-9, atol=1e-11)


def test_atlas_forward_persistent_tokens():
    """model.py:316-320, 359-360: persistent memory tokens are prepended to
    every row and their positions dropped after the final norm.  With the
    persistent rows equal to the embedding rows of token ids z, the logits
    are those of the plain forward on [z, idx] without its first len(z)
    positions, and the carried states are the same.  Appending the tokens,
    or dropping the last positions instead of the first, fails."""
    cfg = _cfg()
    C = 16
    params = _model_params(cfg, C)
    idx = rng.integers(0, cfg["vocab_size"], (2, 11))
    z = np.array([3, 17, 5])
    pp = dict(params, persist_mem=params["wte"][z])
    got, st = R.atlas_forward(idx, pp, cfg)
    full, st_full = R.atlas_forward(np.concatenate([np.broadcast_to(z, (2, 3)), idx], 1), params, cfg)
    assert got.shape == (2, 11, cfg["vocab_size"])
    np.testing.assert_allclose(got, full[:, 3:], rtol=1e-12, atol=1e-12)
    for a, b in zip(st, st_full):
        for x, y in zip(a, b):
            np.testing.assert_allclose(x, y, rtol=1e-12, atol=1e-14)
    appended, _ = R.atlas_forward(np.concatenate([idx, np.broadcast_to(z, (2, 3))], 1), params, cfg)
    assert SC.rel_l2(got, appended[:, :11]) > 1e-3
    assert SC.rel_l2(got, full[:, :11]) > 1e-3


# ---------------------------------------------------------------------------
# MAG forward
# ---------------------------------------------------------------------------

def test_mag_forward_outer_structure_and_causality():
    """mag_transformer.py:63-79,128-166: with attention, memory and MLP output
    projections zero the logits are rms_norm(wte[idx]) lm_head^T; with all
    weights live the forward is causal; and with the attention and MLP
    outputs zero a memory layer contributes exactly x + gate(mem) * mem, so
    a block that adds mem ungated fails."""
    cfg = _cfg(window_size=4)
    C = 16
    params = _model_params(cfg, C, mag=True, mem_layers=(1,))
    idx = rng.integers(0, cfg["vocab_size"], (2, 12))
    zero = copy.deepcopy(params)
    for p in zero["layers"]:
        p["to_out"] = np.zeros_like(p["to_out"])
        p["mlp_proj"] = np.zeros_like(p["mlp_proj"])
        if "c_proj" in p:
            p["c_proj"] = np.zeros_like(p["c_proj"])
    logits, states = R.mag_forward(idx, zero, cfg)
    np.testing.assert_allclose(logits, R.rms_norm(params["wte"][idx]) @ params["lm_head"].T, rtol=1e-12)
    assert states[0] is None and states[1] is not None

    idx2 = idx.copy()
    idx2[:, 7:] = (idx2[:, 7:] + 3) % cfg["vocab_size"]
    l1, _ = R.mag_forward(idx, params, cfg)
    l2, _ = R.mag_forward(idx2, params, cfg)
    np.testing.assert_array_equal(l1[:, :7], l2[:, :7])
    assert np.max(np.abs(l1[:, 7:] - l2[:, 7:])) > 1e-6

    # memory branch alone: x_out = x + gate(mem) * mem at layer 1
    only_mem = copy.deepcopy(params)
    for p in only_mem["layers"]:
        p["to_out"] = np.zeros_like(p["to_out"])
        p["mlp_proj"] = np.zeros_like(p["mlp_proj"])
    x = params["wte"][idx]
    mem, _ = R.memory_layer_forward(R.rms_norm(x), only_mem["layers"][1], cfg)
    x_gated = x + R.memory_gate(mem, only_mem["layers"][1]) * mem
    got, _ = R.mag_forward(idx, only_mem, cfg)
    np.testing.assert_allclose(got, R.rms_norm(x_gated) @ params["lm_head"].T, rtol=1e-10, atol=1e-12)
    x_ungated = x + mem
    assert np.max(np.abs(R.rms_norm(x_ungated) @ params["lm_head"].T - got)) > 1e-3
