"""CPU: pins of the sliding-window attention oracle (oracle/atlas_ref.py
rope_tables / apply_rope / swa_core, following atlas_jax/model.py:49-133)
against an independent per-query brute force, the known answers of the
rotation and the window, and planted mistakes that those checks must catch."""

import numpy as np
import pytest

from oracle import atlas_ref as R


def _qkv(B, T, H, D, seed):
    rng = np.random.default_rng(seed)
    return tuple(rng.standard_normal((B, T, H, D)) for _ in range(3))


@pytest.mark.parametrize("T,window", [(9, 0), (9, 1), (9, 3), (17, 5), (12, 11), (12, 40)])
def test_swa_core_matches_bruteforce(T, window):
    q, k, v = _qkv(2, T, 2, 8, seed=T + window)
    np.testing.assert_allclose(R.swa_core(q, k, v, window), R.swa_bruteforce(q, k, v, window),
                               rtol=1e-12, atol=1e-12)


def test_window_zero_returns_values_and_large_window_is_causal():
    q, k, v = _qkv(1, 15, 3, 16, seed=1)
    np.testing.assert_array_equal(R.swa_core(q, k, v, 0), v)
    full = R.swa_core(q, k, v, 14)
    np.testing.assert_allclose(R.swa_core(q, k, v, 10 ** 6), full, rtol=0, atol=0)
    # the first query only ever sees itself
    np.testing.assert_allclose(full[:, 0], v[:, 0], rtol=1e-13, atol=1e-13)


def test_rope_rotation_properties():
    T, D = 32, 16
    cos, sin = R.rope_tables(T, D)
    rng = np.random.default_rng(2)
    x = rng.standard_normal((1, T, 1, D))
    xr = R.apply_rope(x, cos, sin)
    # every (d, d + D/2) pair keeps its norm
    d2 = D // 2
    n0 = x[..., :d2] ** 2 + x[..., d2:] ** 2
    n1 = xr[..., :d2] ** 2 + xr[..., d2:] ** 2
    np.testing.assert_allclose(n1, n0, rtol=1e-12)
    # rotated dot products depend on the position difference only
    a, b = rng.standard_normal(D), rng.standard_normal(D)
    A = R.apply_rope(np.broadcast_to(a, (1, T, 1, D)), cos, sin)[0, :, 0]
    Bv = R.apply_rope(np.broadcast_to(b, (1, T, 1, D)), cos, sin)[0, :, 0]
    assert abs(A[5] @ Bv[2] - A[13] @ Bv[10]) < 1e-12
    assert abs(A[7] @ Bv[7] - a @ b) < 1e-12
    # direction of model.py:70-71 for e_0 at position 1: (cos 1, ..., sin 1 at d = D/2)
    e0 = np.zeros((1, 2, 1, D))
    e0[0, :, 0, 0] = 1.0
    r = R.apply_rope(e0, *R.rope_tables(2, D))[0, 1, 0]
    assert abs(r[0] - np.cos(1.0)) < 1e-15 and abs(r[d2] - np.sin(1.0)) < 1e-15


def test_planted_mistakes_are_caught(monkeypatch):
    q, k, v = _qkv(1, 10, 1, 8, seed=3)
    ref = R.swa_bruteforce(q, k, v, 3)
    # exclusive window (t - s < window) instead of model.py:125's inclusive one
    exclusive = R.swa_core(q, k, v, 2)
    assert np.abs(exclusive - ref).max() > 1e-3
    # rotation with the sign of the sine flipped in the second half
    orig = R.apply_rope

    def wrong_rope(x, cos, sin):
        x = np.asarray(x, np.float64)
        d2 = x.shape[-1] // 2
        x1, x2 = x[..., :d2], x[..., d2:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return np.concatenate([x1 * c - x2 * s, x2 * c - x1 * s], axis=-1)

    monkeypatch.setattr(R, "apply_rope", wrong_rope)
    assert np.abs(R.swa_core(q, k, v, 3) - ref).max() > 1e-3
    monkeypatch.setattr(R, "apply_rope", orig)
    np.testing.assert_allclose(R.swa_core(q, k, v, 3), ref, rtol=1e-12, atol=1e-12)
