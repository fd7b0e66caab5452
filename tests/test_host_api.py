"""CPU: the host package mirrors the reference configuration and API and has
no CPU fallback for the memory path."""

import dataclasses

import pytest
import torch

import __graft_entry__  # noqa: F401
import atlas_amd
from atlas_amd import AtlasConfig
from oracle import atlas_ref as R


def test_config_defaults_follow_reference():
    """atlas_jax/config.py:6-33 defaults."""
    c = AtlasConfig()
    assert (c.chunk_size, c.ns_steps, c.omega_window, c.poly_degree, c.memory_expand, c.max_lr) == \
        (64, 5, 16, 2, 2, 0.1)
    assert c.deep_memory and not c.fused_chunk and c.geglu_ff
    names = {f.name for f in dataclasses.fields(c)}
    for n in ("sequence_len", "vocab_size", "n_layer", "n_head", "n_embd", "dim_head", "conv_kernel",
              "pe_ste", "use_checkpoint", "dropout", "gate_bias_init", "logit_softcap",
              "num_persist_mem_tokens", "stop_grad_chunks", "window_size", "neural_memory_layers"):
        assert n in names
    assert AtlasConfig(n_embd=512, n_head=8).head_dim == 64
    assert AtlasConfig(n_embd=512, n_head=8, memory_expand=2).expand_dim == 128


def test_coefficients_identical_to_oracle():
    assert [tuple(r) for r in R.PE_COEFFS.tolist()] == [tuple(r) for r in atlas_amd.POLAR_EXPRESS_COEFFS]


def test_no_cpu_fallback():
    x = torch.zeros(1, 8, 2, 4)
    g = torch.zeros(1, 8, 2)
    st = atlas_amd.DeepMemoryState(torch.zeros(1, 2, 4, 8), torch.zeros(1, 2, 8, 4), torch.zeros(1, 2, 4, 8),
                                   torch.zeros(1, 2, 8, 4))
    with pytest.raises(ValueError, match="device"):
        atlas_amd.memory_scan(x, x, x, g, g, g, None, st, 8, 1, 5)
    with pytest.raises(ValueError, match="device"):
        atlas_amd.polar_express(torch.zeros(2, 4, 4))


def test_prologue_backward_arithmetic_matches_oracle():
    """The arithmetic LayerPrologue differentiates in its backward
    (layer_prologue_reference_ops, torch) equals the pinned NumPy prologue
    (memory_layer.py:606-633) on the stacked projection layout."""
    import numpy as np
    import torch
    from oracle import atlas_ref as R
    from atlas_amd.memory_layer import layer_prologue_reference_ops
    import test_oracle_model as TOM
    TOM.rng = np.random.default_rng(9)
    cfg = TOM._cfg()
    C, B, T, H, D = 16, 2, 11, cfg["n_head"], cfg["head_dim"]
    p = TOM._layer_params(cfg, C)
    x = TOM.rng.standard_normal((B, T, C))
    W = np.concatenate([p["c_q"], p["c_k"], p["c_v"], p["gate_alpha_w"], p["gate_eta_w"], p["gate_theta_w"],
                        p["gate_gamma_w"], p["retrieve_w"]], 0)
    proj = torch.tensor(x.reshape(B * T, C) @ W.T)
    cw = torch.tensor(np.stack([p[f"conv_{c}_w"].reshape(H * D, -1) for c in "qkv"]))
    cb = torch.tensor(np.stack([p[f"conv_{c}_b"] for c in "qkv"]))
    gb = torch.tensor(np.stack([p[f"gate_{g}_b"] for g in ("alpha", "eta", "theta", "gamma")]))
    pc = torch.tensor(p["poly_coeffs"])
    meta = (B, T, H, D, 4, 2, 4, True, cfg["max_lr"], torch.float64)
    q, k, v, gates, r = layer_prologue_reference_ops(proj, cw, cb, pc, gb, meta)
    ref = R.memory_layer_prologue(x, p, cfg)
    for got, want in zip((q, k, v, gates[0], gates[1], gates[2], gates[3]), ref):
        np.testing.assert_allclose(got.double().numpy(), want, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(r.double().numpy(), R.sigmoid(x @ p["retrieve_w"].T), rtol=1e-6)


def test_attention_backward_arithmetic_matches_oracle():
    """swa_attention_reference_block (what SWAttention's backward
    differentiates), evaluated block by block over the band, equals the
    pinned swa_core."""
    import numpy as np
    import torch
    from oracle import atlas_ref as R
    from atlas_amd.mag import swa_attention_reference_block
    rng = np.random.default_rng(3)
    B, T, H, D, window, blk = 1, 37, 2, 8, 9, 8
    q, k, v = (rng.standard_normal((B, T, H, D)) for _ in range(3))
    cos, sin = (torch.tensor(a) for a in R.rope_tables(T, D))
    out = []
    for t0 in range(0, T, blk):
        t1 = min(T, t0 + blk)
        s0 = max(0, t0 - window)
        out.append(swa_attention_reference_block(torch.tensor(q[:, t0:t1]), torch.tensor(k[:, s0:t1]),
                                                 torch.tensor(v[:, s0:t1]), window, cos.float(), sin.float(),
                                                 t0, s0).double())
    np.testing.assert_allclose(torch.cat(out, 1).numpy(), R.swa_core(q, k, v, window), rtol=1e-5, atol=1e-6)
