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
