"""Atlas language model forward (atlas_jax/model.py:142-374) on the HIP scan.

Only the memory layers run the hand-written kernels; embedding, RMS norms,
the GEGLU MLP and the LM head are plain torch (hipBLASLt GEMMs).  Names and
structure follow the reference: MLP, Block, Atlas (wte, blocks, lm_head).
Dropout (training-only) is not implemented.
"""

import math

import torch
from torch import nn
import torch.nn.functional as F

from .config import AtlasConfig
from .memory_layer import AtlasMemoryLayer, DeepMemoryState, rms_norm


class MLP(nn.Module):
    """model.py:142-167: GEGLU (silu(gate) * v) with inner width int(4C*2/3),
    or plain GELU with 4C."""

    def __init__(self, config: AtlasConfig, generator=None, device="cuda", dtype=torch.float32):
        super().__init__()
        C = config.n_embd
        self.geglu = config.geglu_ff
        inner = int(C * 4 * 2 / 3) if self.geglu else 4 * C
        self.c_fc = nn.Linear(C, inner * 2 if self.geglu else inner, bias=False, device=device, dtype=dtype)
        self.c_proj = nn.Linear(inner, C, bias=False, device=device, dtype=dtype)
        with torch.no_grad():
            for lin in (self.c_fc, self.c_proj):
                b = 1.0 / math.sqrt(lin.in_features)
                lin.weight.copy_(torch.empty_like(lin.weight).uniform_(-b, b, generator=generator))

    def forward(self, x):
        h = x @ self.c_fc.weight.T
        if self.geglu:
            v, gate = h.chunk(2, dim=-1)
            h = F.silu(gate) * v
        else:
            h = F.gelu(h)
        return h @ self.c_proj.weight.T


class Block(nn.Module):
    """model.py:174-196: x += memory(rms_norm(x)); x += mlp(rms_norm(x))."""

    def __init__(self, config: AtlasConfig, generator=None, device="cuda", dtype=torch.float32):
        super().__init__()
        self.memory = AtlasMemoryLayer(config, generator=generator, device=device, dtype=dtype)
        self.mlp = MLP(config, generator=generator, device=device, dtype=dtype)

    def forward(self, x, memory_state=None):
        mem_out, new_state = self.memory(rms_norm(x), memory_state)
        x = x + mem_out
        x = x + self.mlp(rms_norm(x))
        return x, new_state


def initial_memory_states(config: AtlasConfig, batch_size, device="cuda"):
    """model.py:251-264: W1 = 0, W2 = [I; 0], S = 0 for every layer (fp32)."""
    H, D, E = config.n_head, config.head_dim, config.expand_dim
    states = []
    for _ in range(config.n_layer):
        W1 = torch.zeros(batch_size, H, D, E, device=device)
        W2 = torch.zeros(batch_size, H, E, D, device=device)
        m = min(D, E)
        W2[:, :, :m, :m] = torch.eye(m, device=device)
        states.append(DeepMemoryState(W1, W2, torch.zeros_like(W1), torch.zeros_like(W2)))
    return states


class Atlas(nn.Module):
    """model.py:271-374 without dropout.

    forward(idx (B, T) int64, memory_states=None) -> (logits (B, T, vocab)
    fp32, list of per-layer DeepMemoryState).  memory_states=None starts every
    layer from initial_memory_states (the reference's default).  With
    config.num_persist_mem_tokens = n > 0 the learnable persist_mem (n, C)
    (N(0, 0.02) at init, model.py:288-293) is prepended to every row before
    the blocks, so the memory layers scan T + n tokens, and its positions are
    dropped after the final norm (:316-320, :359-360)."""

    def __init__(self, config: AtlasConfig, generator=None, device="cuda", dtype=torch.float32,
                 pad_vocab_size_to=64, init_std=None):
        super().__init__()
        self.config = config
        self.padded_vocab_size = ((config.vocab_size + pad_vocab_size_to - 1) // pad_vocab_size_to) * pad_vocab_size_to
        self.wte = nn.Embedding(self.padded_vocab_size, config.n_embd, device=device, dtype=dtype)
        self.blocks = nn.ModuleList(
            [Block(config, generator=generator, device=device, dtype=dtype) for _ in range(config.n_layer)])
        self.lm_head = nn.Linear(config.n_embd, self.padded_vocab_size, bias=False, device=device, dtype=dtype)
        n_persist = config.num_persist_mem_tokens
        self.persist_mem = (nn.Parameter(torch.empty(n_persist, config.n_embd, device=device, dtype=dtype))
                            if n_persist > 0 else None)
        with torch.no_grad():
            if self.persist_mem is not None:
                self.persist_mem.normal_(0.0, 0.02, generator=generator)
            self.wte.weight.normal_(0.0, 1.0, generator=generator)
            self.lm_head.weight.normal_(0.0, 0.02, generator=generator)
            self._init_blocks(generator)
            if init_std is not None:
                # synthetic benchmarking: every weight matrix ~ N(0, init_std),
                # gate biases 0 (the bench config's "random init N(0, 0.02)")
                for name, prm in self.named_parameters():
                    if name.endswith(("W1_init", "W2_init", "poly_coeffs", "ln_gamma", "persist_mem")):
                        continue
                    if prm.dim() >= 2:
                        prm.normal_(0.0, init_std, generator=generator)
                    elif "gate" in name:
                        prm.zero_()

    def _init_blocks(self, generator):
        """model.py:199-248: c_proj ~ N(0, 0.02/sqrt(2n)), q/k/v uniform
        +-1/sqrt(C), gate weights 0 and biases gate_bias_init."""
        n = self.config.n_layer
        proj_std = 0.02 / math.sqrt(2 * n)
        for blk in self.blocks:
            mem = blk.memory
            mem.c_proj.weight.normal_(0.0, proj_std, generator=generator)
            blk.mlp.c_proj.weight.normal_(0.0, proj_std, generator=generator)
            C = mem.c_q.weight.shape[1]
            b = 1.0 / math.sqrt(C)
            for lin in (mem.c_q, mem.c_k, mem.c_v):
                lin.weight.uniform_(-b, b, generator=generator)
            for gate in (mem.gate_alpha, mem.gate_eta, mem.gate_theta, mem.gate_gamma):
                if gate is not None:
                    gate.weight.zero_()
                    gate.bias.fill_(self.config.gate_bias_init)

    def forward(self, idx, memory_states=None):
        B, T = idx.shape
        x = self.wte(idx)
        n_persist = 0 if self.persist_mem is None else self.persist_mem.shape[0]
        if n_persist:
            x = torch.cat([self.persist_mem.to(x.dtype).unsqueeze(0).expand(B, -1, -1), x], dim=1)
        if memory_states is None:
            memory_states = initial_memory_states(self.config, B, idx.device)
        new_states = []
        for blk, st in zip(self.blocks, memory_states):
            x, st = blk(x, st)
            new_states.append(st)
        x = rms_norm(x)[:, n_persist:]
        logits = (x @ self.lm_head.weight.T)[..., :self.config.vocab_size].float()
        sc = self.config.logit_softcap
        if sc > 0:
            logits = sc * torch.tanh(logits / sc)
        return logits, new_states
