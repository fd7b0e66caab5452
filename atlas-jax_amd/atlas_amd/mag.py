"""MAG (memory as gate) transformer forward on MI355X: sliding-window
attention with rotary embeddings (atlas_jax/model.py:49-133) and the MAG
blocks (atlas_jax/mag_transformer.py:22-166).

The attention core (rotation, banded causal softmax, value sum) runs in the
HIP library (atlas_swa_fwd); the memory branch is AtlasMemoryLayer on the HIP
scan; projections, norms, the gate and the MLP are torch (hipBLASLt GEMMs).
Names and structure follow the reference: RotaryEmbedding,
SlidingWindowAttention, MemoryGate, MAGBlock, MAGTransformer.  Dropout
(training-only) is not implemented.
"""

import math

import torch
from torch import nn

from . import _lib as L
from .config import AtlasConfig
from .memory_layer import AtlasMemoryLayer, rms_norm
from .model import MLP


class RotaryEmbedding(nn.Module):
    """model.py:49-62: inv_freq = 1 / 10000^(arange(0, dim, 2) / dim) (fp32);
    __call__(seq_len) -> (cos, sin), each (seq_len, dim // 2) fp32."""

    def __init__(self, dim, device="cuda"):
        super().__init__()
        self.dim = dim
        self.register_buffer(
            "inv_freq", 1.0 / (10000.0 ** (torch.arange(0, dim, 2, dtype=torch.float32, device=device) / dim)),
            persistent=False)

    def forward(self, seq_len):
        t = torch.arange(seq_len, dtype=torch.float32, device=self.inv_freq.device)
        freqs = torch.outer(t, self.inv_freq)
        return torch.cos(freqs), torch.sin(freqs)


def _swa_attention_hip(q, k, v, window, cos, sin, with_lse=False):
    """The attention core on atlas_swa_fwd; with_lse also returns the
    softmax log-normalisers (B, H, T) fp32 that atlas_swa_bwd takes."""
    lib = L.get_lib()
    if not (q.is_cuda and k.is_cuda and v.is_cuda):
        raise ValueError("atlas_amd operates on device (cuda/hip) tensors only")
    if q.shape != k.shape or q.shape != v.shape or q.dim() != 4:
        raise ValueError("q, k, v must share one (B, T, H, D) shape")
    if q.stride() != k.stride() or q.stride() != v.stride() or q.stride(-1) != 1:
        raise ValueError("q, k, v must share element strides with a contiguous last dim")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share one dtype")
    B, T, H, D = q.shape
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    if cos.shape != (T, D // 2) or sin.shape != (T, D // 2):
        raise ValueError("cos/sin tables must be (T, D/2)")
    out = torch.empty(B, T, H, D, dtype=q.dtype, device=q.device)
    sb, st, sh = q.stride(0), q.stride(1), q.stride(2)
    if with_lse:
        lse = torch.empty(B, H, T, dtype=torch.float32, device=q.device)
        L.check(lib.atlas_swa_fwd_lse(B, T, H, D, int(window), L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), sb, st,
                                      sh, L.dtype_code(q.dtype), L.ptr(cos), L.ptr(sin), L.ptr(lse),
                                      L.stream_ptr(q.device)))
        return out, lse
    L.check(lib.atlas_swa_fwd(B, T, H, D, int(window), L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), sb, st, sh,
                              L.dtype_code(q.dtype), L.ptr(cos), L.ptr(sin), L.stream_ptr(q.device)))
    return out


def swa_attention_vjp(q, k, v, window, cos, sin, out, lse, gout):
    """(dq, dk, dv) fp32 (B, T, H, D) of the attention core for the cotangent
    gout of its output, on atlas_swa_bwd (the standard attention backward
    with P recomputed from the forward's log-normalisers lse; model.py:109-129
    differentiated)."""
    lib = L.get_lib()
    B, T, H, D = q.shape
    cos = cos.float().contiguous()
    sin = sin.float().contiguous()
    gout = gout.to(out.dtype).contiguous()
    dq = torch.empty(B, T, H, D, dtype=torch.float32, device=q.device)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    ws_bytes = lib.atlas_swa_bwd_workspace_size(B, T, H)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    sb, st, sh = q.stride(0), q.stride(1), q.stride(2)
    L.check(lib.atlas_swa_bwd(B, T, H, D, int(window), L.ptr(q), L.ptr(k), L.ptr(v), L.ptr(out), L.ptr(gout),
                              L.ptr(lse), sb, st, sh, L.dtype_code(q.dtype), L.ptr(cos), L.ptr(sin), L.ptr(dq),
                              L.ptr(dk), L.ptr(dv), L.ptr(ws), ws_bytes, L.stream_ptr(q.device)))
    return dq, dk, dv


def _rope(x, cos, sin):
    """model.py:64-73 on (B, t, H, D) with (t, D/2) tables."""
    d2 = x.shape[-1] // 2
    x1, x2 = x[..., :d2], x[..., d2:]
    c, s_ = cos[None, :, None, :], sin[None, :, None, :]
    return torch.cat([x1 * c - x2 * s_, x2 * c + x1 * s_], dim=-1)


def swa_attention_reference_block(qb, kb, vb, window, cos, sin, t0, s0):
    """Queries t0 .. t0 + len(qb) - 1 of the banded attention (model.py:109-129)
    in fp32 torch operations, from the keys s0 .. s0 + len(kb) - 1 (the
    band they can see, s0 = max(0, t0 - window)): rotary rotation at absolute
    positions, scores / sqrt(D), causal band t - s <= window, softmax, value
    sum.  qb (B, tq, H, D), kb/vb (B, tk, H, D); cos/sin (T, D/2)."""
    tq, tk, D = qb.shape[1], kb.shape[1], qb.shape[-1]
    qr = _rope(qb.float(), cos[t0:t0 + tq], sin[t0:t0 + tq])
    kr = _rope(kb.float(), cos[s0:s0 + tk], sin[s0:s0 + tk])
    sc = torch.einsum("bthd,bshd->bhts", qr, kr) / math.sqrt(D)
    t = torch.arange(t0, t0 + tq, device=qb.device)[:, None]
    s_ = torch.arange(s0, s0 + tk, device=qb.device)[None, :]
    mask = (s_ <= t) & (t - s_ <= window)
    p = torch.softmax(sc.masked_fill(~mask, float("-inf")), dim=-1)
    return torch.einsum("bhts,bshd->bthd", p, vb.float())


class SWAttention(torch.autograd.Function):
    """Sliding-window attention: forward on the HIP kernel (atlas_swa_fwd_lse,
    keeping the softmax log-normalisers), backward on atlas_swa_bwd.
    backward_reference() is the earlier torch backward (recomputing
    swa_attention_reference_block for query blocks of 512 and
    differentiating it), kept as a cross-check."""

    BLOCK = 512

    @staticmethod
    def forward(ctx, q, k, v, window, cos, sin):
        ctx.window = int(window)
        out, lse = _swa_attention_hip(q, k, v, window, cos, sin, with_lse=True)
        ctx.save_for_backward(q, k, v, cos, sin, out, lse)
        return out

    @staticmethod
    def backward(ctx, gout):
        q, k, v, cos, sin, out, lse = ctx.saved_tensors
        dq, dk, dv = swa_attention_vjp(q, k, v, ctx.window, cos, sin, out, lse, gout)
        return dq.to(q.dtype), dk.to(k.dtype), dv.to(v.dtype), None, None, None

    @staticmethod
    def backward_reference(q, k, v, window, cos, sin, gout):
        """(dq, dk, dv) fp32 by differentiating the torch restatement blockwise."""
        T = q.shape[1]
        cosf, sinf = cos.float(), sin.float()
        dq = torch.zeros(q.shape, dtype=torch.float32, device=q.device)
        dk = torch.zeros_like(dq)
        dv = torch.zeros_like(dq)
        for t0 in range(0, T, SWAttention.BLOCK):
            t1 = min(T, t0 + SWAttention.BLOCK)
            s0 = max(0, t0 - window)
            qb = q[:, t0:t1].detach().float().requires_grad_(True)
            kb = k[:, s0:t1].detach().float().requires_grad_(True)
            vb = v[:, s0:t1].detach().float().requires_grad_(True)
            with torch.enable_grad():
                out = swa_attention_reference_block(qb, kb, vb, window, cosf, sinf, t0, s0)
                gq, gk, gv = torch.autograd.grad(out, (qb, kb, vb), gout[:, t0:t1].float())
            dq[:, t0:t1] += gq
            dk[:, s0:t1] += gk
            dv[:, s0:t1] += gv
        return dq, dk, dv


def swa_attention(q, k, v, window, cos, sin):
    """Attention core of model.py:109-129 on the HIP kernel.  q, k, v:
    (B, T, H, D) bf16/fp16 views with identical strides (the last dim
    contiguous); cos, sin: (T, D/2) fp32 -> out (B, T, H, D) contiguous.
    Differentiable with respect to q, k, v (SWAttention)."""
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        return SWAttention.apply(q, k, v, window, cos, sin)
    return _swa_attention_hip(q, k, v, window, cos, sin)


def _uniform_(w, generator):
    b = 1.0 / math.sqrt(w.shape[1])
    w.copy_(torch.empty_like(w).uniform_(-b, b, generator=generator))


class SlidingWindowAttention(nn.Module):
    """model.py:76-133: x -> rms_norm -> qkv (no bias) -> RoPE -> banded causal
    softmax attention (t - s <= window_size) -> to_out (no bias)."""

    def __init__(self, n_embd, n_head, dim_head, window_size, generator=None, device="cuda",
                 dtype=torch.bfloat16):
        super().__init__()
        inner = n_head * dim_head
        self.n_head, self.dim_head, self.window_size, self.n_embd = n_head, dim_head, window_size, n_embd
        self.to_qkv = nn.Linear(n_embd, 3 * inner, bias=False, device=device, dtype=dtype)
        self.to_out = nn.Linear(inner, n_embd, bias=False, device=device, dtype=dtype)
        self.rope = RotaryEmbedding(dim_head, device=device)
        with torch.no_grad():
            _uniform_(self.to_qkv.weight, generator)
            _uniform_(self.to_out.weight, generator)

    def forward(self, x):
        B, T, C = x.shape
        H, D = self.n_head, self.dim_head
        qkv = (rms_norm(x) @ self.to_qkv.weight.T).view(B, T, 3, H, D)
        cos, sin = self.rope(T)
        out = swa_attention(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], self.window_size, cos, sin)
        return out.view(B, T, H * D) @ self.to_out.weight.T


class MemoryGate(nn.Module):
    """mag_transformer.py:22-32: sigmoid(rms_norm(x) W^T + b), element-wise."""

    def __init__(self, dim, generator=None, device="cuda", dtype=torch.bfloat16):
        super().__init__()
        self.linear = nn.Linear(dim, dim, bias=True, device=device, dtype=dtype)
        with torch.no_grad():
            _uniform_(self.linear.weight, generator)
            b = 1.0 / math.sqrt(dim)
            self.linear.bias.copy_(torch.empty_like(self.linear.bias).uniform_(-b, b, generator=generator))

    def forward(self, x):
        return torch.sigmoid(rms_norm(x) @ self.linear.weight.T + self.linear.bias)


class MAGBlock(nn.Module):
    """mag_transformer.py:35-79: x + attn(x) + gate(mem) * mem with
    mem = memory(rms_norm(x)), then x + mlp(rms_norm(x))."""

    def __init__(self, config: AtlasConfig, has_memory: bool, generator=None, device="cuda",
                 dtype=torch.bfloat16):
        super().__init__()
        dim_head = config.head_dim
        self.attn = SlidingWindowAttention(config.n_embd, config.n_head, dim_head, config.window_size,
                                           generator=generator, device=device, dtype=dtype)
        if has_memory:
            self.memory = AtlasMemoryLayer(config, generator=generator, device=device, dtype=dtype)
            self.gate = MemoryGate(config.n_embd, generator=generator, device=device, dtype=dtype)
        else:
            self.memory = None
            self.gate = None
        self.mlp = MLP(config, generator=generator, device=device, dtype=dtype)

    def forward(self, x, memory_state=None):
        attn_out = self.attn(x)
        new_state = None
        if self.memory is not None:
            mem_out, new_state = self.memory(rms_norm(x), memory_state)
            x = x + attn_out + self.gate(mem_out) * mem_out
        else:
            x = x + attn_out
        x = x + self.mlp(rms_norm(x))
        return x, new_state


class MAGTransformer(nn.Module):
    """mag_transformer.py:82-166: embedding, MAG blocks (memory on the layers
    of config.neural_memory_layers, all by default), final norm, LM head
    (N(0, 0.02)); forward(idx, memory_states=None) -> (fp32 logits, states)."""

    def __init__(self, config: AtlasConfig, generator=None, device="cuda", dtype=torch.bfloat16):
        super().__init__()
        self.config = config
        mem_layers = (set(config.neural_memory_layers) if config.neural_memory_layers is not None
                      else set(range(config.n_layer)))
        self.memory_layer_mask = tuple(i in mem_layers for i in range(config.n_layer))
        self.wte = nn.Embedding(config.vocab_size, config.n_embd, device=device, dtype=dtype)
        self.blocks = nn.ModuleList([MAGBlock(config, self.memory_layer_mask[i], generator=generator,
                                              device=device, dtype=dtype) for i in range(config.n_layer)])
        self.lm_head = nn.Linear(config.n_embd, config.vocab_size, bias=False, device=device, dtype=dtype)
        with torch.no_grad():
            self.wte.weight.normal_(0.0, 1.0, generator=generator)
            self.lm_head.weight.normal_(0.0, 0.02, generator=generator)

    def forward(self, idx, memory_states=None):
        x = self.wte(idx)
        if memory_states is None:
            memory_states = [None] * self.config.n_layer
        new_states = []
        for blk, st in zip(self.blocks, memory_states):
            x, st = blk(x, st)
            new_states.append(st)
        x = rms_norm(x)
        return (x @ self.lm_head.weight.T).float(), new_states
