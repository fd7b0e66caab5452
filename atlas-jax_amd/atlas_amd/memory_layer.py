"""Atlas memory layer on MI355X: host-side mirror of the reference API.

Names, argument meanings and return values follow rkstgr/atlas-jax
(atlas_jax/memory_layer.py, atlas_jax/kernels/*.py); the arithmetic of the
memory path runs in the HIP library (include/atlas_scan.h) through ctypes.
torch provides device memory, streams and the dense prologue/epilogue
(projections, causal convolutions, norms, gates).  There is no CPU or torch
fallback for the memory path: without the built library every entry point
raises.

Entry points and the reference interface each one stands in for:
  polar_express / fused_polar_express   memory_layer.py:43-71, kernels/triton_pe.py:26-69
  polar_express_ste                     memory_layer.py:74-76 (forward only)
  linear_scan                           memory_layer.py:256-296, kernels/triton_scan.py:85-111
  fused_chunk_scan                      kernels/fused_chunk.py:321-355 (forward)
  memory_scan                           the chunk loop memory_layer.py:662-716 with
                                        _process_chunk_deep :496-597 (new boundary)
  AtlasMemoryLayer(config)(x, state)    memory_layer.py:336-727
"""

import math
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib as L
from .config import AtlasConfig

# memory_layer.py:34-40 (the same table is compiled into the HIP library).
POLAR_EXPRESS_COEFFS = [
    (8.156554524902461, -22.48329292557795, 15.878769915207462),
    (4.042929935166739, -2.808917465908714, 0.5000178451051316),
    (3.8916678022926607, -2.772484153217685, 0.5060648178503393),
    (3.285753657755655, -2.3681294933425376, 0.46449024233003106),
    (2.3465413258596377, -1.7097828382687081, 0.42323551169305323),
]


class LinearMemoryState(NamedTuple):
    """memory_layer.py:100-103 (linear memory: not provided by the HIP path)."""
    M: torch.Tensor
    S: torch.Tensor


class DeepMemoryState(NamedTuple):
    """memory_layer.py:106-115.  W1, S_W1: (B, H, D, E); W2, S_W2: (B, H, E, D).
    The HIP path keeps the carry in fp32."""
    W1: torch.Tensor
    W2: torch.Tensor
    S_W1: torch.Tensor
    S_W2: torch.Tensor


def _precision(precision, dtype):
    if precision is None:
        return L.COMPUTE_F32 if dtype == torch.float32 else L.COMPUTE_F16
    if precision in ("f32", "fp32", L.COMPUTE_F32):
        return L.COMPUTE_F32
    if precision in ("f16", "fp16", L.COMPUTE_F16):
        return L.COMPUTE_F16
    raise ValueError(f"unknown scan precision {precision!r}")


def _require_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("atlas_amd operates on device (cuda/hip) tensors only")


# ---------------------------------------------------------------------------
# Polar-Express
# ---------------------------------------------------------------------------

def polar_express(X, steps=5, precision=None, norm_eps=True):
    """Batched Polar-Express of (..., d1, d2) matrices; returns X's dtype.
    norm_eps=False gives Muon's eps-free normalisation (optim.py:71)."""
    _require_cuda(X)
    if X.dim() < 2:
        raise ValueError("polar_express expects (..., d1, d2)")
    d1, d2 = X.shape[-2], X.shape[-1]
    Xc = X.contiguous()
    Y = torch.empty_like(Xc)
    n = Xc.numel() // (d1 * d2) if Xc.numel() else 0
    lib = L.get_lib()
    L.check(lib.atlas_pe_batched(n, d1, d2, steps, L.PE_NORM_EPS if norm_eps else L.PE_NORM_NO_EPS,
                                 L.ptr(Xc), L.ptr(Y), L.dtype_code(Xc.dtype),
                                 _precision(precision, Xc.dtype), L.stream_ptr(X.device)))
    return Y


fused_polar_express = polar_express
triton_polar_express = polar_express


def polar_express_ste(X, steps=5, precision=None):
    """Forward of memory_layer.py:74-76 (identical to polar_express)."""
    return polar_express(X, steps, precision)


fused_polar_express_ste = polar_express_ste
triton_polar_express_ste = polar_express_ste


# ---------------------------------------------------------------------------
# Scans
# ---------------------------------------------------------------------------

def linear_scan(h_init, gates, inputs):
    """h_t = g_t h_{t-1} + x_t along axis 1 (fp32).
    h_init (B, H, ...), gates (B, T, H), inputs (B, T, H, ...) ->
    (h_all (B, T, H, ...), h_final (B, H, ...)).  Differentiable (the HIP
    reverse-time scan, kernels/triton_scan.py:119-161) when an input
    requires grad."""
    _require_cuda(h_init, gates, inputs)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (h_init, gates, inputs)):
        from .autograd import LinearScan
        return LinearScan.apply(h_init, gates, inputs)
    B, T, H = gates.shape
    state_shape = inputs.shape[3:]
    N = int(math.prod(state_shape)) if state_shape else 1
    if tuple(h_init.shape) != (B, H, *state_shape):
        raise ValueError(f"h_init shape {tuple(h_init.shape)} != {(B, H, *state_shape)}")
    h0 = h_init.float().contiguous()
    g = gates.float().contiguous()
    x = inputs.float().contiguous()
    h_all = torch.empty((B, T, H, *state_shape), dtype=torch.float32, device=x.device)
    h_final = torch.empty_like(h0)
    L.check(L.get_lib().atlas_linear_scan(B, T, H, N, L.ptr(h0), L.ptr(g), L.ptr(x), L.ptr(h_all),
                                          L.ptr(h_final), L.stream_ptr(x.device)))
    return h_all, h_final


triton_linear_scan = linear_scan


def fused_chunk_scan(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste=False,
                     precision=None):
    """kernels/fused_chunk.py:321-355 (forward): one chunk from precomputed
    momentum inputs.  W1, SW1 (B,H,D,E); W2, SW2 (B,H,E,D); momW1 (B,cs,H,D,E);
    momW2 (B,cs,H,E,D); theta, alpha (B,cs,H); q (B,cs,H,D).
    Returns (y (B,cs,H,D) in q's dtype, DeepMemoryState in fp32).
    Differentiable when an input requires grad (the custom VJP of
    fused_chunk.py:357-379, computed in fp32; pe_ste selects the
    straight-through Polar-Express backward)."""
    _require_cuda(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q)
    if torch.is_grad_enabled() and any(t.requires_grad for t in (W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q)):
        from .autograd import FusedChunkScan
        y, *st = FusedChunkScan.apply(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste)
        return y, DeepMemoryState(*st)
    B, H, D, E = W1.shape
    cs = q.shape[1]
    st = [t.float().contiguous().clone() for t in (W1, W2, SW1, SW2)]
    io = q.dtype
    mw1 = momW1.to(io).contiguous()
    mw2 = momW2.to(io).contiguous()
    qc = q.contiguous()
    th = theta.contiguous()
    al = alpha.to(th.dtype).contiguous()
    y = torch.empty_like(qc)
    lib = L.get_lib()
    ws_bytes = lib.atlas_fused_chunk_workspace_size(B, H, D, E, cs)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    L.check(lib.atlas_fused_chunk_fwd(B, cs, H, D, E, ns_steps, L.dtype_code(io), L.dtype_code(th.dtype),
                                      _precision(precision, io), *(L.ptr(t) for t in st),
                                      L.ptr(mw1), L.ptr(mw2), L.ptr(th), L.ptr(al), L.ptr(qc), L.ptr(y),
                                      L.ptr(ws), ws_bytes, L.stream_ptr(q.device)))
    return y, DeepMemoryState(*st)


def memory_scan(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window, ns_steps,
                precision=None, n_slices=0, pe_ste=False, stop_grad_chunks=False, use_checkpoint=False,
                backward=None, train_precision=None):
    """The whole chunk loop of one memory layer in one library call.

    q, k, v: (B, T, H, D) feature-mapped queries/keys and values (one dtype);
    alpha, eta, theta, gamma: (B, T, H) post-sigmoid gates, eta already times
    max_lr; gamma may be None (no Omega window).  state: DeepMemoryState with
    W1 (B,H,D,E), W2 (B,H,E,D), S_W1, S_W2 (any float dtype; not modified).
    T need not be a multiple of chunk_size (reference padding semantics).
    Returns (y (B, T, H, D) in q's dtype, new DeepMemoryState in fp32).
    When an input requires grad (and grad mode is on) the call takes a
    differentiable fp32 training path; pe_ste selects the straight-through
    Polar-Express backward and stop_grad_chunks detaches the carry between
    chunks.  backward="hip" (the default where atlas_scan_bwd is compiled
    for the shape: D 32 with E <= 128, D 64 with E 64/128, and E 256 with
    train_precision "f16") runs the whole
    backward in the library (autograd.MemoryScanHIP; it always recomputes
    the chunks, so use_checkpoint changes nothing there; train_precision
    "f16" runs its forward in fp16 and keeps that forward's chunk-start
    states for the backward, None / "f32" computes in fp32); backward="torch"
    (the default otherwise) is autograd.memory_scan_autograd, the
    reference's fused-chunk loop differentiated through the inner gradient
    as torch ops, where use_checkpoint recomputes each chunk in the backward
    instead of keeping its intermediates (memory_layer.py:673)."""
    _require_cuda(q, k, v, alpha, eta, theta, gamma)
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad
                                       for t in (q, k, v, alpha, eta, theta, gamma, *state)):
        from . import autograd as AG
        D, E = q.shape[-1], state.W1.shape[-1]
        if backward is None:
            backward = "hip" if AG.hip_backward_supported(D, E, chunk_size, train_precision) else "torch"
        if backward == "hip":
            if not AG.hip_backward_supported(D, E, chunk_size, train_precision):
                raise L.AtlasError(2, f"atlas_scan_bwd is not compiled for D {D}, E {E}, chunk {chunk_size}")
            y, st = AG.memory_scan_hip_autograd(q, k, v, alpha, eta, theta, gamma, state, chunk_size,
                                                omega_window, ns_steps, pe_ste=pe_ste,
                                                stop_grad_chunks=stop_grad_chunks,
                                                precision=train_precision)
        elif backward == "torch":
            y, st = AG.memory_scan_autograd(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window,
                                            ns_steps, pe_ste=pe_ste, stop_grad_chunks=stop_grad_chunks,
                                            use_checkpoint=use_checkpoint)
        else:
            raise ValueError(f"backward must be 'hip' or 'torch', got {backward!r}")
        return y.to(q.dtype), st
    return _scan_forward(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window, ns_steps, precision,
                         n_slices)


def _scan_forward(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window, ns_steps, precision=None,
                  n_slices=0, trace=False):
    """memory_scan's forward on the library (no autograd).  With trace=True
    (atlas_scan_fwd_trace) also returns the chunk-start states, a
    (n_chunks, 4, B, H, D*E) fp32 tensor (W1, W2, S1, S2 per chunk)."""
    B, T, H, D = q.shape
    E = state.W1.shape[-1]
    io = q.dtype
    qc, kc, vc = (t.to(io).contiguous() for t in (q, k, v))
    gdt = alpha.dtype
    al, et, th = (t.to(gdt).contiguous() for t in (alpha, eta, theta))
    ga = None if gamma is None else gamma.to(gdt).contiguous()
    for name, t in (("alpha", al), ("eta", et), ("theta", th)):
        if tuple(t.shape) != (B, T, H):
            raise ValueError(f"{name} shape {tuple(t.shape)} != {(B, T, H)}")
    W1, W2, S1, S2 = (t.float().contiguous().clone() for t in state)
    if tuple(W1.shape) != (B, H, D, E) or tuple(W2.shape) != (B, H, E, D):
        raise ValueError("state shapes do not match (B, H, D, E) / (B, H, E, D)")
    y = torch.empty_like(qc)
    desc = L.ScanDesc(B=B, T=T, H=H, D=D, E=E, chunk_size=chunk_size, omega_window=omega_window,
                      ns_steps=ns_steps, io_dtype=L.dtype_code(io), gate_dtype=L.dtype_code(gdt),
                      compute=_precision(precision, io), n_slices=n_slices)
    lib = L.get_lib()
    ws_bytes = lib.atlas_scan_workspace_size(desc)
    if ws_bytes == 0:
        raise L.AtlasError(1, lib.atlas_last_error().decode(errors="replace"))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
    args = (L.ptr(qc), L.ptr(kc), L.ptr(vc), L.ptr(al), L.ptr(et), L.ptr(th), L.ptr(ga), L.ptr(W1), L.ptr(W2),
            L.ptr(S1), L.ptr(S2), L.ptr(y))
    if not trace:
        L.check(lib.atlas_scan_fwd(desc, *args, L.ptr(ws), ws_bytes, L.stream_ptr(q.device)))
        return y, DeepMemoryState(W1, W2, S1, S2)
    n_chunks = -(-T // chunk_size)
    tr = torch.empty(n_chunks, 4, B, H, D * E, dtype=torch.float32, device=q.device)
    L.check(lib.atlas_scan_fwd_trace(desc, *args, L.ptr(tr), L.ptr(ws), ws_bytes, L.stream_ptr(q.device)))
    return y, DeepMemoryState(W1, W2, S1, S2), tr


# ---------------------------------------------------------------------------
# Dense prologue helpers (torch) and the layer
# ---------------------------------------------------------------------------

def rms_norm(x):
    """memory_layer.py:211-216: computed in fp32, returned in x's dtype."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6)).to(x.dtype)


def init_memory_state(config: AtlasConfig, batch_size: int, device="cuda"):
    """memory_layer.py:118-143 for deep memory: one fp32 state per layer with
    W1 = 0, W2 = [I; 0], S = 0."""
    H, D, E = config.n_head, config.head_dim, config.expand_dim
    if not config.deep_memory:
        raise NotImplementedError("linear memory is not part of the HIP path")
    states = []
    for _ in range(config.n_layer):
        W1 = torch.zeros(batch_size, H, D, E, device=device)
        W2 = torch.zeros(batch_size, H, E, D, device=device)
        m = min(D, E)
        W2[:, :, :m, :m] = torch.eye(m, device=device)
        states.append(DeepMemoryState(W1, W2, torch.zeros_like(W1), torch.zeros_like(W2)))
    return states


class ShortConv(nn.Module):
    """Causal depthwise conv over time (memory_layer.py:303-329): weight
    (C, 1, K), bias (C,); out[t] = bias + sum_j w[j] x[t-(K-1)+j]."""

    def __init__(self, dim, kernel_size=4, generator=None, device=None, dtype=None):
        super().__init__()
        self.kernel_size = kernel_size
        self.weight = nn.Parameter(torch.randn(dim, 1, kernel_size, generator=generator, device=device,
                                               dtype=dtype) * 0.02)
        self.bias = nn.Parameter(torch.zeros(dim, device=device, dtype=dtype))

    def forward(self, x):
        B, T, C = x.shape
        xt = F.pad(x.transpose(1, 2), (self.kernel_size - 1, 0))
        out = F.conv1d(xt, self.weight.to(x.dtype), self.bias.to(x.dtype), groups=C)
        return out.transpose(1, 2)


def _linear(in_f, out_f, bias, generator, device, dtype):
    lin = nn.Linear(in_f, out_f, bias=bias, device=device, dtype=dtype)
    bound = 1.0 / math.sqrt(in_f)
    with torch.no_grad():
        lin.weight.copy_(torch.empty_like(lin.weight).uniform_(-bound, bound, generator=generator))
        if bias:
            lin.bias.copy_(torch.empty_like(lin.bias).uniform_(-bound, bound, generator=generator))
    return lin


def _layer_prologue_hip(proj, cw, cb, pc, gb, meta):
    """atlas_layer_prologue on the stacked projection output proj (B*T, ld)."""
    B, T, H, D, K, poly_degree, n_gates, has_r, max_lr, dtype = meta
    proj = proj.contiguous()
    cw, cb, gb = (t.detach().float().contiguous() for t in (cw, cb, gb))
    pc = pc.detach().float().contiguous() if pc is not None else None
    q = torch.empty(B, T, H, D, dtype=dtype, device=proj.device)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    gates = torch.empty(n_gates, B, T, H, dtype=torch.float32, device=proj.device)
    r = torch.empty(B, T, H, dtype=torch.float32, device=proj.device) if has_r else None
    L.check(L.get_lib().atlas_layer_prologue(B, T, H, D, K, poly_degree, n_gates, int(has_r), L.ptr(proj),
                                             proj.shape[1], L.dtype_code(proj.dtype), L.ptr(cw), L.ptr(cb),
                                             L.ptr(pc), L.ptr(gb), max_lr, L.ptr(q), L.ptr(k), L.ptr(v),
                                             L.dtype_code(dtype), L.ptr(gates), L.ptr(r),
                                             L.stream_ptr(proj.device)))
    return q, k, v, gates, r


def _layer_prologue_bwd_supported(meta):
    B, T, H, D, K, poly_degree, n_gates, has_r, max_lr, dtype = meta
    threads = -(-(H * D // 4) // 64) * 64
    return D in (16, 32, 64) and 1 <= K <= 4 and H * D <= 1024 and n_gates * H <= threads


def _layer_prologue_bwd_hip(proj, cw, cb, pc, gb, meta, gq, gk, gv, ggates, gr):
    """atlas_layer_prologue_bwd: (d proj, d conv_w, d conv_b, d poly, d gate_b)
    for the cotangents of (q, k, v, gates, retrieve) (None = zero)."""
    B, T, H, D, K, poly_degree, n_gates, has_r, max_lr, dtype = meta
    dev = proj.device
    proj = proj.contiguous()
    cwf, cbf, gbf = (t.detach().float().contiguous() for t in (cw, cb, gb))
    pcf = pc.detach().float().contiguous() if pc is not None else None
    gdt = gq.dtype if gq is not None else (gk.dtype if gk is not None else (gv.dtype if gv is not None else dtype))

    def ct(g, shape, dt):
        return (torch.zeros(shape, dtype=dt, device=dev) if g is None else g.to(dt)).contiguous()

    gq, gk, gv = (ct(g, (B, T, H, D), gdt) for g in (gq, gk, gv))
    ggates = ct(ggates, (n_gates, B, T, H), torch.float32)
    gr = ct(gr, (B, T, H), torch.float32) if has_r else None
    ld = proj.shape[1]
    dproj = torch.zeros(proj.shape, dtype=torch.float32, device=dev)
    dcw = torch.empty_like(cwf)
    dcb = torch.empty_like(cbf)
    dgb = torch.empty_like(gbf)
    dpc = torch.empty_like(pcf) if pcf is not None else None
    lib = L.get_lib()
    ws_bytes = lib.atlas_layer_prologue_bwd_workspace_size(B, T, H, D, K, poly_degree, n_gates)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    L.check(lib.atlas_layer_prologue_bwd(B, T, H, D, K, poly_degree, n_gates, int(has_r), L.ptr(proj), ld,
                                         L.dtype_code(proj.dtype), L.ptr(cwf), L.ptr(cbf), L.ptr(pcf), L.ptr(gbf),
                                         max_lr, L.ptr(gq), L.ptr(gk), L.ptr(gv), L.dtype_code(gdt), L.ptr(ggates),
                                         L.ptr(gr), L.ptr(dproj), ld, L.ptr(dcw), L.ptr(dcb), L.ptr(dpc),
                                         L.ptr(dgb), L.ptr(ws), ws_bytes, L.stream_ptr(dev)))
    return dproj, dcw, dcb, dpc, dgb


def layer_prologue_reference_ops(proj, cw, cb, pc, gb, meta):
    """The same prologue as torch operations (fp32), the arithmetic the
    backward differentiates: memory_layer.py:606-633 -- causal depthwise
    convs (:303-329, kernel K, left-padded), q = poly(rms_norm(q)), k =
    rms_norm(poly(k)) (:612-616; both rms_norm for degree 0), sigmoid gates
    with eta times max_lr (:621-633) and the retrieve gate (:720-722)."""
    B, T, H, D, K, poly_degree, n_gates, has_r, max_lr, dtype = meta
    HD = H * D
    x = proj.float().reshape(B, T, -1)
    outs = []
    for i in range(3):
        xi = x[..., i * HD:(i + 1) * HD].transpose(1, 2)                     # (B, HD, T)
        xi = F.pad(xi, (K - 1, 0))
        yi = F.conv1d(xi, cw[i].float().reshape(HD, 1, K), cb[i].float(), groups=HD)
        outs.append(yi.transpose(1, 2).reshape(B, T, H, D))
    q, k, v = outs

    def rms(t):
        return t * torch.rsqrt((t * t).mean(-1, keepdim=True) + 1e-6)

    def poly(t):
        out, tp = pc[0] * t, t
        for c in pc[1:]:
            tp = tp * t
            out = out + c * tp
        return out

    if poly_degree > 0:
        q, k = poly(rms(q)), rms(poly(k))
    else:
        q, k = rms(q), rms(k)
    g = torch.sigmoid(x[..., 3 * HD:3 * HD + n_gates * H].reshape(B, T, n_gates, H) + gb.float()[None, None])
    g = g.permute(2, 0, 1, 3)
    scale = torch.ones(n_gates, 1, 1, 1, device=g.device)
    scale[1] = max_lr
    gates = g * scale
    r = torch.sigmoid(x[..., 3 * HD + n_gates * H:3 * HD + n_gates * H + H]) if has_r else None
    return q.to(dtype), k.to(dtype), v.to(dtype), gates, r


class LayerPrologue(torch.autograd.Function):
    """The HIP prologue kernel with a backward with respect to the stacked
    projection output, the conv weights and biases, the poly coefficients and
    the gate biases: atlas_layer_prologue_bwd for every reference
    configuration's shape (head dims 16/32/64, conv kernels <= 4); other
    shapes recompute layer_prologue_reference_ops (the same arithmetic in
    torch) and differentiate it."""

    @staticmethod
    def forward(ctx, proj, cw, cb, pc, gb, meta):
        ctx.meta = meta
        ctx.has_pc = pc is not None
        ctx.save_for_backward(proj, cw, cb, pc if pc is not None else torch.empty(0, device=proj.device), gb)
        q, k, v, gates, r = _layer_prologue_hip(proj, cw, cb, pc, gb, meta)
        if r is None:
            r = torch.empty(0, device=proj.device)
        return q, k, v, gates, r

    @staticmethod
    def backward(ctx, gq, gk, gv, ggates, gr):
        proj, cw, cb, pc, gb = ctx.saved_tensors
        pc = pc if ctx.has_pc else None
        if _layer_prologue_bwd_supported(ctx.meta):
            dproj, dcw, dcb, dpc, dgb = _layer_prologue_bwd_hip(proj, cw, cb, pc, gb, ctx.meta, gq, gk, gv, ggates,
                                                                gr if ctx.meta[7] else None)
            return (dproj.to(proj.dtype), dcw.to(cw.dtype), dcb.to(cb.dtype),
                    None if pc is None else dpc.to(pc.dtype), dgb.to(gb.dtype), None)
        ins = [t.detach().requires_grad_(True) if t is not None else None for t in (proj, cw, cb, pc, gb)]
        with torch.enable_grad():
            outs = layer_prologue_reference_ops(*ins, ctx.meta)
        pairs = [(o, g) for o, g in zip(outs, (gq, gk, gv, ggates, gr)) if o is not None and g is not None]
        leaves = [t for t in ins if t is not None]
        grads = torch.autograd.grad([o for o, _ in pairs], leaves, [g for _, g in pairs], allow_unused=True)
        it = iter(grads)
        res = []
        for t in ins:
            if t is None:
                res.append(None)
            else:
                g = next(it)
                res.append(None if g is None else g.to(t.dtype))
        return (*res, None)


class AtlasMemoryLayer(nn.Module):
    """Multi-head memory layer (memory_layer.py:336-727), deep memory only.

    forward(x (B,T,C), memory_state=None) -> (y (B,T,C), DeepMemoryState).
    Parameter names follow the reference (c_q, c_k, c_v, c_proj, conv_q/k/v,
    gate_alpha/eta/theta/gamma, poly_coeffs, ln_gamma, W1_init, W2_init,
    retrieve_gate).
    Initialisation follows the reference's distributions with torch's RNG
    (the JAX random streams themselves cannot be reproduced)."""

    def __init__(self, config: AtlasConfig, generator=None, device="cuda", dtype=torch.float32):
        super().__init__()
        if not config.deep_memory:
            raise NotImplementedError("linear memory is not part of the HIP path")
        H, D, E, C = config.n_head, config.head_dim, config.expand_dim, config.n_embd
        self.config = config
        self.n_head, self.head_dim, self.expand_dim = H, D, E
        self.chunk_size, self.ns_steps = config.chunk_size, config.ns_steps
        self.omega_window, self.poly_degree = config.omega_window, config.poly_degree
        self.max_lr = config.max_lr
        g = generator
        inner = H * D
        self.c_q = _linear(C, inner, False, g, device, dtype)
        self.c_k = _linear(C, inner, False, g, device, dtype)
        self.c_v = _linear(C, inner, False, g, device, dtype)
        self.c_proj = _linear(inner, C, False, g, device, dtype)
        self.conv_q = ShortConv(inner, config.conv_kernel, g, device, dtype)
        self.conv_k = ShortConv(inner, config.conv_kernel, g, device, dtype)
        self.conv_v = ShortConv(inner, config.conv_kernel, g, device, dtype)
        self.gate_alpha = _linear(C, H, True, g, device, dtype)
        self.gate_eta = _linear(C, H, True, g, device, dtype)
        self.gate_theta = _linear(C, H, True, g, device, dtype)
        self.gate_gamma = _linear(C, H, True, g, device, dtype) if self.omega_window > 1 else None
        self.poly_coeffs = (nn.Parameter(torch.ones(self.poly_degree, device=device, dtype=torch.float32))
                            if self.poly_degree > 0 else None)
        # memory_layer.py:368, :446: declared and zero-initialised by the
        # reference but read by none of its forward paths; kept so that
        # checkpoints carry the same leaves
        self.ln_gamma = nn.Parameter(torch.zeros(H, D, device=device, dtype=torch.float32))
        b1 = math.sqrt(6.0 / (D + E))
        self.W1_init = nn.Parameter(torch.empty(H, D, E, device=device).uniform_(-b1, b1, generator=g))
        self.W2_init = nn.Parameter(torch.empty(H, E, D, device=device).uniform_(-b1, b1, generator=g))
        self.retrieve_gate = _linear(C, H, False, g, device, dtype) if H > 1 else None

    def _prologue_params(self):
        """The prologue's parameters in the reference's order: projection rows
        [c_q; c_k; c_v; gate_alpha; gate_eta; gate_theta(; gate_gamma)
        (; retrieve_gate)], gate biases, conv weights and biases, poly
        coefficients."""
        ws = [self.c_q.weight, self.c_k.weight, self.c_v.weight, self.gate_alpha.weight, self.gate_eta.weight,
              self.gate_theta.weight]
        bs = [self.gate_alpha.bias, self.gate_eta.bias, self.gate_theta.bias]
        if self.gate_gamma is not None:
            ws.append(self.gate_gamma.weight)
            bs.append(self.gate_gamma.bias)
        if self.retrieve_gate is not None:
            ws.append(self.retrieve_gate.weight)
        conv = [self.conv_q.weight, self.conv_k.weight, self.conv_v.weight, self.conv_q.bias, self.conv_k.bias,
                self.conv_v.bias]
        return ws, bs, conv

    def _stack(self, ws, bs, conv):
        W = torch.cat(list(ws), 0)
        gb = torch.stack([b.float() for b in bs], 0)
        cw = torch.stack([c.float().reshape(c.shape[0], -1) for c in conv[:3]], 0)
        cb = torch.stack([c.float() for c in conv[3:]], 0)
        pc = self.poly_coeffs.float() if self.poly_coeffs is not None else None
        return W, gb, cw, cb, pc

    def _stacked_projection(self):
        """W_all = [c_q; c_k; c_v; gate_alpha; gate_eta; gate_theta(; gate_gamma)
        (; retrieve_gate)] and the gate biases (n_gates, H), conv weights and
        biases and poly coefficients.  With gradients on (and a parameter that
        requires them) these are the live parameters, so the projection GEMM
        and the prologue backward reach every weight; otherwise a detached
        copy cached until a parameter changes."""
        ws, bs, conv = self._prologue_params()
        params = ws + bs + conv + ([self.poly_coeffs] if self.poly_coeffs is not None else [])
        if torch.is_grad_enabled() and any(t.requires_grad for t in params):
            return self._stack(ws, bs, conv)
        key = tuple((t.data_ptr(), t._version) for t in params)
        if getattr(self, "_proj_cache", None) is None or self._proj_cache[0] != key:
            with torch.no_grad():
                W, gb, cw, cb, pc = self._stack(ws, bs, conv)
                W, gb, cw, cb = (t.contiguous() for t in (W, gb, cw, cb))
                pc = pc.contiguous() if pc is not None else None
            self._proj_cache = (key, W, gb, cw, cb, pc)
        return self._proj_cache[1:]

    def prologue(self, x):
        """memory_layer.py:606-633 (+ the retrieve gate of :720-722): one GEMM
        x @ W_all^T (hipBLASLt through torch), then the fused HIP prologue
        (convolutions, q/k norm + polynomial map, gates).  Returns q, k, v
        (B,T,H,D) in x's dtype, alpha, eta, theta, gamma (B,T,H) fp32 (gamma
        None without an Omega window) and the retrieve gate (B,T,H) or None.
        Differentiable: with gradients on, the HIP forward is wrapped in
        LayerPrologue, whose backward differentiates the same arithmetic."""
        _require_cuda(x)
        B, T, C = x.shape
        W, gb, cw, cb, pc = self._stacked_projection()
        proj = x.reshape(B * T, C) @ W.to(x.dtype).T
        n_gates = gb.shape[0]
        meta = (B, T, self.n_head, self.head_dim, self.conv_q.kernel_size,
                self.poly_degree if pc is not None else 0, n_gates, self.retrieve_gate is not None,
                float(self.max_lr), x.dtype)
        if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in (proj, gb, cw, cb, pc)):
            q, k, v, gates, r = LayerPrologue.apply(proj, cw, cb, pc, gb, meta)
        else:
            q, k, v, gates, r = _layer_prologue_hip(proj, cw, cb, pc, gb, meta)
        gamma = gates[3] if n_gates == 4 else None
        return q, k, v, gates[0], gates[1], gates[2], gamma, r

    def default_state(self, B, device):
        """memory_layer.py:635-643: learnable initial weights, zero momentum
        (W1_init / W2_init stay in the autograd graph)."""
        H, D, E = self.n_head, self.head_dim, self.expand_dim
        W1 = self.W1_init.float().unsqueeze(0).expand(B, H, D, E)
        W2 = self.W2_init.float().unsqueeze(0).expand(B, H, E, D)
        return DeepMemoryState(W1, W2, torch.zeros(B, H, D, E, device=device), torch.zeros(B, H, E, D, device=device))

    def forward(self, x, memory_state=None):
        B, T, C = x.shape
        q, k, v, alpha, eta, theta, gamma, r = self.prologue(x)
        if memory_state is None:
            memory_state = self.default_state(B, x.device)
        y, state = memory_scan(q, k, v, alpha, eta, theta, gamma, memory_state, self.chunk_size,
                               self.omega_window, self.ns_steps, self.config.scan_precision,
                               pe_ste=self.config.pe_ste, stop_grad_chunks=self.config.stop_grad_chunks,
                               use_checkpoint=self.config.use_checkpoint,
                               backward=self.config.scan_backward,
                               train_precision=self.config.scan_train_precision)
        if r is not None:
            y = y * r.unsqueeze(-1).to(y.dtype)
        y = y.reshape(B, T, -1) @ self.c_proj.weight.to(y.dtype).T
        return y, state
