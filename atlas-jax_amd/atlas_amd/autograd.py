"""Backward passes (training) of the scan operators.

  linear_scan_vjp / LinearScan     the custom VJP of triton_linear_scan
                                   (kernels/triton_scan.py:119-161) on the HIP
                                   reverse-time scan (atlas_linear_scan_bwd).
  polar_express_vjp                the VJP of polar_express
                                   (memory_layer.py:43-71) through every
                                   Newton-Schulz step (iterates recomputed in
                                   fp32, batched GEMMs).
  fused_chunk_scan_vjp /           the custom VJP of fused_chunk_scan
  FusedChunkScan                   (kernels/fused_chunk.py:357-376): the
                                   reference recomputes _regular_fwd (:279-314)
                                   and differentiates it; here the recompute
                                   runs on the HIP scans and batched
                                   Polar-Express, the scans' backward on the
                                   HIP reverse scan, and the read-out and
                                   Polar-Express backward as fp32 batched
                                   GEMMs.  pe_ste=True makes the
                                   Polar-Express backward the identity
                                   (memory_layer.py:74-76).

  MemoryScanHIP /                  the training path of the whole layer on
  memory_scan_hip_autograd         the HIP backward (atlas_scan_bwd): forward
                                   on the fp32 whole-layer scan, backward by
                                   the library's chunk-by-chunk reverse pass
                                   (recompute from stored chunk-start states,
                                   read-out, memory and momentum scan adjoints,
                                   Polar-Express VJP, Omega and inner-gradient
                                   adjoints).  The default training path for
                                   the shapes it is compiled for.

  memory_scan_autograd             the training path of the whole layer:
                                   the reference's fused-chunk loop
                                   (memory_layer.py:649-711 with
                                   _process_chunk_deep :496-541) with the
                                   inner gradient and Omega window as
                                   differentiable fp32 torch ops and the
                                   sequential part on FusedChunkScan.
"""

import math

import torch
import torch.utils.checkpoint

from . import _lib as L
from .memory_layer import POLAR_EXPRESS_COEFFS, _require_cuda, linear_scan, polar_express

_SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)


def linear_scan_vjp(h_init, gates, h_all, dh_all, dh_final):
    """(d_h_init, d_gates, d_inputs) of h_t = g_t h_{t-1} + x_t for upstream
    dh_all (B, T, H, ...) and dh_final (B, H, ...) (either may be None)."""
    _require_cuda(h_init, gates, h_all)
    B, T, H = gates.shape
    state_shape = h_all.shape[3:]
    N = int(math.prod(state_shape)) if state_shape else 1
    h0 = h_init.float().contiguous()
    g = gates.float().contiguous()
    ha = h_all.float().contiguous()
    da = None if dh_all is None else dh_all.float().contiguous()
    df = None if dh_final is None else dh_final.float().contiguous()
    d_h0 = torch.empty_like(h0)
    d_g = torch.empty_like(g)
    d_x = torch.empty_like(ha)
    lib = L.get_lib()
    ws_bytes = lib.atlas_linear_scan_bwd_workspace_size(B, T, H, N)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=ha.device)
    L.check(lib.atlas_linear_scan_bwd(B, T, H, N, L.ptr(h0), L.ptr(g), L.ptr(ha), L.ptr(da), L.ptr(df),
                                      L.ptr(d_h0), L.ptr(d_g), L.ptr(d_x), L.ptr(ws), ws_bytes,
                                      L.stream_ptr(ha.device)))
    return d_h0, d_g, d_x


class LinearScan(torch.autograd.Function):
    """Differentiable linear_scan (forward and backward on the HIP scans)."""

    @staticmethod
    def forward(ctx, h_init, gates, inputs):
        h_all, h_final = linear_scan(h_init, gates, inputs)
        ctx.save_for_backward(h_init, gates, h_all)
        return h_all, h_final

    @staticmethod
    def backward(ctx, dh_all, dh_final):
        h_init, gates, h_all = ctx.saved_tensors
        d_h0, d_g, d_x = linear_scan_vjp(h_init, gates, h_all, dh_all, dh_final)
        return d_h0.to(h_init.dtype), d_g.to(gates.dtype), d_x


def pe_vjp_supported(d1, d2, precision="f32"):
    """Matrix shapes atlas_pe_vjp_batched is compiled for (either
    precision)."""
    del precision
    D, E = min(d1, d2), max(d1, d2)
    return (D == 32 and E in (32, 64, 128)) or (D == 64 and E in (64, 128, 256))


def polar_express_vjp(X, G, steps=5, norm_eps=True, precision="f32"):
    """VJP of polar_express (memory_layer.py:43-71) at X for the cotangent G,
    both (..., d1, d2): the normalisation X / (sqrt(sum X^2 + eps) * 1.01 +
    1e-6) and `steps` odd-quintic iterations, differentiated exactly
    (wide/square: A = X X^T, X' = a X + (b A + c A^2) X; tall inputs through
    the transpose).  On the library (atlas_pe_vjp_batched, fp32 or fp16
    matrix-core operands) for the shapes it is compiled for; other shapes,
    and the normalisation without the 1e-12 term, as fp32 batched GEMMs."""
    if not 0 <= steps <= len(POLAR_EXPRESS_COEFFS):
        raise ValueError(f"steps must be in [0, {len(POLAR_EXPRESS_COEFFS)}]")
    d1, d2 = X.shape[-2], X.shape[-1]
    if norm_eps and pe_vjp_supported(d1, d2, precision):
        _require_cuda(X, G)
        Xc = X.float().contiguous()
        dX = G.float().contiguous().clone()
        n = Xc.numel() // (d1 * d2)
        lib = L.get_lib()
        ws_bytes = lib.atlas_pe_vjp_workspace_size(d1, d2, steps)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=Xc.device)
        compute = L.COMPUTE_F16 if precision in ("f16", "fp16") else L.COMPUTE_F32
        L.check(lib.atlas_pe_vjp_batched(n, d1, d2, steps, L.ptr(Xc), L.ptr(dX), compute, L.ptr(ws), ws_bytes,
                                         L.stream_ptr(Xc.device)))
        return dX
    S = X.float()
    Gf = G.float()
    tall = S.shape[-2] > S.shape[-1]
    if tall:
        S, Gf = S.mT, Gf.mT
    eps = 1e-12 if norm_eps else 0.0
    n = torch.sqrt((S * S).sum(dim=(-2, -1), keepdim=True) + eps)
    nrm = n * 1.01 + 1e-6
    iterates = [S / nrm]
    for a, b, c in POLAR_EXPRESS_COEFFS[:steps - 1] if steps > 0 else []:
        Y = iterates[-1]
        A = Y @ Y.mT
        iterates.append(a * Y + (b * A + c * (A @ A)) @ Y)
    Gb = Gf
    for k in range(steps - 1, -1, -1):
        a, b, c = POLAR_EXPRESS_COEFFS[k]
        Y = iterates[k]
        A = Y @ Y.mT
        Bm = b * A + c * (A @ A)
        Gh = Gb @ Y.mT
        Gs = Gh + Gh.mT
        Gb = a * Gb + Bm @ Gb + (b * Gs + c * (Gs @ A + A @ Gs)) @ Y
    dS = Gb / nrm - ((Gb * S).sum(dim=(-2, -1), keepdim=True) * 1.01 / (nrm * nrm * n)) * S
    return dS.mT if tall else dS


def _gelu_tanh(x):
    return 0.5 * x * (1.0 + torch.tanh(_SQRT_2_OVER_PI * (x + 0.044715 * x ** 3)))


def _gelu_tanh_grad(x):
    t = torch.tanh(_SQRT_2_OVER_PI * (x + 0.044715 * x ** 3))
    return 0.5 * (1.0 + t) + 0.5 * x * (1.0 - t * t) * _SQRT_2_OVER_PI * (1.0 + 3 * 0.044715 * x * x)


def fused_chunk_scan_vjp(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste, gy, gW1, gW2, gS1,
                         gS2):
    """Gradients of fused_chunk_scan's (y, W1_end, W2_end, S1_end, S2_end)
    with respect to (W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q), for the
    cotangents gy (B,cs,H,D) and gW1..gS2 (end states; None = zero).
    Follows the recompute-then-differentiate of kernels/fused_chunk.py:357-376
    with _regular_fwd (:279-314)."""
    f = torch.float32
    W1f, W2f, S1f, S2f = (t.to(f) for t in (W1, W2, SW1, SW2))
    th, al, qf = theta.to(f), alpha.to(f), q.to(f)
    # recompute the forward: momentum scans, Polar-Express, memory scans
    S1_all, _ = linear_scan(S1f, th, momW1.to(f))
    S2_all, _ = linear_scan(S2f, th, momW2.to(f))
    P1 = polar_express(S1_all, ns_steps, precision="f32")
    P2 = polar_express(S2_all, ns_steps, precision="f32")
    W1_all, _ = linear_scan(W1f, al, P1)
    W2_all, _ = linear_scan(W2f, al, P2)
    # read-out y = q + W1_t gelu_tanh(W2_t q)
    gyf = torch.zeros_like(qf) if gy is None else gy.to(f)
    h = torch.einsum("bthed,bthd->bthe", W2_all, qf)
    g = _gelu_tanh(h)
    gh = torch.einsum("bthde,bthd->bthe", W1_all, gyf) * _gelu_tanh_grad(h)
    gq = gyf + torch.einsum("bthed,bthe->bthd", W2_all, gh)
    dW1_y = gyf.unsqueeze(-1) * g.unsqueeze(-2)      # (B,cs,H,D,E)
    dW2_y = gh.unsqueeze(-1) * qf.unsqueeze(-2)      # (B,cs,H,E,D)
    # memory scans
    gW1_0, ga1, GW1 = linear_scan_vjp(W1f, al, W1_all, dW1_y, gW1)
    gW2_0, ga2, GW2 = linear_scan_vjp(W2f, al, W2_all, dW2_y, gW2)
    # Polar-Express (identity under the straight-through estimator)
    if pe_ste:
        gP1, gP2 = GW1, GW2
    else:
        gP1 = polar_express_vjp(S1_all, GW1, ns_steps)
        gP2 = polar_express_vjp(S2_all, GW2, ns_steps)
    # momentum scans
    gS1_0, gt1, gm1 = linear_scan_vjp(S1f, th, S1_all, gP1, gS1)
    gS2_0, gt2, gm2 = linear_scan_vjp(S2f, th, S2_all, gP2, gS2)
    return (gW1_0.to(W1.dtype), gW2_0.to(W2.dtype), gS1_0.to(SW1.dtype), gS2_0.to(SW2.dtype),
            gm1.to(momW1.dtype), gm2.to(momW2.dtype), (gt1 + gt2).to(theta.dtype), (ga1 + ga2).to(alpha.dtype),
            gq.to(q.dtype))


class FusedChunkScan(torch.autograd.Function):
    """fused_chunk_scan with the custom VJP of kernels/fused_chunk.py:321-379:
    forward on the HIP operator (fp32 arithmetic), backward by
    fused_chunk_scan_vjp."""

    @staticmethod
    def forward(ctx, W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste):
        from .memory_layer import fused_chunk_scan
        y, st = fused_chunk_scan(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q, ns_steps, pe_ste,
                                 precision="f32")
        ctx.save_for_backward(W1, W2, SW1, SW2, momW1, momW2, theta, alpha, q)
        ctx.ns_steps, ctx.pe_ste = ns_steps, pe_ste
        return (y, *st)

    @staticmethod
    def backward(ctx, gy, gW1, gW2, gS1, gS2):
        grads = fused_chunk_scan_vjp(*ctx.saved_tensors, ctx.ns_steps, ctx.pe_ste, gy, gW1, gW2, gS1, gS2)
        return (*grads, None, None)


def _gelu_erf_derivative(x):
    """memory_layer.py:225-230: Phi(x) + x phi(x), exact erf form."""
    return 0.5 * (1.0 + torch.erf(x * (1.0 / math.sqrt(2.0)))) + x * torch.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def _omega_aggregate(u, gamma, omega_window):
    """memory_layer.py:233-253: G_t = sum_{i=max(0,t-w+1)}^{t} gamma_i u_i
    within the chunk (axis 1), as a cumsum minus the cumsum shifted by w."""
    weighted = gamma.reshape(*gamma.shape, *(1,) * (u.dim() - 3)) * u
    cum = torch.cumsum(weighted, dim=1)
    cs = u.shape[1]
    if omega_window >= cs:
        return cum
    shifted = torch.cat([torch.zeros_like(cum[:, :omega_window]), cum[:, :-omega_window]], dim=1)
    return cum - shifted


def _chunk_momentum(W1, W2, k, v, eta, gamma, omega_window):
    """The token-parallel half of _process_chunk_deep (memory_layer.py:504-533)
    in fp32 torch ops: memory forward at the chunk-start weights, the inner
    gradient (scale 2/D; u_W2 mixes the erf GELU derivative into the tanh
    forward, as the reference does), the Omega window and mom = -eta G.
    k, v (B,cs,H,D); eta, gamma (B,cs,H); W1 (B,H,D,E), W2 (B,H,E,D)."""
    D = k.shape[-1]
    h = torch.einsum("bhed,bchd->bche", W2, k)
    act = _gelu_tanh(h)
    err = k + torch.einsum("bhde,bche->bchd", W1, act) - v
    scale = 2.0 / D
    u1 = scale * err.unsqueeze(-1) * act.unsqueeze(-2)                      # (B,cs,H,D,E)
    chain = torch.einsum("bhde,bchd->bche", W1, err) * _gelu_erf_derivative(h)
    u2 = scale * chain.unsqueeze(-1) * k.unsqueeze(-2)                      # (B,cs,H,E,D)
    if omega_window > 1 and gamma is not None:
        u1 = _omega_aggregate(u1, gamma, omega_window)
        u2 = _omega_aggregate(u2, gamma, omega_window)
    e = eta.unsqueeze(-1).unsqueeze(-1)
    return -(e * u1), -(e * u2)


def _chunk_step(W1, W2, S1, S2, q, k, v, alpha, eta, theta, gamma, omega_window, ns_steps, pe_ste):
    """One chunk of the training path: momentum inputs (token-parallel, torch)
    and the sequential part (FusedChunkScan) -> (y, W1, W2, S1, S2)."""
    m1, m2 = _chunk_momentum(W1, W2, k, v, eta, gamma, omega_window)
    return FusedChunkScan.apply(W1, W2, S1, S2, m1, m2, theta, alpha, q, ns_steps, pe_ste)


def memory_scan_autograd(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window, ns_steps,
                         pe_ste=False, stop_grad_chunks=False, use_checkpoint=False):
    """Differentiable whole-layer chunk loop (training path of memory_scan).

    Follows the reference's fused-chunk training path: the chunk loop of
    AtlasMemoryLayer.__call__ (memory_layer.py:649-711, padding T to a
    multiple of chunk_size with alpha=1, eta=theta=gamma=0, q=k=v=0), each
    chunk's _process_chunk_deep (:496-541) differentiated by autograd through
    the token-parallel inner gradient and Omega window, and the sequential
    part on fused_chunk_scan, whose custom VJP (fused_chunk.py:357-379) runs
    on the HIP scans.  stop_grad_chunks detaches the carry between chunks
    (:665).  use_checkpoint is the reference's per-chunk jax.checkpoint
    (:673): each chunk's intermediates (its (B,cs,H,D,E) momentum inputs
    and the operator's saved inputs) are dropped after the forward and
    recomputed in the backward, so only the per-chunk carries stay alive.
    All arithmetic fp32; returns (y (B,T,H,D) fp32, DeepMemoryState fp32)
    with the same values as memory_scan's fp32 forward."""
    from .memory_layer import DeepMemoryState
    _require_cuda(q, k, v, alpha, eta, theta)
    B, T, H, D = q.shape
    cs = chunk_size
    f = torch.float32
    q, k, v = (t.to(f) for t in (q, k, v))
    alpha, eta, theta = (t.to(f) for t in (alpha, eta, theta))
    gamma = None if gamma is None else gamma.to(f)
    if T % cs:
        pad = cs - T % cs

        def _pad(t, val):
            return torch.nn.functional.pad(t, (0, 0) * (t.dim() - 2) + (0, pad), value=val)
        q, k, v = _pad(q, 0.0), _pad(k, 0.0), _pad(v, 0.0)
        alpha, eta, theta = _pad(alpha, 1.0), _pad(eta, 0.0), _pad(theta, 0.0)
        gamma = None if gamma is None else _pad(gamma, 0.0)
    W1, W2, S1, S2 = (t.to(f) for t in state)
    ys = []
    for c in range(q.shape[1] // cs):
        sl = slice(c * cs, (c + 1) * cs)
        if stop_grad_chunks:
            W1, W2, S1, S2 = (t.detach() for t in (W1, W2, S1, S2))
        args = (W1, W2, S1, S2, q[:, sl], k[:, sl], v[:, sl], alpha[:, sl], eta[:, sl], theta[:, sl],
                None if gamma is None else gamma[:, sl], omega_window, ns_steps, pe_ste)
        if use_checkpoint:
            y_c, W1, W2, S1, S2 = torch.utils.checkpoint.checkpoint(_chunk_step, *args, use_reentrant=False)
        else:
            y_c, W1, W2, S1, S2 = _chunk_step(*args)
        ys.append(y_c)
    y = torch.cat(ys, dim=1)[:, :T]
    return y, DeepMemoryState(W1, W2, S1, S2)


# ---------------------------------------------------------------------------
# Whole-layer training path on the HIP backward (atlas_scan_bwd)
# ---------------------------------------------------------------------------

def hip_backward_supported(D, E, chunk_size, precision=None):
    """Shapes atlas_scan_bwd is compiled for (either Polar-Express
    precision)."""
    del precision
    return ((D == 32 and E in (32, 64, 128)) or (D == 64 and E in (64, 128, 256))) and 1 <= chunk_size <= 256


def _pad_time(t, pad, val):
    return torch.nn.functional.pad(t, (0, 0) * (t.dim() - 2) + (0, pad), value=val) if pad else t


class MemoryScanHIP(torch.autograd.Function):
    """memory_scan differentiated by the library: forward on the HIP scan
    in `precision` (fp16: atlas_scan_fwd_trace, keeping every chunk's start
    state for the backward), backward by atlas_scan_bwd (fp32).  Inputs are padded to a multiple of the chunk size with the
    reference's values (alpha 1, eta = theta = gamma = 0, q = k = v = 0;
    memory_layer.py:649-660) and the padded rows of the gradients dropped."""

    @staticmethod
    def forward(ctx, q, k, v, alpha, eta, theta, gamma, W1, W2, S1, S2, chunk_size, omega_window, ns_steps,
                pe_ste, stop_grad_chunks, precision):
        from .memory_layer import DeepMemoryState, _scan_forward
        B, T, H, D = q.shape
        pad = (-T) % chunk_size
        f = torch.float32
        xs = [_pad_time(t.to(f), pad, 0.0).contiguous() for t in (q, k, v)]
        gs = [_pad_time(alpha.to(f), pad, 1.0).contiguous()] + [_pad_time(t.to(f), pad, 0.0).contiguous()
                                                                 for t in (eta, theta)]
        ga = None if gamma is None else _pad_time(gamma.to(f), pad, 0.0).contiguous()
        st = [t.to(f).contiguous() for t in (W1, W2, S1, S2)]
        if precision is None:   # the training path computes in fp32 unless fp16 is asked for
            precision = "f32"
        # fp16 forward: keep its chunk-start states, so the backward skips its
        # own forward pass and linearises around this trajectory.  fp32
        # forward: the backward retraces in fp32 with the kernels it
        # recomputes the chunks with (measured closer to fp32 evaluation of
        # the reference: 1-2x its error, against 2.5-4.5x around the fp32
        # phase kernels' trajectory).
        keep = precision in ("f16", "fp16")
        with torch.no_grad():
            r = _scan_forward(*xs, *gs, ga, DeepMemoryState(*st), chunk_size, omega_window, ns_steps,
                              precision=precision, trace=keep)
        y, out = r[0], r[1]
        trace = r[2] if keep else torch.empty(0, device=q.device)
        ctx.keep_trace = keep
        ctx.save_for_backward(*xs, *gs, *([] if ga is None else [ga]), *st, trace)
        ctx.cfg = (T, pad, chunk_size, omega_window, ns_steps, pe_ste, stop_grad_chunks, gamma is not None)
        ctx.dtypes = [t.dtype for t in (q, k, v, alpha, eta, theta)] + \
            [None if gamma is None else gamma.dtype] + [t.dtype for t in (W1, W2, S1, S2)]
        return (y[:, :T], *out)

    @staticmethod
    def backward(ctx, dy, dW1, dW2, dS1, dS2):
        T, pad, cs, w, ns, pe_ste, stop, has_g = ctx.cfg
        saved = list(ctx.saved_tensors)
        q, k, v, al, et, th = saved[:6]
        ga = saved[6] if has_g else None
        W1, W2, S1, S2 = saved[-5:-1]
        trace = saved[-1] if ctx.keep_trace else None
        B, Tp, H, D = q.shape
        E = W1.shape[-1]
        f = torch.float32
        dyp = None if dy is None else _pad_time(dy.to(f), pad, 0.0).contiguous()
        cst = [None if t is None else t.to(f).contiguous() for t in (dW1, dW2, dS1, dS2)]
        dq, dk, dv = (torch.empty_like(q) for _ in range(3))
        dal, det, dth = (torch.empty_like(al) for _ in range(3))
        dga = torch.empty_like(al) if has_g else None
        dst = [torch.empty_like(t) for t in (W1, W2, S1, S2)]
        desc = L.ScanDesc(B=B, T=Tp, H=H, D=D, E=E, chunk_size=cs, omega_window=w, ns_steps=ns,
                          io_dtype=0, gate_dtype=0, compute=L.COMPUTE_F16 if ctx.keep_trace else L.COMPUTE_F32,
                          n_slices=0)
        lib = L.get_lib()
        ws_bytes = lib.atlas_scan_bwd_workspace_size(desc)
        if ws_bytes == 0:
            raise L.AtlasError(1, lib.atlas_last_error().decode(errors="replace"))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device)
        flags = (1 if pe_ste else 0) | (2 if stop else 0)
        L.check(lib.atlas_scan_bwd(desc, flags, *(L.ptr(t) for t in (q, k, v, al, et, th)), L.ptr(ga),
                                   *(L.ptr(t) for t in (W1, W2, S1, S2)), L.ptr(trace), L.ptr(dyp),
                                   *(L.ptr(t) for t in cst), *(L.ptr(t) for t in (dq, dk, dv, dal, det, dth)),
                                   L.ptr(dga), *(L.ptr(t) for t in dst), L.ptr(ws), ws_bytes,
                                   L.stream_ptr(q.device)))
        grads = [g[:, :T] for g in (dq, dk, dv, dal, det, dth)] + [None if dga is None else dga[:, :T]]
        grads += [None] * 4 if stop else dst
        out = [None if g is None or dt is None else g.to(dt) for g, dt in zip(grads, ctx.dtypes)]
        return (*out, None, None, None, None, None, None)


def memory_scan_hip_autograd(q, k, v, alpha, eta, theta, gamma, state, chunk_size, omega_window, ns_steps,
                             pe_ste=False, stop_grad_chunks=False, precision=None):
    """Differentiable whole-layer scan on the HIP backward: returns
    (y (B, T, H, D) fp32, DeepMemoryState fp32) with the values of
    memory_scan's forward in `precision` (None: fp32); the backward is
    fp32."""
    from .memory_layer import DeepMemoryState
    _require_cuda(q, k, v, alpha, eta, theta)
    y, W1, W2, S1, S2 = MemoryScanHIP.apply(q, k, v, alpha, eta, theta, gamma, *state, chunk_size, omega_window,
                                           ns_steps, pe_ste, stop_grad_chunks, precision)
    return y, DeepMemoryState(W1, W2, S1, S2)
