"""Muon on the GPU (atlas_jax/optim.py:56-108): Nesterov momentum, Polar-Express
orthogonalisation, NorMuon variance reduction and cautious weight decay for
2-D (or stacked 3-D) weight matrices.

Polar-Express: matrices whose smaller side is <= 64 and larger side <= 256
run on the batched HIP kernels (atlas_pe_batched with the eps-free norm of
optim.py:71; one wave per matrix, a pair of waves above 128); larger ones are GEMM-shaped and go through
torch's matmul (hipBLASLt) in fp32.  The elementwise parts are torch.
"""

from typing import NamedTuple

import torch

from . import _lib as L
from .memory_layer import POLAR_EXPRESS_COEFFS, polar_express


class MuonState(NamedTuple):
    momentum: torch.Tensor        # first moment buffer
    second_moment: torch.Tensor   # factored second moment (NorMuon)


def _fits_batched_kernel(d1, d2):
    return min(d1, d2) <= 64 and max(d1, d2) <= 256


def muon_polar_express(G, steps=5):
    """Muon's Polar-Express (optim.py:69-83) on (..., d1, d2), computed in fp32
    and returned in fp32: X / (||X||_F * 1.01 + 1e-6), then `steps` odd-quintic
    iterations (tall: X (bA + cA^2) with A = X^T X; otherwise (bA + cA^2) X)."""
    if G.dim() < 2:
        raise ValueError("muon_polar_express expects (..., d1, d2)")
    d1, d2 = G.shape[-2], G.shape[-1]
    X = G.float()
    if X.is_cuda and _fits_batched_kernel(d1, d2):
        return polar_express(X, steps, precision="f32", norm_eps=False)
    if not 0 <= steps <= len(POLAR_EXPRESS_COEFFS):
        raise ValueError(f"steps must be in [0, {len(POLAR_EXPRESS_COEFFS)}]")
    L.get_lib()   # the GPU path requires the built library (no CPU fallback)
    if not X.is_cuda:
        raise ValueError("atlas_amd operates on device (cuda/hip) tensors only")
    X = X / (torch.sqrt((X * X).sum(dim=(-2, -1), keepdim=True)) * 1.01 + 1e-6)
    tall = d1 > d2
    for a, b, c in POLAR_EXPRESS_COEFFS[:steps]:
        if tall:
            A = X.mT @ X
            X = a * X + X @ (b * A + c * (A @ A))
        else:
            A = X @ X.mT
            X = a * X + (b * A + c * (A @ A)) @ X
    return X


def muon_leaf_init(param):
    """optim.py:42-53: zero momentum; second moment (..., rows, 1) for tall or
    square parameters, (..., 1, cols) for wide ones."""
    shape = param.shape
    sm = (*shape[:-2], shape[-2], 1) if shape[-2] >= shape[-1] else (*shape[:-2], 1, shape[-1])
    return MuonState(torch.zeros_like(param), torch.zeros(sm, dtype=param.dtype, device=param.device))


def muon_leaf_update(grad, state, param, learning_rate, momentum, beta2, weight_decay, ns_steps):
    """optim.py:56-108 for one parameter.  Returns (update, new MuonState);
    the caller applies param += update."""
    dtype = grad.dtype
    shape = grad.shape
    lr_scale = max(1.0, shape[-2] / shape[-1]) ** 0.5
    new_momentum = state.momentum * momentum + grad * (1 - momentum)
    g = grad * (1 - momentum) + new_momentum * momentum
    g = muon_polar_express(g, ns_steps).to(dtype)
    red = -1 if shape[-2] >= shape[-1] else -2
    n_red = shape[red]
    gf = g.float()
    v_mean = (gf * gf).mean(dim=red, keepdim=True)
    v_norm = torch.sqrt(v_mean.sum(dim=(-2, -1), keepdim=True) * n_red)
    new_second = state.second_moment * beta2 + v_mean.to(dtype) * (1 - beta2)
    step = torch.rsqrt(torch.clamp(new_second, min=1e-10).float())
    v_norm_new = torch.sqrt((v_mean * n_red * step * step).sum(dim=(-2, -1), keepdim=True))
    g = g * (step * (v_norm / torch.clamp(v_norm_new, min=1e-10))).to(dtype)
    if param is not None and weight_decay > 0:
        mask = (g * param) >= 0
        update = -(learning_rate * lr_scale * g + learning_rate * lr_scale * weight_decay * param * mask)
    else:
        update = -learning_rate * lr_scale * g
    return update, MuonState(new_momentum, new_second)


class Muon(torch.optim.Optimizer):
    """torch.optim wrapper of muon_leaf_update for 2-D / stacked 3-D parameters
    (optim.py:111-146 defaults: lr 0.02, momentum 0.95, beta2 0.9, no decay,
    5 Polar-Express steps)."""

    def __init__(self, params, lr=0.02, momentum=0.95, beta2=0.9, weight_decay=0.0, ns_steps=5):
        super().__init__(params, dict(lr=lr, momentum=momentum, beta2=beta2, weight_decay=weight_decay,
                                      ns_steps=ns_steps))

    @torch.no_grad()
    def step(self, closure=None):
        loss = closure() if closure is not None else None
        for group in self.param_groups:
            for p in group["params"]:
                if p.grad is None:
                    continue
                if p.dim() < 2:
                    raise ValueError("Muon updates matrices only (2-D or stacked 3-D)")
                st = self.state[p]
                if "muon" not in st:
                    st["muon"] = muon_leaf_init(p)
                upd, st["muon"] = muon_leaf_update(p.grad, st["muon"], p, group["lr"], group["momentum"],
                                                   group["beta2"], group["weight_decay"], group["ns_steps"])
                p.add_(upd)
        return loss
