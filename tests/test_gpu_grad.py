"""GPU parity of the backward passes against float64 torch autograd on the
CPU (oracle/atlas_ref_torch.py): the linear-scan VJP (HIP reverse-time scan,
atlas_linear_scan_bwd) and the custom VJP of fused_chunk_scan, with and
without the straight-through Polar-Express backward.  Tolerance: rel-L2
1e-4 per gradient (fp32 arithmetic)."""

import numpy as np
import pytest

import scan_cases as SC
from oracle import atlas_ref_torch as RT

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("B,T,H,shape,with_final", [(2, 16, 3, (4, 8), True), (1, 64, 2, (64, 128), True),
                                                     (2, 5, 1, (300,), False)])
def test_linear_scan_vjp(B, T, H, shape, with_final):
    torch = _torch()
    from atlas_amd import linear_scan
    g = torch.Generator().manual_seed(T)
    h0 = torch.randn(B, H, *shape, generator=g, dtype=torch.float64)
    gates = torch.rand(B, T, H, generator=g, dtype=torch.float64)
    x = torch.randn(B, T, H, *shape, generator=g, dtype=torch.float64)
    dall = torch.randn(B, T, H, *shape, generator=g, dtype=torch.float64)
    dfin = torch.randn(B, H, *shape, generator=g, dtype=torch.float64) if with_final else None
    ins = [t.clone().requires_grad_(True) for t in (h0, gates, x)]
    outs = RT.linear_scan_t(*ins)
    ref = torch.autograd.grad([outs[0]] + ([outs[1]] if with_final else []), ins,
                              [dall] + ([dfin] if with_final else []))
    gi = [t.float().cuda().requires_grad_(True) for t in (h0, gates, x)]
    h_all, h_fin = linear_scan(*gi)
    got = torch.autograd.grad([h_all] + ([h_fin] if with_final else []), gi,
                              [dall.float().cuda()] + ([dfin.float().cuda()] if with_final else []))
    for name, a, b in zip(("h_init", "gates", "inputs"), got, ref):
        e = SC.rel_l2(a.cpu().numpy(), b.numpy())
        print(f"linear_scan vjp {name}: rel-L2 {e:.2e}", flush=True)
        assert e <= 1e-5


@pytest.mark.parametrize("B,cs,H,D,E,pe_ste", [(1, 8, 2, 32, 64, False), (1, 8, 2, 32, 64, True),
                                               (2, 16, 1, 64, 128, False), (1, 6, 1, 32, 32, False)])
def test_fused_chunk_scan_vjp(B, cs, H, D, E, pe_ste):
    torch = _torch()
    from atlas_amd import fused_chunk_scan
    g = torch.Generator().manual_seed(cs + D + E)
    f64 = torch.float64
    W1 = torch.randn(B, H, D, E, generator=g, dtype=f64) / D ** 0.5
    W2 = torch.randn(B, H, E, D, generator=g, dtype=f64) / D ** 0.5
    SW1 = torch.randn(B, H, D, E, generator=g, dtype=f64) * 0.1
    SW2 = torch.randn(B, H, E, D, generator=g, dtype=f64) * 0.1
    m1 = torch.randn(B, cs, H, D, E, generator=g, dtype=f64) * 0.1
    m2 = torch.randn(B, cs, H, E, D, generator=g, dtype=f64) * 0.1
    theta = torch.sigmoid(torch.randn(B, cs, H, generator=g, dtype=f64))
    alpha = torch.sigmoid(torch.randn(B, cs, H, generator=g, dtype=f64))
    q = torch.randn(B, cs, H, D, generator=g, dtype=f64)
    q = q / q.norm(dim=-1, keepdim=True)
    inputs = [W1, W2, SW1, SW2, m1, m2, theta, alpha, q]
    outs_ref = RT.fused_chunk_regular_t(*inputs, 5, pe_ste)
    cts = [torch.randn(o.shape, generator=g, dtype=f64) for o in outs_ref]
    ref = RT.fused_chunk_vjp_t(inputs, cts, 5, pe_ste)

    gi = [t.float().cuda().requires_grad_(True) for t in inputs]
    y, st = fused_chunk_scan(*gi, 5, pe_ste)
    got = torch.autograd.grad([y, *st], gi, [c.float().cuda() for c in cts])
    torch.cuda.synchronize()
    names = ("W1", "W2", "SW1", "SW2", "momW1", "momW2", "theta", "alpha", "q")
    for name, a, b in zip(names, got, ref):
        e = SC.rel_l2(a.cpu().numpy().astype(np.float64), b.numpy())
        print(f"fused_chunk vjp pe_ste={pe_ste} {name}: rel-L2 {e:.2e}", flush=True)
        assert e <= 1e-4, f"{name}: {e:.3e}"
