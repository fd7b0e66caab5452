"""GPU parity of Muon's Polar-Express and leaf update (optim.py:56-108)
against the float64 oracle.  Small matrices (<= 64 x 256) run on the batched
HIP kernels, larger ones on the fp32 GEMM chain.  Tolerance: rel-L2 1e-4
(fp32 arithmetic)."""

import numpy as np
import pytest

import scan_cases as SC
from oracle import atlas_ref as R

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


@pytest.mark.parametrize("shape", [(3, 48, 80), (5, 128, 64), (3, 64, 256), (2, 200, 40), (512, 512), (2, 1024, 512), (512, 1365)])
def test_muon_polar_express(shape):
    torch = _torch()
    from atlas_amd import muon_polar_express
    g = torch.Generator(device="cuda").manual_seed(1)
    G = torch.randn(*shape, device="cuda", generator=g)
    Y = muon_polar_express(G, 5)
    torch.cuda.synchronize()
    ref = R.muon_polar_express(G.cpu().numpy().astype(np.float64), 5)
    e = SC.rel_l2(Y.cpu().numpy(), ref)
    print(f"muon PE {shape}: rel-L2 {e:.2e}", flush=True)
    assert e < 1e-4


@pytest.mark.parametrize("shape,wd", [((96, 160), 0.0), ((384, 256), 0.01)])
def test_muon_leaf_update(shape, wd):
    torch = _torch()
    from atlas_amd import MuonState, muon_leaf_update
    g = torch.Generator(device="cuda").manual_seed(2)
    grad = torch.randn(*shape, device="cuda", generator=g)
    mom = torch.randn(*shape, device="cuda", generator=g) * 0.5
    sm_shape = (shape[0], 1) if shape[0] >= shape[1] else (1, shape[1])
    sec = torch.rand(*sm_shape, device="cuda", generator=g) * 1e-3
    param = torch.randn(*shape, device="cuda", generator=g)
    upd, st = muon_leaf_update(grad, MuonState(mom, sec), param, 0.02, 0.95, 0.9, wd, 5)
    torch.cuda.synchronize()
    n = lambda t: t.cpu().numpy().astype(np.float64)  # noqa: E731
    u_ref, m_ref, s_ref = R.muon_leaf_update(n(grad), n(mom), n(sec), n(param), 0.02, 0.95, 0.9, wd, 5)
    for name, a, b in (("update", upd, u_ref), ("momentum", st.momentum, m_ref), ("second", st.second_moment, s_ref)):
        e = SC.rel_l2(n(a), b)
        print(f"muon leaf {shape} {name}: rel-L2 {e:.2e}", flush=True)
        assert e < 1e-4


def test_muon_optimizer_step():
    torch = _torch()
    from atlas_amd import Muon
    g = torch.Generator(device="cuda").manual_seed(3)
    w = torch.nn.Parameter(torch.randn(64, 96, device="cuda", generator=g))
    w0 = w.detach().clone()
    opt = Muon([w], lr=0.01)
    w.grad = torch.randn(64, 96, device="cuda", generator=g)
    opt.step()
    torch.cuda.synchronize()
    assert not torch.equal(w.detach(), w0)
    assert torch.isfinite(w).all()
