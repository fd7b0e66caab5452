"""GPU parity of atlas_pe_batched (Polar-Express) against the float64 oracle
(memory_layer.py:43-71) and its SVD closed form.  Tolerance: rel-L2 1e-4 in
fp32 mode; 2e-2 in fp16-MFMA mode."""

import os

import numpy as np
import pytest

from oracle import atlas_ref as R
import scan_cases as SC

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _pe_gpu(X, ns, precision, dtype="f32", norm_eps=True):
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from atlas_amd import polar_express
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dtype]
    t = torch.tensor(np.asarray(X, np.float32), device="cuda").to(dt)
    y = polar_express(t, ns, precision=precision, norm_eps=norm_eps)
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


SHAPES = [(8, 32, 32), (6, 64, 64), (5, 64, 128), (5, 128, 64), (7, 16, 48), (3, 40, 100), (4, 32, 128),
          (5, 64, 256), (3, 256, 64), (3, 20, 200), (4, 50, 160),
          # short sides 65..128: the workgroup-per-matrix kernel (head dims 96 and
          # 128 of the reference's default and wide configurations)
          (3, 96, 192), (3, 192, 96), (2, 128, 256), (2, 256, 128), (3, 96, 96), (2, 100, 200), (2, 70, 90)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("ns", [0, 1, 5])
def test_pe_f32(shape, ns):
    rng = np.random.default_rng(hash(shape) % 2**32 + ns)
    X = rng.standard_normal(shape).astype(np.float32).astype(np.float64)
    ref = R.polar_express(X, ns)
    got = _pe_gpu(X, ns, "f32")
    err = SC.rel_l2(got, ref)
    print(shape, ns, f"{err:.2e}")
    assert err <= 1e-4


@pytest.mark.parametrize("shape", SHAPES)
def test_pe_f16(shape):
    rng = np.random.default_rng(7 + shape[1])
    X = rng.standard_normal(shape).astype(np.float32).astype(np.float64)
    ref = R.polar_express(X, 5)
    got = _pe_gpu(X, 5, "f16")
    err = SC.rel_l2(got, ref)
    print(shape, f"{err:.2e}")
    assert err <= 2e-2


def test_pe_bf16_io_and_no_eps_norm():
    rng = np.random.default_rng(3)
    X = SC.bf16_round(rng.standard_normal((4, 64, 128)))
    ref = R.muon_polar_express(X, 5)
    got = _pe_gpu(X, 5, "f32", dtype="bf16", norm_eps=False)
    # output rounded to bf16 (2^-9 relative)
    assert SC.rel_l2(got, ref) <= 5e-3


def test_pe_matches_svd_form_and_zero_input():
    rng = np.random.default_rng(4)
    X = rng.standard_normal((3, 64, 128)).astype(np.float32).astype(np.float64)
    got = _pe_gpu(X, 5, "f32")
    assert SC.rel_l2(got, R.polar_express_svd(X, 5)) <= 1e-4
    z = _pe_gpu(np.zeros((2, 32, 64)), 5, "f32")
    assert np.abs(z).max() == 0.0


@pytest.mark.parametrize("d1,d2", [(64, 128), (128, 64), (64, 64), (32, 128), (32, 32), (64, 256), (256, 64)])
@pytest.mark.parametrize("precision", ["f32", "f16"])
def test_pe_vjp_batched(d1, d2, precision):
    """atlas_pe_vjp_batched against float64 autograd of polar_express
    (oracle/atlas_ref_torch.polar_express_t): momentum-like matrices (a
    random part and a few rank-1 terms), ns 0, 1 and 5, and a batch scaled
    to 1e-7 (momentum below the normalisation's 1e-6, the case that needs
    the fp16 operands' power-of-two scaling).  fp32 operands within 1e-5,
    fp16 operands within 5e-3 rel-L2 (simulated: 9e-4 mean, 1.8e-3 worst).
    64 x 256 runs on a pair of waves in fp16, and in fp32 on the
    workgroup-per-matrix kernel with the iterate and cotangent in its global
    scratch."""
    torch = _torch()
    from atlas_amd.autograd import polar_express_vjp
    from oracle import atlas_ref_torch as RT
    g = torch.Generator().manual_seed(d1 * 7 + d2)
    n = 24
    X = torch.randn(n, d1, d2, generator=g, dtype=torch.float64) * 0.1
    for _ in range(3):
        X = X + torch.randn(n, d1, 1, generator=g, dtype=torch.float64) * torch.randn(n, 1, d2, generator=g,
                                                                                       dtype=torch.float64)
    X[n // 2:] *= 1e-7
    G = torch.randn(n, d1, d2, generator=g, dtype=torch.float64)
    bound = 1e-5 if precision == "f32" else 5e-3
    for ns in (0, 1, 5):
        Xr = X.clone().requires_grad_(True)
        ref, = torch.autograd.grad(RT.polar_express_t(Xr, ns), Xr, G)
        got = polar_express_vjp(X.float().cuda(), G.float().cuda(), ns, precision=precision)
        torch.cuda.synchronize()
        for lo, hi, what in ((0, n // 2, "unit"), (n // 2, n, "tiny")):
            e = SC.rel_l2(got[lo:hi].double().cpu().numpy(), ref[lo:hi].numpy())
            print(f"pe vjp {d1}x{d2} {precision} ns {ns} {what}: rel-L2 {e:.2e}", flush=True)
            assert e <= bound, (ns, what, e)


@pytest.mark.parametrize("d1,d2", [(64, 256), (256, 64)])
def test_pe_vjp_pair_many_matrices(d1, d2):
    """The 64 x 256 fp16 VJP (a pair of waves per matrix, partial products
    summed through the pair's LDS) over 256 matrices, enough workgroups for
    every CU to run both pairs concurrently: finite everywhere and within the
    fp16 bound of float64 autograd.  (A batch of 24 did not expose a missing
    barrier before the pair's exchange, which a batch of 128 turned into
    NaNs.)"""
    torch = _torch()
    from atlas_amd.autograd import polar_express_vjp
    from oracle import atlas_ref_torch as RT
    g = torch.Generator().manual_seed(d1 + 3 * d2)
    n = 256
    X = torch.randn(n, d1, d2, generator=g, dtype=torch.float64) * 0.1
    X = X + torch.randn(n, d1, 1, generator=g, dtype=torch.float64) * torch.randn(n, 1, d2, generator=g,
                                                                                  dtype=torch.float64)
    G = torch.randn(n, d1, d2, generator=g, dtype=torch.float64)
    Xr = X.clone().requires_grad_(True)
    ref, = torch.autograd.grad(RT.polar_express_t(Xr, 5), Xr, G)
    got = polar_express_vjp(X.float().cuda(), G.float().cuda(), 5, precision="f16")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(got).all())
    e = SC.rel_l2(got.double().cpu().numpy(), ref.numpy())
    print(f"pe vjp pair {d1}x{d2} n {n}: rel-L2 {e:.2e}", flush=True)
    assert e <= 5e-3


@pytest.mark.parametrize("d1,d2", [(64, 256), (256, 64)])
def test_pe_vjp_f32_wide_many_matrices(d1, d2):
    """The 64 x 256 fp32 VJP (one workgroup per matrix, the iterate and the
    cotangent in the workgroup's global scratch) over 300 matrices: more
    than the 256 persistent workgroups, so some take a second matrix over
    their scratch's previous contents.  Every matrix within the fp32 bound
    (1e-5 rel-L2) of float64 autograd."""
    torch = _torch()
    from atlas_amd.autograd import polar_express_vjp
    from oracle import atlas_ref_torch as RT
    g = torch.Generator().manual_seed(d1 + 5 * d2)
    n = 300
    X = torch.randn(n, d1, d2, generator=g, dtype=torch.float64) * 0.1
    X = X + torch.randn(n, d1, 1, generator=g, dtype=torch.float64) * torch.randn(n, 1, d2, generator=g,
                                                                                  dtype=torch.float64)
    G = torch.randn(n, d1, d2, generator=g, dtype=torch.float64)
    Xr = X.clone().requires_grad_(True)
    ref, = torch.autograd.grad(RT.polar_express_t(Xr, 5), Xr, G)
    got = polar_express_vjp(X.float().cuda(), G.float().cuda(), 5, precision="f32").double().cpu()
    torch.cuda.synchronize()
    errs = (got - ref).flatten(1).norm(dim=1) / ref.flatten(1).norm(dim=1)
    print(f"pe vjp f32 {d1}x{d2} n {n}: worst per-matrix rel-L2 {errs.max().item():.2e}", flush=True)
    assert bool(torch.isfinite(got).all()) and errs.max().item() <= 1e-5


@pytest.mark.parametrize("shape", [(4, 64, 128), (4, 128, 64), (3, 64, 256), (2, 96, 192)])
@pytest.mark.parametrize("precision", ["f32", "f16"])
def test_pe_fp16_io(shape, precision):
    """fp16 input and output (ATLAS_DTYPE_F16) through the one-wave, pair
    and workgroup-per-matrix kernels: against the float64 oracle of the
    fp16-rounded input, within the compute mode's bar plus the output's
    fp16 rounding (2^-11 relative per element, 5e-4 rel-L2 allowed)."""
    rng = np.random.default_rng(11 + shape[1] + shape[2])
    X = rng.standard_normal(shape).astype(np.float16).astype(np.float64)
    ref = R.polar_express(X, 5)
    got = _pe_gpu(X, 5, precision, dtype="f16")
    err = SC.rel_l2(got, ref)
    print(shape, precision, f"{err:.2e}")
    assert err <= (1e-4 + 5e-4 if precision == "f32" else 2e-2)


def _draw_pe_cases(n, seed):
    """Seeded Polar-Express cases over the whole supported range: any sizes
    with the short side <= 128 and the long side <= 256 (odd sizes
    included: the kernels pad to their tiles), one to five matrices, 0-5
    steps, with and without the normalisation's epsilon, fp32 compute on
    fp32 data or fp16 compute on bf16 / fp16 data."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        a, b = int(rng.integers(1, 129)), int(rng.integers(1, 257))
        d1, d2 = (a, b) if rng.random() < 0.5 else (b, a)
        prec = "f16" if rng.random() < 0.4 else "f32"
        io = ("bf16" if rng.random() < 0.5 else "f16") if prec == "f16" else "f32"
        out.append(dict(n=int(rng.integers(1, 6)), d1=d1, d2=d2, ns=int(rng.integers(0, 6)), precision=prec,
                        io=io, norm_eps=bool(rng.random() < 0.8), seed=int(rng.integers(1 << 30))))
    return out


# ATLAS_PE_SWEEP_CASES draws a longer sweep (the first cases are the same)
PE_CASES = _draw_pe_cases(int(os.environ.get("ATLAS_PE_SWEEP_CASES", "24")), seed=20261206)


@pytest.mark.parametrize("idx", range(len(PE_CASES)))
def test_pe_sweep(idx):
    """Against the float64 oracle on the same (io-rounded) input: rel-L2 1e-4
    in fp32 compute; in fp16 compute 2e-2, or 3x the error of a CPU
    simulation of the iteration with fp16-rounded operands and fp32
    accumulation (test_precision_choice._pe_rounded) where that is larger:
    thin matrices after few steps amplify operand rounding (a 234 x 7 case
    at three steps: 2.15e-2 on the GPU, 1.2e-2 .. 1.6e-2 simulated over
    seeds, the GPU's own rounding order being another sample)."""
    c = PE_CASES[idx]
    print(f"pe sweep case {idx}: {c}", flush=True)
    rng = np.random.default_rng(c["seed"])
    X = rng.standard_normal((c["n"], c["d1"], c["d2"])).astype(np.float32)
    if c["io"] != "f32":
        torch = _torch()
        dt = torch.bfloat16 if c["io"] == "bf16" else torch.float16
        X = torch.tensor(X).to(dt).float().numpy()   # the oracle sees the rounded input
    X = X.astype(np.float64)
    ref = R.polar_express(X, c["ns"]) if c["norm_eps"] else R.muon_polar_express(X, c["ns"])
    got = _pe_gpu(X, c["ns"], c["precision"], c["io"], norm_eps=c["norm_eps"])
    err = SC.rel_l2(got, ref)
    bound = 1e-4
    if c["precision"] == "f16":
        from test_precision_choice import _pe_rounded
        bound = max(2e-2, 3.0 * SC.rel_l2(_pe_rounded("f16")(X, c["ns"]), ref))
    print(f"pe sweep case {idx}: rel-L2 {err:.2e} (bound {bound:.2e})", flush=True)
    assert err <= bound, f"case {idx} {c}: {err:.3e} > {bound:.3e}"
