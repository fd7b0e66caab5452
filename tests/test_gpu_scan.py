"""GPU parity of atlas_scan_fwd (through the C ABI) against the float64 oracle.

Tolerances (relative L2, from the stated bar): fp32 scan 1e-4; fp16-MFMA
scan on bf16 inputs 2e-2.  Compared per chunk from the oracle's own chunk-start
state (teacher-forced, see scan_cases.py) over whole sequences, and end to end
over short horizons.
"""

import numpy as np
import pytest

import scan_cases as SC
from oracle import atlas_ref as R

pytestmark = pytest.mark.gpu

TOL = {"f32": 1e-4, "f16": 2e-2}


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def run_gpu(inp, cs, w, ns, precision, io="f32", n_slices=0):
    torch = _torch()
    from atlas_amd import memory_scan, DeepMemoryState
    dev = "cuda"
    tio = torch.float32 if io == "f32" else torch.bfloat16

    def t(a, dt=torch.float32):
        return None if a is None else torch.tensor(np.asarray(a, np.float32), device=dev).to(dt)

    st = DeepMemoryState(*(t(s) for s in inp["state"]))
    y, new = memory_scan(t(inp["q"], tio), t(inp["k"], tio), t(inp["v"], tio), t(inp["alpha"]), t(inp["eta"]),
                         t(inp["theta"]), t(inp["gamma"]), st, cs, w, ns, precision=precision,
                         n_slices=n_slices)
    torch.cuda.synchronize()
    return y.float().cpu().numpy(), tuple(s.cpu().numpy() for s in new)


def teacher_forced(B, T, H, D, E, cs, w, ns, precision, io="f32", seed=0, init="rand", with_gamma=True,
                   n_slices=0):
    inp = SC.make_inputs(B, T, H, D, E, seed=seed, init=init, io=io, with_gamma=with_gamma)
    y_ref, states = SC.oracle_trajectory(inp, cs, w, ns)
    tf = SC.teacher_forced_inputs(inp, states, cs)
    y, st = run_gpu(tf, cs, w, ns, precision, io, n_slices)
    nc = T // cs
    return SC.worst_chunk_errors(y, st, y_ref, states, B, nc, cs)


def _assert_within(errs, tol, label):
    print(label, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    for k, v in errs.items():
        assert v <= tol, f"{label}: {k} rel-L2 {v:.3e} > {tol}"


# ---------------------------------------------------------------------------
# Config 1 (fp32, B1 T1024 H4 D32 E32 cs64 w16 ns5), every chunk
# ---------------------------------------------------------------------------

def test_c1_teacher_forced_f32():
    errs = teacher_forced(1, 1024, 4, 32, 32, 64, 16, 5, "f32", seed=0)
    _assert_within(errs, TOL["f32"], "C1 f32")


def test_c1_teacher_forced_f16():
    errs = teacher_forced(1, 1024, 4, 32, 32, 64, 16, 5, "f16", seed=0)
    _assert_within(errs, TOL["f16"], "C1 f16")


# ---------------------------------------------------------------------------
# Config-2 shape (D64 E128 cs64 w32 ns5, bf16 inputs) on a reduced B/T/H
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("init", ["model", "rand"])
def test_c2_shape_teacher_forced_f16(init):
    errs = teacher_forced(1, 512, 2, 64, 128, 64, 32, 5, "f16", io="bf16", seed=3, init=init)
    _assert_within(errs, TOL["f16"], f"C2-shape f16 {init}")


def test_c2_shape_teacher_forced_f32():
    errs = teacher_forced(1, 256, 2, 64, 128, 64, 32, 5, "f32", io="f32", seed=4, init="model")
    _assert_within(errs, TOL["f32"], "C2-shape f32")


# ---------------------------------------------------------------------------
# Wide memories (E = 256): config-3 shape (cs64 w64) and config-5 shape
# (cs128 w16) on reduced B/T/H, bf16 inputs, fp16 matrix-core operands
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("init,n_slices", [("model", 2), ("rand", 0), ("rand", 4)])
def test_c3_shape_teacher_forced_f16(init, n_slices):
    errs = teacher_forced(1, 256, 2, 64, 256, 64, 64, 5, "f16", io="bf16", seed=12, init=init, n_slices=n_slices)
    _assert_within(errs, TOL["f16"], f"C3-shape f16 {init} n_slices={n_slices}")


def test_c3_shape_tiny_momentum_f16():
    """C3 shape with k and v scaled by 1e-4: the chunk-start momenta are
    2.7e-11 .. 1e-14, far below fp16's subnormals, so the chunk-start momentum
    staged in LDS as fp16 must carry its power-of-two scale, and the
    normalisation's 1e-6 makes P and the memory tiny as well (the memory
    decays from 0.5 to 8e-6 over the four chunks)."""
    inp = SC.make_inputs(1, 256, 2, 64, 256, seed=15, init="rand", io="f32")
    for name in ("k", "v"):
        inp[name] = (inp[name] * 1e-4).astype(np.float32)
    y_ref, states = SC.oracle_trajectory(inp, 64, 64, 5)
    tf = SC.teacher_forced_inputs(inp, states, 64)
    y, st = run_gpu(tf, 64, 64, 5, "f16", "f32")
    errs = SC.worst_chunk_errors(y, st, y_ref, states, 1, 4, 64)
    _assert_within(errs, TOL["f16"], "C3-shape f16 tiny momentum")


@pytest.mark.parametrize("n_slices", [0, 8, 4])
def test_c5_shape_teacher_forced_f16(n_slices):
    errs = teacher_forced(1, 256, 2, 64, 256, 128, 16, 5, "f16", io="bf16", seed=13, init="rand",
                          n_slices=n_slices)
    _assert_within(errs, TOL["f16"], f"C5-shape f16 n_slices={n_slices}")


@pytest.mark.parametrize("T", [64, 192, 150])
def test_wide_end_to_end_f16(T):
    """State carried across 1-3 chunks (odd and even counts, ragged T)."""
    B, H, D, E, cs, w, ns = 1, 2, 64, 256, 64, 64, 5
    inp = SC.make_inputs(B, T, H, D, E, seed=14, io="bf16", init="model")
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = run_gpu(inp, cs, w, ns, "f16", io="bf16")
    errs = {"y": SC.rel_l2(y, y_ref)}
    for m, name in enumerate(("W1", "W2", "S1", "S2")):
        if np.linalg.norm(st_ref[m]) == 0:
            assert np.abs(st[m]).max() == 0.0, f"{name} must be exactly zero after padding"
        else:
            errs[name] = SC.rel_l2(st[m], st_ref[m])
    _assert_within(errs, TOL["f16"], f"wide end-to-end T={T}")


# ---------------------------------------------------------------------------
# Omega window variants, shapes, slices
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("w,with_gamma", [(1, False), (4, True), (64, True), (100, True), (8, False)])
def test_omega_variants_f32(w, with_gamma):
    errs = teacher_forced(2, 128, 2, 32, 64, 64, w, 5, "f32", seed=5, with_gamma=with_gamma)
    _assert_within(errs, TOL["f32"], f"omega w={w} gamma={with_gamma}")


@pytest.mark.parametrize("D,E", [(32, 32), (32, 64), (32, 128), (64, 64), (64, 128)])
def test_shapes_f32(D, E):
    errs = teacher_forced(1, 128, 2, D, E, 64, 16, 5, "f32", seed=6)
    _assert_within(errs, TOL["f32"], f"shape D={D} E={E}")


@pytest.mark.parametrize("cs,ns", [(8, 3), (16, 5), (32, 1), (128, 5), (64, 0)])
def test_chunk_sizes_and_steps_f32(cs, ns):
    errs = teacher_forced(1, 256, 2, 32, 64, cs, 8, ns, "f32", seed=7)
    _assert_within(errs, TOL["f32"], f"cs={cs} ns={ns}")


@pytest.mark.parametrize("n_slices", [2, 4, 8, 16])
def test_slice_counts_f32(n_slices):
    errs = teacher_forced(1, 128, 2, 32, 64, 64, 16, 5, "f32", seed=8, n_slices=n_slices)
    _assert_within(errs, TOL["f32"], f"n_slices={n_slices}")


# ---------------------------------------------------------------------------
# End to end (state carried by the library across chunks), short horizons
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("T", [64, 128, 100, 37])
def test_end_to_end_short_f32(T):
    """Two chunks end to end, and ragged T (reference padding: alpha=1,
    eta=theta=gamma=0 -> the returned momentum is zero)."""
    B, H, D, E, cs, w, ns = 2, 2, 32, 64, 64, 16, 5
    inp = SC.make_inputs(B, T, H, D, E, seed=9)
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = run_gpu(inp, cs, w, ns, "f32")
    errs = {"y": SC.rel_l2(y, y_ref)}
    for m, name in enumerate(("W1", "W2", "S1", "S2")):
        if np.linalg.norm(st_ref[m]) == 0:
            assert np.abs(st[m]).max() == 0.0, f"{name} must be exactly zero after padding"
        else:
            errs[name] = SC.rel_l2(st[m], st_ref[m])
    _assert_within(errs, TOL["f32"], f"end-to-end T={T}")


def test_end_to_end_short_f16_bf16():
    B, T, H, D, E, cs, w, ns = 1, 128, 2, 64, 128, 64, 32, 5
    inp = SC.make_inputs(B, T, H, D, E, seed=10, io="bf16", init="model")
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = run_gpu(inp, cs, w, ns, "f16", io="bf16")
    errs = {"y": SC.rel_l2(y, y_ref)}
    errs.update({n: SC.rel_l2(a, b) for n, a, b in zip(("W1", "W2", "S1", "S2"), st, st_ref)})
    _assert_within(errs, TOL["f16"], "end-to-end f16")


@pytest.mark.parametrize("n_slices,io", [(2, "bf16"), (4, "f32")])
def test_end_to_end_f16_odd_chunks(n_slices, io):
    """Three chunks (odd: the final state lands in the workspace copies) with a
    ragged tail, through the launch that runs a chunk's prep beside the
    previous chunk's read-out."""
    B, T, H, D, E, cs, w, ns = 1, 164, 2, 64, 128, 64, 32, 5
    inp = SC.make_inputs(B, T, H, D, E, seed=14, io=io)
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = run_gpu(inp, cs, w, ns, "f16", io=io, n_slices=n_slices)
    errs = {"y": SC.rel_l2(y, y_ref)}
    errs.update({n: SC.rel_l2(a, b) for n, a, b in zip(("W1", "W2", "S1", "S2"), st, st_ref)
                 if np.linalg.norm(b) > 0})
    _assert_within(errs, TOL["f16"], f"end-to-end f16 odd chunks n_slices={n_slices} io={io}")


@pytest.mark.parametrize("E", [128, 256])
def test_deterministic(E):
    inp = SC.make_inputs(1, 256, 2, 64, E, seed=11, io="bf16")
    a = run_gpu(inp, 64, 32, 5, "f16", io="bf16")
    b = run_gpu(inp, 64, 32, 5, "f16", io="bf16")
    assert np.array_equal(a[0], b[0])
    for x, y in zip(a[1], b[1]):
        assert np.array_equal(x, y)


# ---------------------------------------------------------------------------
# The benchmark's launch itself: 64 streams (C2) and 192 streams (C3) with
# the automatic slice count, bf16 inputs, fp16 compute
# ---------------------------------------------------------------------------

def _launch_case(B, H, D, E, cs, w, ns, init, seed, sample):
    """B*H streams of two chunks each from per-stream start states (random,
    with momentum, or the model's initial state), in ONE call with the
    automatic slice count -- the launch the benchmark times.  Checked two
    ways: (1) the streams in `sample` (spread over the stream index, so a
    wrong stream or slice mapping shows) end to end against the float64
    oracle at the 2e-2 bar (two chunks are inside the fp16 horizon); (2)
    every stream bitwise against the same streams run in four smaller calls
    with the same slice count (each stream's arithmetic is independent of
    the launch size and of the workgroup-to-XCD mapping)."""
    torch = _torch()
    from atlas_amd import DeepMemoryState, memory_scan
    from atlas_amd import _lib as L
    T = 2 * cs
    inp = SC.make_inputs(B, T, H, D, E, seed=seed, init=init, io="bf16", s_scale=0.0 if init == "model" else 2e-3)
    lib = L.get_lib()
    desc = L.ScanDesc(B=B, T=T, H=H, D=D, E=E, chunk_size=cs, omega_window=w, ns_steps=ns, io_dtype=L.DTYPE_BF16,
                      gate_dtype=L.DTYPE_F32, compute=L.COMPUTE_F16)
    assert lib.atlas_scan_workspace_size(desc) > 0
    print(f"launch case: {B * H} streams, D{D} E{E} cs{cs} w{w} init {init}", flush=True)

    def t(a, dt=torch.float32):
        return None if a is None else torch.tensor(np.asarray(a, np.float32), device="cuda").to(dt)

    def run(b0, b1, n_slices):
        sl = slice(b0, b1)
        st = DeepMemoryState(*(t(s[sl]) for s in inp["state"]))
        y, new = memory_scan(t(inp["q"][sl], torch.bfloat16), t(inp["k"][sl], torch.bfloat16),
                             t(inp["v"][sl], torch.bfloat16), t(inp["alpha"][sl]), t(inp["eta"][sl]),
                             t(inp["theta"][sl]), t(inp["gamma"][sl]), st, cs, w, ns, precision="f16",
                             n_slices=n_slices)
        torch.cuda.synchronize()
        return y, new

    y, st = run(0, B, 0)
    assert bool(torch.isfinite(y.float()).all()) and all(bool(torch.isfinite(s).all()) for s in st)
    # (2) the same streams in four calls with the slice count the big call chose (cs / 16 here)
    nsl = cs // 16
    q4 = B // 4
    for i in range(4):
        yi, sti = run(i * q4, (i + 1) * q4, nsl)
        assert torch.equal(yi, y[i * q4:(i + 1) * q4]), f"y of streams {i * q4}..{(i + 1) * q4 - 1} differ"
        for m, (a, b) in enumerate(zip(sti, st)):
            assert torch.equal(a, b[i * q4:(i + 1) * q4]), f"state {m} of batch rows {i * q4}.. differs"
    # (1) sampled streams against the oracle
    worst = {}
    for b, h in sample:
        one = {k_: (None if inp[k_] is None else inp[k_][b:b + 1, :, h:h + 1]) for k_ in
               ("q", "k", "v", "alpha", "eta", "theta", "gamma")}
        s0 = tuple(s[b:b + 1, h:h + 1] for s in inp["state"])
        y_ref, st_ref = R.memory_scan(one["q"], one["k"], one["v"], one["alpha"], one["eta"], one["theta"],
                                      one["gamma"], s0, cs, w, ns)
        errs = {"y": SC.rel_l2(y[b:b + 1, :, h:h + 1].float().cpu().numpy(), y_ref)}
        for name, a, r in zip(("W1", "W2", "S1", "S2"), st, st_ref):
            errs[name] = SC.rel_l2(a[b:b + 1, h:h + 1].cpu().numpy(), r)
        for k_, v_ in errs.items():
            worst[k_] = max(worst.get(k_, 0.0), v_)
    _assert_within(worst, TOL["f16"], f"{B * H}-stream launch, {len(sample)} sampled streams")


@pytest.mark.parametrize("init", ["model", "rand"])
def test_c2_benchmark_launch_64_streams(init):
    """C2's launch: 64 streams (B8 H8), D64 E128 cs64 w32, 4 slices of 16
    tokens (256 workgroups, one round), the direct cross-slice sums, W_end
    and the merged next-chunk prep + y launch."""
    sample = [(0, 0), (1, 5), (3, 2), (4, 7), (6, 3), (7, 7)]
    _launch_case(8, 8, 64, 128, 64, 32, 5, init, seed=61, sample=sample)


def test_c3_benchmark_launch_192_streams():
    """C3's launch: 192 streams (B16 H12), D64 E256 cs64 w64: the pair-of-
    waves kernels, 4 slices, 768 workgroups in three rounds."""
    sample = [(0, 0), (5, 11), (10, 4), (15, 11)]
    _launch_case(16, 12, 64, 256, 64, 64, 5, "rand", seed=62, sample=sample)
