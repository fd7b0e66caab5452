"""GPU parity of the generic forward path: shapes and chunk sizes the phase
kernels are not built for (any D <= 64 and E <= 256 that are multiples of 4,
E = 256 in fp32, chunk sizes outside 4..128 or not multiples of 4), against
the float64 oracle through the same C ABI (atlas_scan_fwd routes them).

The reference layer takes any head and memory sizes (memory_layer.py
:392-419; only its fused plugin needs powers of two).  Compared per chunk
from the oracle's chunk-start states (teacher-forced, scan_cases.py) and end
to end over short horizons (ragged T included), at the fp32 bar 1e-4 and
the fp16-operand bar 2e-2; the forward's state trace of the generic path
against chunk-prefix runs; and a memory layer of head size 48 trained end to
end (the torch-composed backward) against float64 autograd."""

import numpy as np
import pytest

import scan_cases as SC
from oracle import atlas_ref as R
from test_gpu_scan import TOL, _assert_within, run_gpu, teacher_forced

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D,E", [(48, 96), (32, 96), (16, 48), (64, 256), (40, 200), (96, 192), (128, 256),
                                 (96, 96), (128, 128)])
def test_generic_shapes_teacher_forced_f32(D, E):
    errs = teacher_forced(1, 128, 2, D, E, 64, 16, 5, "f32", seed=31)
    _assert_within(errs, TOL["f32"], f"generic D={D} E={E} f32")


@pytest.mark.parametrize("D,E", [(48, 96), (64, 256), (96, 192)])
def test_generic_shapes_teacher_forced_f16(D, E):
    errs = teacher_forced(1, 128, 2, D, E, 64, 32, 5, "f16", io="bf16", seed=32)
    _assert_within(errs, TOL["f16"], f"generic D={D} E={E} f16")


@pytest.mark.parametrize("cs,w", [(6, 3), (50, 16), (256, 64), (512, 64), (1000, 128)])
def test_generic_chunk_sizes_f32(cs, w):
    T = 2 * cs if cs < 256 else cs
    errs = teacher_forced(1, T, 2, 32, 64, cs, w, 5, "f32", seed=33)
    _assert_within(errs, TOL["f32"], f"generic cs={cs} w={w}")


@pytest.mark.parametrize("D,E,init", [(64, 128, "model"), (32, 128, "rand")])
def test_chunk128_f32_over_phase_lds(D, E, init):
    """fp32 at chunk 128 with E = 128: the fp32 phase kernel's LDS layout
    needs more than a CU's 160 KiB there (218 / 164 KB), so make_plan refuses
    the shape and atlas_scan_fwd takes the generic forward (found by a
    1 024-case run of test_gpu_sweep, where the launch used to fail).  Checked
    as the sweep checks its cases (float64 oracle per chunk; the fp32 floor
    where 128-token decays reach fp32's denormal range)."""
    from test_gpu_sweep import check_case
    c = dict(D=D, E=E, cs=128, w=1 if init == "model" else 16, ns=5, nc=2, H=2, gamma=True, init=init,
             precision="f32", seed=36, io="f32")
    check_case(c, f"chunk 128 D={D} E={E} f32")


@pytest.mark.parametrize("T", [96, 70])
def test_generic_end_to_end_f32(T):
    """Two chunks carried by the library (and ragged T: the padded rows leave
    zero momentum, memory_layer.py:650-660).  End to end the recurrence
    amplifies rounding (tests/test_precision_drift.py), so the bound is the
    fp32-relative one of the golden end-to-end tests: at most 3x the worst
    member of an ensemble of fp32 evaluations of the reference semantics."""
    from test_gpu_golden import _e2e_check, _fp32_envelope
    B, H, D, E, cs, w, ns = 2, 2, 48, 96, 48, 8, 5
    inp = SC.make_inputs(B, T, H, D, E, seed=34)
    y_ref, st_ref = R.memory_scan(inp["q"], inp["k"], inp["v"], inp["alpha"], inp["eta"], inp["theta"],
                                  inp["gamma"], inp["state"], cs, w, ns)
    y, st = run_gpu(inp, cs, w, ns, "f32")
    errs = {"y": SC.rel_l2(y, y_ref)}
    for m, name in enumerate(("W1", "W2", "S1", "S2")):
        if np.linalg.norm(st_ref[m]) == 0:
            assert np.abs(st[m]).max() == 0.0, f"{name} must be exactly zero after padding"
        else:
            errs[name] = SC.rel_l2(st[m], st_ref[m])
    env = _fp32_envelope(inp, inp["state"], cs, w, ns, y_ref, st_ref)
    _e2e_check(f"generic end-to-end T={T}", errs, {k: env[k] for k in errs})


def test_generic_state_trace():
    """atlas_scan_fwd_trace on the generic path writes each chunk's start
    state: the final state of the same scan on the chunk prefix (bitwise,
    the same kernels)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from atlas_amd import DeepMemoryState
    from atlas_amd.memory_layer import _scan_forward
    inp = SC.make_inputs(1, 144, 2, 48, 96, seed=35, s_scale=0.05)
    t = [torch.tensor(inp[n], dtype=torch.float32, device="cuda") for n in
         ("q", "k", "v", "alpha", "eta", "theta", "gamma")]
    st = DeepMemoryState(*(torch.tensor(s, dtype=torch.float32, device="cuda") for s in inp["state"]))
    y, fin, tr = _scan_forward(*t, st, 48, 16, 5, precision="f32", trace=True)
    torch.cuda.synchronize()
    assert tr.shape == (3, 4, 1, 2, 48 * 96)
    for c in (1, 2):
        _, pre = _scan_forward(*(a[:, :48 * c] for a in t), st, 48, 16, 5, precision="f32")
        torch.cuda.synchronize()
        for i, s in enumerate(pre):
            assert torch.equal(tr[c, i].reshape(s.shape), s), (c, i)


def test_generic_layer_trains():
    """AtlasMemoryLayer with head size 48 (E 96): forward on the generic
    path, gradients through the torch-composed training path (the library
    backward is built for D 32/64) against float64 autograd of the layer
    oracle, within 1e-3 (fp32)."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from atlas_amd import AtlasConfig, AtlasMemoryLayer
    from oracle import atlas_ref_torch as RT
    cfg = AtlasConfig(n_embd=96, n_head=2, chunk_size=16, conv_kernel=2, ns_steps=3, omega_window=4,
                      memory_expand=2, scan_precision="f32")
    gen = torch.Generator(device="cuda").manual_seed(41)
    layer = AtlasMemoryLayer(cfg, generator=gen, device="cuda")
    with torch.no_grad():
        for g in (layer.gate_alpha, layer.gate_eta, layer.gate_theta, layer.gate_gamma):
            g.weight.normal_(0.0, 0.2, generator=gen)
            g.bias.normal_(0.0, 0.5, generator=gen)
    x = torch.randn(1, 40, 96, device="cuda", generator=gen)
    y, _ = layer(x)
    ct = torch.randn(y.shape, device="cuda", generator=gen)
    (y * ct).sum().backward()
    torch.cuda.synchronize()
    names = [("c_q", layer.c_q.weight), ("c_v", layer.c_v.weight), ("W1_init", layer.W1_init),
             ("gate_eta_w", layer.gate_eta.weight), ("conv_k_w", layer.conv_k.weight)]
    p = {"c_q": layer.c_q.weight, "c_k": layer.c_k.weight, "c_v": layer.c_v.weight, "c_proj": layer.c_proj.weight,
         "poly_coeffs": layer.poly_coeffs, "W1_init": layer.W1_init, "W2_init": layer.W2_init,
         "retrieve_w": layer.retrieve_gate.weight}
    for c in "qkv":
        conv = getattr(layer, "conv_" + c)
        p[f"conv_{c}_w"], p[f"conv_{c}_b"] = conv.weight, conv.bias
    for g in ("alpha", "eta", "theta", "gamma"):
        lin = getattr(layer, "gate_" + g)
        p[f"gate_{g}_w"], p[f"gate_{g}_b"] = lin.weight, lin.bias
    pt = {k: v.detach().double().cpu().requires_grad_(True) for k, v in p.items()}
    ocfg = dict(n_head=2, head_dim=48, expand_dim=96, poly_degree=2, max_lr=cfg.max_lr, omega_window=4,
                chunk_size=16, ns_steps=3)
    y_r, _ = RT.memory_layer_forward_t(x.double().cpu(), pt, ocfg)
    e_y = SC.rel_l2(y.detach().cpu().numpy(), y_r.detach().numpy())
    print(f"generic layer forward: rel-L2 {e_y:.2e}", flush=True)
    assert e_y <= 1e-4
    (y_r * ct.double().cpu()).sum().backward()
    for key, prm in names:
        e = SC.rel_l2(prm.grad.double().cpu().numpy(), pt[key].grad.numpy())
        print(f"generic layer grad {key}: rel-L2 {e:.2e}", flush=True)
        assert e <= 1e-3, key
