"""GPU: the models train end to end -- gradients reach every parameter.

The reference differentiates the whole model (tests/test_model.py:49-70,
atlas_jax/train.py:138-185): projections, convolutions, polynomial
coefficients, gates, output projections, MLPs, embedding and head, and in
the standalone layer / MAG blocks the learnable initial memory
(memory_layer.py:635-643).  Here the same loss is differentiated through the
HIP forward paths (prologue kernel, memory scan, attention kernel) and their
backwards, and every parameter's gradient is compared with float64 torch
autograd of the oracle restatement (oracle/atlas_ref_torch.py atlas_forward_t
/ mag_forward_t, pinned to the NumPy oracle and to finite differences in
tests/test_oracle_grad.py).

Bounds (relative L2 per parameter tensor), fp32 model with the fp32 scan:
  - straight-through Polar-Express (pe_ste, memory_layer.py:74-76): 1e-4, or
    4x the error of the same oracle evaluated in fp32 on the CPU where that
    is larger;
  - the full Polar-Express derivative: 1e-3, or 4x the fp32 oracle's error.
    The derivative of the odd-quintic iteration amplifies forward rounding
    through every chunk: the fp32 oracle itself is 1e-4 - 3e-4 off float64
    here, and the HIP path 3e-4 - 5e-4 (both printed).
fp16 MAG model against float64: every tensor within 1e-1 (a missing or wrong
gradient path is off by O(1)) and all gradients together (one concatenated
vector) within the 16-bit bound 2e-2; gradients with a small norm, such as the
gate biases (sums over tokens that largely cancel), carry the fp16 rounding of
the activations at a larger relative size (measured up to 3.9e-2).
"""

import numpy as np
import pytest

import scan_cases as SC

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _layer_map(layer):
    """(oracle key, parameter) pairs of one memory layer."""
    out = [("c_q", layer.c_q.weight), ("c_k", layer.c_k.weight), ("c_v", layer.c_v.weight),
           ("c_proj", layer.c_proj.weight), ("W1_init", layer.W1_init), ("W2_init", layer.W2_init),
           ("ln_gamma", layer.ln_gamma)]
    if layer.poly_coeffs is not None:
        out.append(("poly_coeffs", layer.poly_coeffs))
    if layer.retrieve_gate is not None:
        out.append(("retrieve_w", layer.retrieve_gate.weight))
    for c in "qkv":
        conv = getattr(layer, "conv_" + c)
        out += [(f"conv_{c}_w", conv.weight), (f"conv_{c}_b", conv.bias)]
    for g in ("alpha", "eta", "theta", "gamma"):
        lin = getattr(layer, "gate_" + g)
        if lin is not None:
            out += [(f"gate_{g}_w", lin.weight), (f"gate_{g}_b", lin.bias)]
    return out


def _oracle_grads(torch, fwd, named, idx, targets, cfg, dtype):
    """Loss and gradients of the oracle forward in `dtype` on the CPU:
    named = [(layer index or None, key, parameter)] of the GPU model."""
    params = {"layers": [dict() for _ in range(cfg["n_layer"])]}
    leaves = []
    for li, key, prm in named:
        t = prm.detach().double().cpu().to(dtype).requires_grad_(True)
        leaves.append(t)
        if li is None:
            params[key] = t
        else:
            params["layers"][li][key] = t
    logits, _ = fwd(idx.cpu(), params, cfg)
    V = logits.shape[-1]
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, V), targets.cpu().reshape(-1))
    grads = torch.autograd.grad(loss, leaves, allow_unused=True)
    return loss.item(), [torch.zeros_like(t) if g is None else g for t, g in zip(leaves, grads)]


def _compare(named, gpu_grads, ref64, ref32, floor, factor):
    worst = 0.0
    ref32 = ref32 if ref32 is not None else [None] * len(named)
    for (li, key, prm), g, r64, r32 in zip(named, gpu_grads, ref64, ref32):
        g = np.zeros(prm.shape) if g is None else g.detach().double().cpu().numpy()
        r = r64.numpy()
        name = key if li is None else f"layer{li}.{key}"
        if np.linalg.norm(r) == 0:
            print(f"grad {name}: reference zero, |gpu| {np.abs(g).max():.1e}", flush=True)
            assert np.abs(g).max() == 0.0, name
            continue
        e = SC.rel_l2(g, r)
        e32 = SC.rel_l2(r32.numpy(), r) if r32 is not None else 0.0
        bound = max(floor, factor * e32)
        print(f"grad {name}: rel-L2 {e:.2e} (fp32 oracle {e32:.2e}, bound {bound:.1e})", flush=True)
        assert e <= bound, f"{name}: {e:.3e} > {bound:.3e}"
        worst = max(worst, e)
    return worst


@pytest.mark.parametrize("use_checkpoint,pe_ste,backward", [(True, True, None), (False, False, None),
                                                             (True, False, "torch")])
def test_atlas_model_gradients(use_checkpoint, pe_ste, backward):
    """Two-layer Atlas (the reference's small test config widened to the
    compiled head size: D 32, E 64, chunk 16, conv 2, ns 3, Omega 4, softcap
    15), fp32, T = 40 (ragged: three chunks with padding), cross-entropy
    loss; every parameter's gradient against float64 autograd.  The
    checkpointed case also carries two persistent memory tokens
    (model.py:316-320), so the scans see T = 42."""
    torch = _torch()
    from atlas_amd import Atlas, AtlasConfig
    from oracle import atlas_ref_torch as RT
    cfg = AtlasConfig(n_layer=2, n_embd=64, n_head=2, vocab_size=64, chunk_size=16, conv_kernel=2, ns_steps=3,
                      omega_window=4, poly_degree=2, memory_expand=2, logit_softcap=15.0, scan_precision="f32",
                      use_checkpoint=use_checkpoint, pe_ste=pe_ste, scan_backward=backward,
                      num_persist_mem_tokens=2 if use_checkpoint else 0)
    gen = torch.Generator(device="cuda").manual_seed(17)
    model = Atlas(cfg, generator=gen, device="cuda")
    with torch.no_grad():   # gates that vary per token
        for blk in model.blocks:
            for g in (blk.memory.gate_alpha, blk.memory.gate_eta, blk.memory.gate_theta, blk.memory.gate_gamma):
                g.weight.normal_(0.0, 0.2, generator=gen)
                g.bias.normal_(0.0, 0.5, generator=gen)
    idx = torch.randint(0, cfg.vocab_size, (2, 40), device="cuda", generator=gen)
    targets = torch.randint(0, cfg.vocab_size, (2, 40), device="cuda", generator=gen)
    print(f"Atlas gradients (use_checkpoint={use_checkpoint}, pe_ste={pe_ste}, backward={backward})", flush=True)
    logits, _ = model(idx)
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, cfg.vocab_size), targets.reshape(-1))
    loss.backward()
    torch.cuda.synchronize()
    named = [(None, "wte", model.wte.weight), (None, "lm_head", model.lm_head.weight)]
    if model.persist_mem is not None:
        named.append((None, "persist_mem", model.persist_mem))
    for li, blk in enumerate(model.blocks):
        named += [(li, k, p) for k, p in _layer_map(blk.memory)]
        named += [(li, "mlp_fc", blk.mlp.c_fc.weight), (li, "mlp_proj", blk.mlp.c_proj.weight)]
    assert {id(p) for _, _, p in named} == {id(p) for p in model.parameters()}
    ocfg = dict(n_layer=2, n_head=2, head_dim=32, expand_dim=64, poly_degree=2, max_lr=cfg.max_lr, omega_window=4,
                chunk_size=16, ns_steps=3, vocab_size=64, logit_softcap=15.0, pe_ste=pe_ste)
    l64, g64 = _oracle_grads(torch, RT.atlas_forward_t, named, idx, targets, ocfg, torch.float64)
    l32, g32 = _oracle_grads(torch, RT.atlas_forward_t, named, idx, targets, ocfg, torch.float32)
    print(f"loss gpu {loss.item():.8f} oracle {l64:.8f}", flush=True)
    assert abs(loss.item() - l64) <= 1e-5 * abs(l64)
    _compare(named, [p.grad for _, _, p in named], g64, g32, 1e-4 if pe_ste else 1e-3, 4.0)


def test_checkpointing_keeps_gradients_and_saves_memory():
    """use_checkpoint (memory_layer.py:673) drops each chunk's intermediates
    after the forward on the torch training path: the same gradients
    (bitwise: the recompute runs the same kernels), less peak memory, on one
    memory layer with 8 chunks.  (The library backward always recomputes.)"""
    torch = _torch()
    from atlas_amd import AtlasConfig, AtlasMemoryLayer
    out = {}
    for ck in (False, True):
        cfg = AtlasConfig(n_embd=256, n_head=4, chunk_size=64, omega_window=16, memory_expand=2,
                          scan_precision="f32", use_checkpoint=ck, scan_backward="torch")
        gen = torch.Generator(device="cuda").manual_seed(3)
        layer = AtlasMemoryLayer(cfg, generator=gen, device="cuda")
        x = torch.randn(2, 512, 256, device="cuda", generator=gen)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        base = torch.cuda.memory_allocated()
        y, _ = layer(x)
        (y * y).sum().backward()
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - base
        out[ck] = (peak, [None if p.grad is None else p.grad.clone() for p in layer.parameters()])
        print(f"use_checkpoint={ck}: peak {peak / 2**20:.1f} MiB", flush=True)
    assert out[True][0] < out[False][0]
    for a, b in zip(out[True][1], out[False][1]):
        assert (a is None and b is None) or torch.equal(a, b)   # ln_gamma: no gradient


def test_mag_model_gradients():
    """Two-layer MAG (memory on layer 1; attention window 12, chunk 16, D 64,
    E 128) in fp16, T = 40: every parameter's gradient, the memory layer's
    learnable initial weights included, against float64 autograd (per tensor
    1e-1, all together 2e-2)."""
    torch = _torch()
    from atlas_amd import AtlasConfig
    from atlas_amd.mag import MAGTransformer
    from oracle import atlas_ref_torch as RT
    cfg = AtlasConfig(n_layer=2, n_embd=128, n_head=2, vocab_size=64, chunk_size=16, conv_kernel=4, ns_steps=3,
                      omega_window=4, poly_degree=2, memory_expand=2, window_size=12, neural_memory_layers=(1,))
    gen = torch.Generator(device="cuda").manual_seed(29)
    model = MAGTransformer(cfg, generator=gen, device="cuda", dtype=torch.float16)
    idx = torch.randint(0, cfg.vocab_size, (1, 40), device="cuda", generator=gen)
    targets = torch.randint(0, cfg.vocab_size, (1, 40), device="cuda", generator=gen)
    print("MAG gradients (fp16)", flush=True)
    logits, _ = model(idx)
    loss = torch.nn.functional.cross_entropy(logits.float().reshape(-1, cfg.vocab_size), targets.reshape(-1))
    loss.backward()
    torch.cuda.synchronize()
    named = [(None, "wte", model.wte.weight), (None, "lm_head", model.lm_head.weight)]
    for li, blk in enumerate(model.blocks):
        named += [(li, "to_qkv", blk.attn.to_qkv.weight), (li, "to_out", blk.attn.to_out.weight),
                  (li, "mlp_fc", blk.mlp.c_fc.weight), (li, "mlp_proj", blk.mlp.c_proj.weight)]
        if blk.memory is not None:
            named += [(li, k, p) for k, p in _layer_map(blk.memory)]
            named += [(li, "gate_w", blk.gate.linear.weight), (li, "gate_b", blk.gate.linear.bias)]
    assert {id(p) for _, _, p in named} == {id(p) for p in model.parameters()}
    ocfg = dict(n_layer=2, n_head=2, head_dim=64, expand_dim=128, poly_degree=2, max_lr=cfg.max_lr, omega_window=4,
                chunk_size=16, ns_steps=3, vocab_size=64, window_size=12)
    l64, g64 = _oracle_grads(torch, RT.mag_forward_t, named, idx, targets, ocfg, torch.float64)
    print(f"loss gpu {loss.item():.6f} oracle {l64:.6f}", flush=True)
    assert abs(loss.item() - l64) <= 2e-2 * abs(l64)
    grads = [torch.zeros_like(p) if p.grad is None else p.grad for _, _, p in named]   # ln_gamma: none
    _compare(named, grads, g64, None, 1e-1, 0.0)
    flat = np.concatenate([g.detach().double().cpu().numpy().ravel() for g in grads])
    ref = np.concatenate([r.numpy().ravel() for r in g64])
    e = SC.rel_l2(flat, ref)
    print(f"MAG all gradients: rel-L2 {e:.2e}", flush=True)
    assert e <= 2e-2


def test_atlas_model_gradients_e256_library_backward():
    """The C3/C5 layer shape (D 64, E 256) inside a model trains on the
    library backward: a two-layer Atlas in fp32 (n_embd 128, 2 heads,
    memory_expand 4, chunk 16, Omega 4, ns 3, T 40 ragged) with scan_backward
    "hip", scan_train_precision "f16" -- atlas_scan_bwd's fp16 Polar-Express
    mode -- and the straight-through Polar-Express
    (pe_ste, memory_layer.py:74-76).  memory_scan raises instead of falling
    back when the route is not available; the spy below checks that it was
    taken once per layer.  The model itself is fp32, so the fp16 rounding is
    the scan's; bounds of the 16-bit bar: every tensor 1e-1, all gradients
    together 2e-2 (measured 9.7e-3).  (Through the full Polar-Express
    derivative the fp16 mode's gradients are 8e-2 (E 128) and 0.27 (E 256)
    off float64 on this model, the fp32 modes 1e-4: its derivative amplifies
    the fp16 operand rounding.)"""
    torch = _torch()
    from atlas_amd import Atlas, AtlasConfig
    from atlas_amd import autograd as AG
    from oracle import atlas_ref_torch as RT
    cfg = AtlasConfig(n_layer=2, n_embd=128, n_head=2, vocab_size=64, chunk_size=16, conv_kernel=2, ns_steps=3,
                      omega_window=4, poly_degree=2, memory_expand=4, logit_softcap=15.0, scan_precision="f32",
                      scan_backward="hip", scan_train_precision="f16", pe_ste=True)
    assert cfg.head_dim == 64 and cfg.expand_dim == 256
    assert AG.hip_backward_supported(64, 256, 16, "f16") and AG.hip_backward_supported(64, 256, 16, None)
    gen = torch.Generator(device="cuda").manual_seed(31)
    model = Atlas(cfg, generator=gen, device="cuda")
    with torch.no_grad():   # gates that vary per token
        for blk in model.blocks:
            for g in (blk.memory.gate_alpha, blk.memory.gate_eta, blk.memory.gate_theta, blk.memory.gate_gamma):
                g.weight.normal_(0.0, 0.2, generator=gen)
                g.bias.normal_(0.0, 0.5, generator=gen)
    idx = torch.randint(0, cfg.vocab_size, (2, 40), device="cuda", generator=gen)
    targets = torch.randint(0, cfg.vocab_size, (2, 40), device="cuda", generator=gen)
    calls = []
    orig = AG.memory_scan_hip_autograd

    def spy(*a, **kw):
        calls.append(kw.get("precision"))
        return orig(*a, **kw)

    AG.memory_scan_hip_autograd = spy
    try:
        print("Atlas gradients (fp32 model, E 256, library backward in fp16 mode, pe_ste)", flush=True)
        logits, _ = model(idx)
        loss = torch.nn.functional.cross_entropy(logits.reshape(-1, cfg.vocab_size), targets.reshape(-1))
        loss.backward()
        torch.cuda.synchronize()
    finally:
        AG.memory_scan_hip_autograd = orig
    assert calls == ["f16", "f16"], calls
    named = [(None, "wte", model.wte.weight), (None, "lm_head", model.lm_head.weight)]
    for li, blk in enumerate(model.blocks):
        named += [(li, k, p) for k, p in _layer_map(blk.memory)]
        named += [(li, "mlp_fc", blk.mlp.c_fc.weight), (li, "mlp_proj", blk.mlp.c_proj.weight)]
    assert {id(p) for _, _, p in named} == {id(p) for p in model.parameters()}
    ocfg = dict(n_layer=2, n_head=2, head_dim=64, expand_dim=256, poly_degree=2, max_lr=cfg.max_lr, omega_window=4,
                chunk_size=16, ns_steps=3, vocab_size=64, logit_softcap=15.0, pe_ste=True)
    l64, g64 = _oracle_grads(torch, RT.atlas_forward_t, named, idx, targets, ocfg, torch.float64)
    print(f"loss gpu {loss.item():.8f} oracle {l64:.8f}", flush=True)
    assert abs(loss.item() - l64) <= 2e-2 * abs(l64)
    grads = [torch.zeros_like(p) if p.grad is None else p.grad for _, _, p in named]   # ln_gamma: none
    _compare(named, grads, g64, None, 1e-1, 0.0)
    flat = np.concatenate([g.detach().double().cpu().numpy().ravel() for g in grads])
    ref = np.concatenate([r.numpy().ravel() for r in g64])
    e = SC.rel_l2(flat, ref)
    print(f"Atlas (E 256, fp16 training mode, pe_ste) all gradients: rel-L2 {e:.2e}", flush=True)
    assert e <= 2e-2
