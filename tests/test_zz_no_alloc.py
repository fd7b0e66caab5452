"""GPU: the allocation-free scan entry point (atlas_scan_fwd_noalloc) against
the workspace entry point (atlas_scan_fwd), both through the C ABI.

Two calls in a row on the same GPU share the library's scratch array: the
first at the config-2 per-layer shape (B8 H8 D64 E128 cs64, 17 chunks, bf16
inputs, fp16 matrix-core mode; its default workspace is larger than the
scratch, so the allocation-free call holds the gate tables of fewer chunks at
a time, an odd count ending in a one-chunk window), the second smaller (B2, a ragged T of 150, fp32
parity mode) so that it runs over the first call's leftovers.  The same
kernels run in the same order on the same inputs, so the outputs must agree
bit for bit with the workspace entry point's.  A shape whose workspace cannot
fit the scratch is refused with ATLAS_ERR_WORKSPACE before any GPU work."""

import ctypes

import pytest

pytestmark = pytest.mark.gpu


def _torch():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def _inputs(torch, B, T, H, D, E, io, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q, k, v = (torch.nn.functional.normalize(torch.randn(B, T, H, D, device="cuda", generator=g), dim=-1).to(io)
               for _ in range(3))
    gates = [torch.sigmoid(torch.randn(B, T, H, device="cuda", generator=g)) for _ in range(4)]
    gates[1] = gates[1] * 0.1
    W1 = torch.randn(B, H, D, E, device="cuda", generator=g) / D ** 0.5
    W2 = torch.randn(B, H, E, D, device="cuda", generator=g) / D ** 0.5
    S1 = torch.randn(B, H, D, E, device="cuda", generator=g) * 1e-3
    S2 = torch.randn(B, H, E, D, device="cuda", generator=g) * 1e-3
    return (q, k, v), gates, (W1, W2, S1, S2)


def _run(torch, lib, L, desc, xs, gates, state, noalloc):
    st = [s.clone() for s in state]
    y = torch.empty_like(xs[0])
    ptrs = [L.ptr(t) for t in (*xs, *gates)] + [L.ptr(s) for s in st] + [L.ptr(y)]
    stream = L.stream_ptr(xs[0].device)
    if noalloc:
        rc = lib.atlas_scan_fwd_noalloc(desc, *ptrs, stream)
    else:
        ws_bytes = lib.atlas_scan_workspace_size(desc)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda")
        rc = lib.atlas_scan_fwd(desc, *ptrs, L.ptr(ws), ws_bytes, stream)
    L.check(rc)
    torch.cuda.synchronize()
    return y, st


@pytest.mark.parametrize("first,second", [
    (dict(B=8, T=1088, io="bf16", compute=1), dict(B=2, T=150, io="f32", compute=0)),
])
def test_noalloc_matches_workspace_entry_point(first, second):
    torch = _torch()
    from atlas_amd import _lib as L
    lib = L.get_lib()
    H, D, E, cs, w, ns = 8, 64, 128, 64, 32, 5
    assert lib.atlas_scan_noalloc_scratch_bytes() == 64 << 20
    big = L.ScanDesc(B=8, T=1088, H=H, D=D, E=E, chunk_size=cs, omega_window=w, ns_steps=ns, io_dtype=1,
                     gate_dtype=0, compute=1)
    assert lib.atlas_scan_workspace_size(big) > lib.atlas_scan_noalloc_scratch_bytes()
    for call, cfg in enumerate((first, second)):
        io = torch.bfloat16 if cfg["io"] == "bf16" else torch.float32
        print(f"noalloc call {call}: B{cfg['B']} T{cfg['T']} H{H} D{D} E{E} io {cfg['io']} "
              f"compute {cfg['compute']}", flush=True)
        xs, gates, state = _inputs(torch, cfg["B"], cfg["T"], H, D, E, io, seed=100 + call)
        desc = L.ScanDesc(B=cfg["B"], T=cfg["T"], H=H, D=D, E=E, chunk_size=cs, omega_window=w, ns_steps=ns,
                          io_dtype=L.dtype_code(io), gate_dtype=L.DTYPE_F32, compute=cfg["compute"])
        y_ref, st_ref = _run(torch, lib, L, desc, xs, gates, state, noalloc=False)
        y, st = _run(torch, lib, L, desc, xs, gates, state, noalloc=True)
        assert torch.equal(y, y_ref), f"call {call}: y differs"
        for name, a, b in zip(("W1", "W2", "S1", "S2"), st, st_ref):
            assert torch.equal(a, b), f"call {call}: {name} differs"
        assert torch.isfinite(y.float()).all()


def test_noalloc_refuses_workspace_beyond_scratch():
    _torch()
    from atlas_amd import _lib as L
    lib = L.get_lib()
    # the config-3 layer (192 streams, E = 256) needs more than 64 MiB
    desc = L.ScanDesc(B=16, T=4096, H=12, D=64, E=256, chunk_size=64, omega_window=64, ns_steps=5,
                      io_dtype=L.DTYPE_BF16, gate_dtype=L.DTYPE_F32, compute=L.COMPUTE_F16)
    # NULL tensor pointers: the shape is refused before the pointers are looked
    # at; were it ever accepted, the host's NULL check would return an error
    # (rc 1) before any launch instead of handing kernels made-up addresses
    null = ctypes.c_void_p(0)
    rc = lib.atlas_scan_fwd_noalloc(desc, *([null] * 7), *([null] * 4), null, null)
    assert rc == 4 and "workspace" in lib.atlas_last_error().decode()


def test_noalloc_refuses_per_token_path_shapes():
    """Shapes that atlas_scan_fwd sends to its per-token path (here D = 48)
    are refused by the allocation-free entry with ATLAS_ERR_UNSUPPORTED_SHAPE
    (NULL tensor pointers, as above: nothing can launch)."""
    _torch()
    from atlas_amd import _lib as L
    lib = L.get_lib()
    desc = L.ScanDesc(B=1, T=128, H=2, D=48, E=96, chunk_size=64, omega_window=16, ns_steps=5,
                      io_dtype=L.DTYPE_F32, gate_dtype=L.DTYPE_F32, compute=L.COMPUTE_F32)
    null = ctypes.c_void_p(0)
    rc = lib.atlas_scan_fwd_noalloc(desc, *([null] * 7), *([null] * 4), null, null)
    assert rc == 2, (rc, lib.atlas_last_error().decode())
