"""CPU: the C-ABI library loads, exports every function include/atlas_scan.h
declares, agrees with the ctypes descriptor layout, and rejects bad arguments
on the host (no GPU work is launched by these calls)."""

import ctypes
import os
import subprocess

import pytest

import __graft_entry__  # noqa: F401  (sets sys.path)
from atlas_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(L.LIB_PATH):
        from atlas_amd.build import build
        build()
    return L.get_lib()


def test_exports_every_declared_symbol(lib):
    declared = L.header_symbols()
    assert "atlas_scan_fwd" in declared and len(declared) >= 9
    out = subprocess.run(["nm", "-D", "--defined-only", L.LIB_PATH], capture_output=True, text=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        getattr(lib, s)


def test_abi_version(lib):
    assert lib.atlas_abi_version() == 1


def test_desc_layout_matches_header(tmp_path):
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "atlas_scan.h"\n'
                   'int main(void){printf("%zu %zu %zu\\n", sizeof(atlas_scan_desc), '
                   'offsetof(atlas_scan_desc, x_stride_b), offsetof(atlas_scan_desc, g_stride_t));return 0;}\n')
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)], check=True)
    size, off_b, off_gt = map(int, subprocess.run([str(exe)], capture_output=True, text=True).stdout.split())
    assert size == ctypes.sizeof(L.ScanDesc)
    assert off_b == L.ScanDesc.x_stride_b.offset
    assert off_gt == L.ScanDesc.g_stride_t.offset


def _desc(**kw):
    base = dict(B=8, T=4096, H=8, D=64, E=128, chunk_size=64, omega_window=32, ns_steps=5, io_dtype=1,
                gate_dtype=0, compute=1)
    base.update(kw)
    return L.ScanDesc(**base)


def test_workspace_size_and_shape_errors(lib):
    assert lib.atlas_scan_workspace_size(_desc()) > 0
    for bad, word in ((dict(D=132), "not compiled"), (dict(ns_steps=6), "ns_steps"), (dict(compute=7), "compute"),
                      (dict(T=0), "must be >= 1"), (dict(n_slices=3), "n_slices")):
        assert lib.atlas_scan_workspace_size(_desc(**bad)) == 0
        assert word in lib.atlas_last_error().decode()


def test_generic_path_shapes(lib):
    """Shapes and chunk sizes the phase kernels are not built for take the
    generic per-token path (its workspace holds the chunk's per-token
    matrices, so it is larger than the phase kernels'); D above 128 or E
    above 256 or not multiples of 4 are refused."""
    fast = lib.atlas_scan_workspace_size(_desc())
    for ok in (dict(chunk_size=6), dict(D=48, E=96), dict(D=32, E=200), dict(E=256, compute=0),
               dict(D=16, E=48, chunk_size=256), dict(x_stride_h=68), dict(D=96, E=192), dict(D=128, E=256)):
        n = lib.atlas_scan_workspace_size(_desc(**ok))
        assert n > 0, ok
    assert lib.atlas_scan_workspace_size(_desc(chunk_size=6)) > fast
    for bad in (dict(D=132), dict(D=48, E=98), dict(E=264), dict(D=30)):
        assert lib.atlas_scan_workspace_size(_desc(**bad)) == 0, bad


def test_wide_memory_shapes(lib):
    """E = 256 (configs 3 and 5) is planned for the pair kernels with fp16
    matrix-core operands; its fp32 mode takes the generic path (a larger
    workspace); E = 512 is not built."""
    assert lib.atlas_scan_workspace_size(_desc(E=256, B=16, H=12, omega_window=64)) > 0
    assert lib.atlas_scan_workspace_size(_desc(E=256, B=4, T=16384, H=12, chunk_size=128, omega_window=16)) > 0
    assert lib.atlas_scan_workspace_size(_desc(E=256, compute=0)) > lib.atlas_scan_workspace_size(_desc(E=256))
    assert lib.atlas_scan_workspace_size(_desc(E=512)) == 0
    assert "not compiled" in lib.atlas_last_error().decode()
    # the wide path's extra workspace (same slicing: 192 streams, 2 slices of
    # 32 tokens): per-wave memory partials (2 D*E per slice) and the
    # transposed S1 pair, on top of the E-proportional buffers
    small = lib.atlas_scan_workspace_size(_desc(E=128, B=16, H=12))
    wide = lib.atlas_scan_workspace_size(_desc(E=256, B=16, H=12))
    streams, nsl, D = 16 * 12, 2, 64
    assert wide - small >= 4 * streams * (nsl * 2 * D * 256 + 2 * D * 256)


def test_scan_rejects_null_and_small_workspace(lib):
    d = _desc()
    z = ctypes.c_void_p(0)
    one = ctypes.c_void_p(16)
    st = lib.atlas_scan_fwd(d, z, z, z, z, z, z, z, z, z, z, z, z, z, 0, z)
    assert st == 1 and "NULL" in lib.atlas_last_error().decode()
    st = lib.atlas_scan_fwd(d, *([one] * 7), *([one] * 4), one, one, 8, z)
    assert st == 4 and "workspace" in lib.atlas_last_error().decode()


def test_pe_and_scan_ops_reject_bad_arguments(lib):
    z = ctypes.c_void_p(0)
    assert lib.atlas_pe_batched(-1, 8, 8, 5, 0, z, z, 0, 0, z) == 1
    assert lib.atlas_pe_batched(0, 8, 8, 5, 0, z, z, 0, 0, z) == 0   # empty batch: no work
    assert lib.atlas_pe_batched(4, 8, 8, 9, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 0, z) == 1
    assert lib.atlas_pe_batched(4, 130, 200, 5, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 0, z) == 2
    assert lib.atlas_pe_batched(4, 64, 300, 5, 0, ctypes.c_void_p(16), ctypes.c_void_p(16), 0, 0, z) == 2
    assert lib.atlas_linear_scan(0, 4, 1, 8, z, z, z, z, z, z) == 1
    assert lib.atlas_linear_scan_bwd_workspace_size(2, 16, 3, 512) == 2 * 16 * 3 * 8 * 4
    one = ctypes.c_void_p(16)
    assert lib.atlas_linear_scan_bwd(2, 16, 3, 512, one, one, one, z, z, z, one, one, one, 4096, z) == 1
    assert lib.atlas_linear_scan_bwd(2, 16, 3, 512, one, one, one, z, z, one, one, one, one, 8, z) == 4
    assert lib.atlas_fused_chunk_fwd(1, 8, 1, 32, 32, 5, 0, 0, 0, *([z] * 10), z, 0, z) == 1
    assert lib.atlas_profile_read(9, ctypes.byref(ctypes.c_int64()), ctypes.byref(ctypes.c_double())) == 1


def test_scan_rejects_misaligned_pointers(lib):
    """q/k/v/y and the state are accessed with 16-byte vector loads: offset
    views are refused on the host before anything is launched."""
    d = _desc()
    ws = lib.atlas_scan_workspace_size(d)
    ok = ctypes.c_void_p(1 << 20)
    bad = ctypes.c_void_p((1 << 20) + 8)
    ptrs = [ok] * 7 + [ok] * 4 + [ok]
    for i, word in ((0, "q, k, v and y"), (2, "q, k, v and y"), (7, "W1, W2, S1 and S2"), (10, "W1, W2, S1 and S2"),
                    (11, "q, k, v and y")):
        args = list(ptrs)
        args[i] = bad
        st = lib.atlas_scan_fwd(d, *args, ok, ws, ctypes.c_void_p(0))
        assert st == 1 and word in lib.atlas_last_error().decode(), (i, lib.atlas_last_error())
    st = lib.atlas_scan_fwd(d, *ptrs, bad, ws, ctypes.c_void_p(0))
    assert st == 1 and "workspace" in lib.atlas_last_error().decode()


def test_workspace_does_not_grow_with_sequence_length(lib):
    """The gate tables are held for a window of chunks, so the workspace
    depends on B*H, D, E and the chunk size, not on T (C2 and C4 shapes)."""
    c2 = [lib.atlas_scan_workspace_size(_desc(T=T)) for T in (4096, 65536, 1 << 20)]
    assert c2[0] == c2[1] == c2[2]
    c4 = [lib.atlas_scan_workspace_size(_desc(B=1, H=16, T=T, omega_window=64)) for T in (8192, 131072, 1 << 20)]
    assert c4[0] == c4[1] == c4[2]
    assert c4[0] < 64 << 20


def _bwd_desc(**kw):
    d = dict(B=2, T=128, H=2, D=64, E=128, chunk_size=64, omega_window=32, ns_steps=5, io_dtype=0,
             gate_dtype=0, compute=0, n_slices=0)
    d.update(kw)
    return L.ScanDesc(**d)


def test_scan_bwd_workspace_and_argument_checks(lib):
    """atlas_scan_bwd's host-side checks: supported shapes only, fp32, dense
    strides, T a multiple of the chunk, NULL pointers, workspace size, and
    16-byte alignment (all rejected before any launch)."""
    ok = lib.atlas_scan_bwd_workspace_size(_bwd_desc())
    # trace (one chunk start) + 8 per-token matrices dominate
    BH, DE, cs = 4, 64 * 128, 64
    assert ok >= 4 * (4 * BH * DE + 8 * BH * cs * DE)
    # fp16 operands: no Polar-Express VJP scratch, the same per-token arrays
    f16 = lib.atlas_scan_bwd_workspace_size(_bwd_desc(compute=1))
    assert 4 * (4 * BH * DE + 8 * BH * cs * DE) <= f16 < ok
    # E = 256 in either mode (fp32: the VJP's scratch also holds the iterate and the cotangent)
    w16 = lib.atlas_scan_bwd_workspace_size(_bwd_desc(E=256, compute=1))
    assert w16 > f16 and lib.atlas_scan_bwd_workspace_size(_bwd_desc(E=256)) > w16
    for bad in (dict(E=192), dict(D=48), dict(T=100), dict(io_dtype=1), dict(compute=2), dict(chunk_size=512),
                dict(ns_steps=6)):
        assert lib.atlas_scan_bwd_workspace_size(_bwd_desc(**bad)) == 0, bad
    d = _bwd_desc()
    d2 = _bwd_desc(x_stride_h=128)
    assert lib.atlas_scan_bwd_workspace_size(d2) == 0 and "dense" in lib.atlas_last_error().decode()
    z = ctypes.c_void_p(0)
    one = ctypes.c_void_p(256)
    # q k v alpha eta theta | gamma | W1 W2 S1 S2 | trace | dy dW1 dW2 dS1 dS2 | dq .. dtheta | dgamma | dW1_0 ..
    args = [one] * 6 + [z] + [one] * 4 + [z] + [z] * 5 + [one] * 6 + [z] + [one] * 4
    assert lib.atlas_scan_bwd(d, 0, *args, one, 16, z) == 4
    assert "workspace" in lib.atlas_last_error().decode()
    assert lib.atlas_scan_bwd(d, 0, *([z] * 28), one, ok, z) == 1
    assert lib.atlas_scan_bwd(d, 8, *args, one, ok, z) == 1   # unknown flag bit
    mis = list(args)
    mis[1] = ctypes.c_void_p(260)   # k off by 4 bytes
    assert lib.atlas_scan_bwd(d, 0, *mis, one, ok, z) == 1
    assert "aligned" in lib.atlas_last_error().decode()
    assert lib.atlas_scan_bwd(_bwd_desc(E=192), 0, *args, one, ok, z) == 2
    tr = list(args)
    tr[11] = ctypes.c_void_p(264)   # a misaligned state trace
    assert lib.atlas_scan_bwd(d, 0, *tr, one, ok, z) == 1 and "trace" in lib.atlas_last_error().decode()
    # the forward's trace variant refuses a NULL or misaligned trace
    fd = _bwd_desc(E=256, io_dtype=1, compute=1)
    assert lib.atlas_scan_fwd_trace(fd, *([one] * 7), *([one] * 4), one, z, one, 1 << 30, z) == 1
    assert lib.atlas_scan_fwd_trace(_bwd_desc(), *([one] * 7), *([one] * 4), one, z, one, 1 << 30, z) == 1
    assert lib.atlas_scan_fwd_trace(_bwd_desc(), *([one] * 7), *([one] * 4), one, ctypes.c_void_p(264), one,
                                    1 << 30, z) == 1


def test_pe_vjp_argument_checks(lib):
    """atlas_pe_vjp_batched: compiled shapes (either orientation), workspace,
    compute mode, alignment."""
    z = ctypes.c_void_p(0)
    one = ctypes.c_void_p(256)
    need = lib.atlas_pe_vjp_workspace_size(64, 128, 5)
    assert need > 0 and need == lib.atlas_pe_vjp_workspace_size(128, 64, 5)
    # 64 x 256 in either mode (the fp32 kernel also keeps the iterate and the
    # cotangent in its scratch); 32 x 256 and ns 6: not built
    wide = lib.atlas_pe_vjp_workspace_size(64, 256, 5)
    assert wide > 2 * need and lib.atlas_pe_vjp_workspace_size(64, 128, 6) == 0
    assert lib.atlas_pe_vjp_workspace_size(32, 256, 5) == 0
    assert lib.atlas_pe_vjp_batched(0, 64, 128, 5, z, z, 0, z, 0, z) == 0       # empty batch: no work
    assert lib.atlas_pe_vjp_batched(4, 32, 256, 5, one, one, 0, one, wide, z) == 2
    assert lib.atlas_pe_vjp_batched(4, 64, 256, 5, one, one, 0, one, need, z) == 4   # workspace too small
    assert lib.atlas_pe_vjp_batched(4, 64, 128, 5, one, one, 0, one, 16, z) == 4
    assert lib.atlas_pe_vjp_batched(4, 64, 128, 5, one, one, 3, one, need, z) == 1
    assert lib.atlas_pe_vjp_batched(4, 64, 128, 5, ctypes.c_void_p(260), one, 0, one, need, z) == 1
