"""ctypes binding of libatlas_hip.so (the C ABI in include/atlas_scan.h).

The library is loaded from atlas_amd/_lib/ (built in-tree by atlas_amd.build).
torch is imported first so that the HIP runtime torch ships with is the one
the library binds to (both use the soname libamdhip64.so.7).  There is no
fallback: if the library is missing, get_lib() raises.
"""

import ctypes
import os
import re

import torch  # noqa: F401  (loads the HIP runtime before the library)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libatlas_hip.so")
HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__)))),
                      "include", "atlas_scan.h")

ATLAS_OK = 0
STATUS_NAMES = {0: "ATLAS_OK", 1: "ATLAS_ERR_INVALID_ARGUMENT", 2: "ATLAS_ERR_UNSUPPORTED_SHAPE",
                3: "ATLAS_ERR_HIP", 4: "ATLAS_ERR_WORKSPACE"}
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
COMPUTE_F32, COMPUTE_F16 = 0, 1
PE_NORM_EPS, PE_NORM_NO_EPS = 0, 1


class ScanDesc(ctypes.Structure):
    """Mirror of atlas_scan_desc."""
    _fields_ = [
        ("B", ctypes.c_int32), ("T", ctypes.c_int32), ("H", ctypes.c_int32),
        ("D", ctypes.c_int32), ("E", ctypes.c_int32),
        ("chunk_size", ctypes.c_int32), ("omega_window", ctypes.c_int32),
        ("ns_steps", ctypes.c_int32), ("io_dtype", ctypes.c_int32),
        ("gate_dtype", ctypes.c_int32), ("compute", ctypes.c_int32),
        ("n_slices", ctypes.c_int32),
        ("x_stride_b", ctypes.c_int64), ("x_stride_t", ctypes.c_int64), ("x_stride_h", ctypes.c_int64),
        ("g_stride_b", ctypes.c_int64), ("g_stride_t", ctypes.c_int64),
    ]


class AtlasError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status


_lib = None
_P = ctypes.c_void_p


def _declare(lib):
    i32, i64, sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t
    fp = ctypes.POINTER(ctypes.c_float)
    lib.atlas_abi_version.restype = i32
    lib.atlas_abi_version.argtypes = []
    lib.atlas_last_error.restype = ctypes.c_char_p
    lib.atlas_last_error.argtypes = []
    lib.atlas_scan_workspace_size.restype = sz
    lib.atlas_scan_workspace_size.argtypes = [ctypes.POINTER(ScanDesc)]
    lib.atlas_scan_fwd.restype = ctypes.c_int
    lib.atlas_scan_fwd.argtypes = [ctypes.POINTER(ScanDesc)] + [_P] * 7 + [_P] * 4 + [_P, _P, sz, _P]
    lib.atlas_scan_noalloc_scratch_bytes.restype = sz
    lib.atlas_scan_noalloc_scratch_bytes.argtypes = []
    lib.atlas_scan_fwd_noalloc.restype = ctypes.c_int
    lib.atlas_scan_fwd_noalloc.argtypes = [ctypes.POINTER(ScanDesc)] + [_P] * 7 + [_P] * 4 + [_P, _P]
    lib.atlas_fused_chunk_workspace_size.restype = sz
    lib.atlas_fused_chunk_workspace_size.argtypes = [i32] * 5
    lib.atlas_fused_chunk_fwd.restype = ctypes.c_int
    lib.atlas_fused_chunk_fwd.argtypes = [i32] * 9 + [_P] * 4 + [_P] * 5 + [_P, _P, sz, _P]
    lib.atlas_pe_batched.restype = ctypes.c_int
    lib.atlas_pe_batched.argtypes = [i64, i32, i32, i32, i32, _P, _P, i32, i32, _P]
    lib.atlas_profile_enable.restype = ctypes.c_int
    lib.atlas_profile_enable.argtypes = [i32]
    lib.atlas_profile_read.restype = ctypes.c_int
    lib.atlas_profile_read.argtypes = [i32, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_double)]
    lib.atlas_profile_mfma_rate.restype = ctypes.c_int
    lib.atlas_profile_mfma_rate.argtypes = [i32, ctypes.POINTER(ctypes.c_double), _P]
    lib.atlas_layer_prologue.restype = ctypes.c_int
    lib.atlas_layer_prologue.argtypes = ([i32] * 8 + [_P, i64, i32] + [_P] * 4 + [ctypes.c_float] +
                                         [_P] * 3 + [i32] + [_P, _P, _P])
    lib.atlas_layer_prologue_bwd_workspace_size.restype = sz
    lib.atlas_layer_prologue_bwd_workspace_size.argtypes = [i32] * 7
    lib.atlas_layer_prologue_bwd.restype = ctypes.c_int
    lib.atlas_layer_prologue_bwd.argtypes = ([i32] * 8 + [_P, i64, i32] + [_P] * 4 + [ctypes.c_float] +
                                             [_P] * 3 + [i32] + [_P, _P, _P, i64] + [_P] * 4 + [_P, sz, _P])
    lib.atlas_linear_scan_bwd_workspace_size.restype = sz
    lib.atlas_linear_scan_bwd_workspace_size.argtypes = [i32, i32, i32, i64]
    lib.atlas_linear_scan_bwd.restype = ctypes.c_int
    lib.atlas_linear_scan_bwd.argtypes = [i32, i32, i32, i64] + [_P] * 9 + [sz, _P]
    lib.atlas_swa_fwd.restype = ctypes.c_int
    lib.atlas_swa_fwd.argtypes = [i32] * 5 + [_P] * 4 + [i64] * 3 + [i32, _P, _P, _P]
    lib.atlas_swa_fwd_lse.restype = ctypes.c_int
    lib.atlas_swa_fwd_lse.argtypes = [i32] * 5 + [_P] * 4 + [i64] * 3 + [i32, _P, _P, _P, _P]
    lib.atlas_swa_bwd_workspace_size.restype = sz
    lib.atlas_swa_bwd_workspace_size.argtypes = [i32] * 3
    lib.atlas_swa_bwd.restype = ctypes.c_int
    lib.atlas_swa_bwd.argtypes = [i32] * 5 + [_P] * 6 + [i64] * 3 + [i32, _P, _P, _P, _P, _P, _P, sz, _P]
    lib.atlas_scan_bwd_workspace_size.restype = sz
    lib.atlas_scan_bwd_workspace_size.argtypes = [ctypes.POINTER(ScanDesc)]
    lib.atlas_scan_bwd.restype = ctypes.c_int
    lib.atlas_scan_bwd.argtypes = [ctypes.POINTER(ScanDesc), i32] + [_P] * 7 + [_P] * 4 + [_P] + [_P] * 5 + \
        [_P] * 7 + [_P] * 4 + [_P, sz, _P]
    lib.atlas_pe_vjp_workspace_size.restype = sz
    lib.atlas_pe_vjp_workspace_size.argtypes = [i32, i32, i32]
    lib.atlas_pe_vjp_batched.restype = ctypes.c_int
    lib.atlas_pe_vjp_batched.argtypes = [i64, i32, i32, i32, _P, _P, i32, _P, sz, _P]
    lib.atlas_scan_fwd_trace.restype = ctypes.c_int
    lib.atlas_scan_fwd_trace.argtypes = [ctypes.POINTER(ScanDesc)] + [_P] * 7 + [_P] * 4 + [_P, _P, _P, sz, _P]
    lib.atlas_linear_scan.restype = ctypes.c_int
    lib.atlas_linear_scan.argtypes = [i32, i32, i32, i64, _P, _P, _P, _P, _P, _P]
    del fp
    return lib


def get_lib():
    """Load (once) and return the ctypes handle; raises if the library is absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH} missing (run `python -m atlas_amd.build` "
                "or __graft_entry__.build()); there is no CPU fallback")
        _lib = _declare(ctypes.CDLL(LIB_PATH))
    return _lib


def header_symbols(path=HEADER):
    """Names of the functions declared in include/atlas_scan.h."""
    text = open(path).read()
    return sorted(set(re.findall(r"\b(atlas_[a-z_]+)\s*\(", text)))


def check(status):
    if status != ATLAS_OK:
        msg = get_lib().atlas_last_error().decode(errors="replace")
        raise AtlasError(status, msg)


def dtype_code(t):
    if t == torch.float32:
        return DTYPE_F32
    if t == torch.bfloat16:
        return DTYPE_BF16
    if t == torch.float16:
        return DTYPE_F16
    raise TypeError(f"unsupported dtype {t}")


def stream_ptr(device=None):
    """hipStream_t of torch's current stream on `device`, as a void*."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def profile_read(kind):
    """(launches, total_ms) recorded for one kernel kind since profiling was enabled."""
    n, ms = ctypes.c_int64(), ctypes.c_double()
    check(get_lib().atlas_profile_read(kind, ctypes.byref(n), ctypes.byref(ms)))
    return n.value, ms.value


def mfma_rate(waves_per_simd=1, device=None):
    """Sustained dense fp16 matrix-core rate (TFLOP/s) with pseudo-random
    operands on every CU (atlas_profile_mfma_rate; synchronises)."""
    v = ctypes.c_double()
    check(get_lib().atlas_profile_mfma_rate(waves_per_simd, ctypes.byref(v), stream_ptr(device)))
    return v.value


def ptr(t):
    return ctypes.c_void_p(0 if t is None else t.data_ptr())
