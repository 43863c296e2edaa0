"""ctypes binding of libgrinqh_hip.so (C ABI declared in include/grinqh.h).

The library is built in-tree by ``vllm-grinqh-plugin_amd/build.py`` for gfx950.
There is no fallback: if the library or a HIP device is missing, every entry
point raises instead of computing anything on the CPU.
"""
from __future__ import annotations

import ctypes
import os
import threading

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libgrinqh_hip.so")

GRINQH_OK = 0
GRINQH_ERR_INVALID = 1
GRINQH_ERR_HIP = 2
GRINQH_ERR_WORKSPACE = 3
GRINQH_ERR_SCRATCH = 4
NOALLOC_SCRATCH_BYTES = 64 << 20
SIGMA_CHUNK_ROWS = 16

DTYPE_F16 = 0
DTYPE_BF16 = 1

MODE_REFERENCE = 0
MODE_UNION = 1
MODE_DENSE = 2

ABI_VERSION = 1

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f4 = ctypes.c_float * 4

# name -> (restype, argtypes); mirrors include/grinqh.h
SIGNATURES = {
    "grinqh_abi_version": (_i32, []),
    "grinqh_status_string": (ctypes.c_char_p, [_i32]),
    "grinqh_pack_planes": (_i32, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "grinqh_prepare_weight": (_i32, [_vp, _vp, _i64, _i64, _i32, _vp]),
    "grinqh_unpack_planes": (_i32, [_vp, _vp, _i64, _vp, _i64, _i64, _i32, _vp]),
    "grinqh_dequantize": (_i32, [_vp, _vp, _vp, _i64, _i64, _i32, _i32, _i32, _vp]),
    "grinqh_grade": (_i32, [_vp, _i64, _i64, _i64, _i32, _i32, _f4, _vp, _vp, _vp]),
    "grinqh_workspace_bytes": (ctypes.c_size_t, [_i64, _i64, _i64, _i32, _i32]),
    "grinqh_gemm_or_gemv": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _f4, _i32,
                                   _vp, ctypes.c_size_t, _vp]),
    "grinqh_gemv_batch_union": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _f4,
                                       _vp, ctypes.c_size_t, _vp]),
    "grinqh_prefill_dense": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32,
                                    _vp, ctypes.c_size_t, _vp]),
    "grinqh_gemm_or_gemv_noalloc": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32,
                                           _f4, _i32, _vp]),
    "grinqh_rmsnorm_sigma": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_float, _vp, _vp, _i32, _vp]),
    "grinqh_silu_mul_sigma": (_i32, [_vp, _i64, _i64, _i64, _vp, _vp, _i32, _vp]),
    "grinqh_gemv_batch_union_sigma": (_i32, [_vp, _i64, _i64, _i64, _i64, _i32, _vp, _vp, _vp, _vp, _i32, _i32, _f4,
                                             _vp, _vp, ctypes.c_size_t, _vp]),
    "grinqh_time_next_product": (_i32, [_vp, _vp]),
    "grinqh_product_kernel": (_i32, [_i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                     ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
}

KERNEL_GEMV = 1
KERNEL_DECODE = 2
KERNEL_TALL = 3
KERNEL_LIBRARY = 4
KERNEL_FUSED = 5
KERNEL_NAMES = {KERNEL_GEMV: "gemv_kernel", KERNEL_DECODE: "decode_kernel", KERNEL_TALL: "prefill_tall_kernel",
                KERNEL_LIBRARY: "dequant_nk_kernel + library GEMM", KERNEL_FUSED: "prefill_kernel"}


def product_kernel(M: int, K: int, ldx: int, N: int, dtype: int, max_bits: int, group_size: int, mode: int,
                   noalloc: bool = False):
    """(kernel id, rows per block, K ranges of the split tiles) of the kernel
    that serves such a product (grinqh_product_kernel); nothing is launched."""
    lib = load_library()
    rows, sp = _i32(0), _i32(0)
    k = lib.grinqh_product_kernel(M, K, ldx, N, dtype, max_bits, group_size, mode, int(bool(noalloc)),
                                  ctypes.byref(rows), ctypes.byref(sp))
    if k < 0:
        check(-k, "grinqh_product_kernel")
    return k, rows.value, sp.value

_lock = threading.Lock()
_lib = None


def library_path() -> str:
    """The in-tree build, or the library named by the GRINQH_LIB environment variable."""
    return os.environ.get("GRINQH_LIB") or _LIB_PATH


def load_library(path: str | None = None) -> ctypes.CDLL:
    """Load (once) and type the C ABI.  Loading needs no GPU."""
    global _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = path or library_path()
        if not os.path.exists(p):
            raise RuntimeError(
                f"GRINQH HIP library not found at {p}; build it with "
                "`python vllm-grinqh-plugin_amd/build.py` (hipcc, gfx950)")
        lib = ctypes.CDLL(p)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.grinqh_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"libgrinqh_hip.so ABI version {ver}, expected {ABI_VERSION}; rebuild it")
        if path is None:
            _lib = lib
        return lib


def check(status: int, what: str) -> None:
    """Turn a non-zero C status into the Python exception the reference raises
    for the same class of error (ValueError for bad arguments)."""
    if status == GRINQH_OK:
        return
    msg = f"{what}: {load_library().grinqh_status_string(status).decode()} (status {status})"
    if status in (GRINQH_ERR_INVALID, GRINQH_ERR_WORKSPACE, GRINQH_ERR_SCRATCH):
        raise ValueError(msg)
    raise RuntimeError(msg)


def thresholds_f32(thresholds) -> ctypes.Array:
    """Thresholds as the reference kernel compares them: zero padded/truncated
    to 4 (grinqh/grinqh.py:111) and rounded to fp32 (Triton promotes the
    constexpr float to fp32 before comparing, grinqh/kernel.py:100-106)."""
    t = [float(v) for v in list(thresholds)] + [0.0] * 4
    return _f4(*t[:4])
