"""CPU checks of the C ABI: libgrinqh_hip.so loads without a GPU, exports every
function include/grinqh.h declares with the documented signature, and rejects
bad arguments before touching the device."""
import ctypes
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "grinqh.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(grinqh_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from grinqh import _lib
    return _lib.load_library()


def test_every_declared_symbol_is_exported_and_typed(lib):
    from grinqh import _lib
    names = _declared()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
        assert n in _lib.SIGNATURES, f"{n} missing from the ctypes binding"
    assert set(_lib.SIGNATURES) == set(names)


def test_version_and_status_strings(lib):
    assert lib.grinqh_abi_version() == 1
    for s in range(4):
        assert lib.grinqh_status_string(s)
    assert lib.grinqh_status_string(99) == b"unknown status"


def test_library_path_honours_environment(monkeypatch):
    from grinqh import _lib
    monkeypatch.setenv("GRINQH_LIB", "/opt/elsewhere/libgrinqh_hip.so")
    assert _lib.library_path() == "/opt/elsewhere/libgrinqh_hip.so"
    monkeypatch.delenv("GRINQH_LIB")
    assert _lib.library_path().endswith("libgrinqh_hip.so")


def test_workspace_query(lib):
    # M=1 o_proj shape: split-K needs one fp32 [M][N] slab per K range.
    ws = lib.grinqh_workspace_bytes(1, 4096, 4096, 8, 0)
    assert ws >= 2 * 4096 * 4 and ws % (4096 * 4) == 0
    assert lib.grinqh_workspace_bytes(0, 4096, 4096, 8, 0) == 0
    # union batches beyond one launch also carry the K-float sigma area
    assert lib.grinqh_workspace_bytes(200, 4096, 4096, 8, 1) >= lib.grinqh_workspace_bytes(200, 4096, 4096, 8, 2)


def test_workspace_query_library_gemm_path(lib):
    """The large-batch prefill path (dequantized weight + library GEMM) sizes
    the workspace for the K-contiguous weight (2*N*K bytes) after the fused
    kernel's regions (the GEMM itself takes no workspace).  The query has no dtype, so it
    covers the path whenever either dtype may take it: from 512 rows, from
    224 in bf16, at 257-511 rows when K <= 8192 or the fused grid would need
    more than one round (gate_up's N); never when N / 16 is not a multiple of
    4; dense and union alike."""
    K = 4096
    dense, union = 2, 1
    library = lambda M, N, mode: lib.grinqh_workspace_bytes(M, K, N, 8, mode) >= 2 * N * K
    for mode in (dense, union):
        assert library(512, 6144, mode) and library(2048, 28672, mode) and library(300, 28672, mode)
        assert library(224, 6144, mode) and not library(223, 6144, mode) and not library(128, 28672, mode)
        assert not library(4096, 4112, mode)
    # the union layout adds sigma, its chunk maxima and the row flags to the dense one
    assert lib.grinqh_workspace_bytes(2048, K, 6144, 8, union) > lib.grinqh_workspace_bytes(2048, K, 6144, 8, dense)
    # the fused kernel's split-K partials stay in front of the library regions
    assert lib.grinqh_workspace_bytes(240, K, 4096, 8, dense) >= 2 * 4096 * K + 8 * 240 * 4096 * 4


def test_invalid_arguments_rejected_on_host(lib):
    from grinqh import _lib
    t = _lib.thresholds_f32([0.0] * 4)
    INVALID = _lib.GRINQH_ERR_INVALID
    base = dict(M=1, K=4096, ldx=4096, N=4096, dt=0, b=8, gs=128, mode=0)

    def call(**kw):
        a = {**base, **kw}
        dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
        return lib.grinqh_gemm_or_gemv(dummy, a["M"], a["K"], a["ldx"], a["N"], a["dt"], dummy, dummy, None,
                                       dummy, a["b"], a["gs"], t, a["mode"], None, 0, None)

    assert call(b=5) == INVALID
    assert call(b=10) == INVALID
    assert call(K=4016, ldx=4016) == INVALID
    assert call(N=4100) == INVALID
    assert call(gs=48) == INVALID
    assert call(dt=7) == INVALID
    assert call(mode=9) == INVALID
    assert call(ldx=4100) == INVALID
    assert call(M=-1) == INVALID
    assert call(M=0) == _lib.GRINQH_OK  # empty batch: nothing to do
    assert call() == _lib.GRINQH_ERR_WORKSPACE  # needs split-K workspace
    assert lib.grinqh_pack_planes(None, None, 4, 20, 8, None) == INVALID
    assert lib.grinqh_unpack_planes(None, None, 1, None, 4, 32, 5, None) == INVALID
    assert lib.grinqh_grade(None, 1, 32, 32, 0, 3, t, None, None, None) == INVALID


def test_activations_beyond_32_bit_offsets_rejected(lib):
    """Kernels that address x through 32-bit buffer offsets refuse an x of
    2 GiB or more instead of reading wrong rows: the fused prefill (taken at
    every batch size when N/16 is not a multiple of 4) for the whole batch,
    the GEMV / decode kernels for the rows of one launch."""
    from grinqh import _lib
    t = _lib.thresholds_f32([0.0] * 4)
    dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    ws = ctypes.c_void_p(1 << 20)

    def call(M, K, ldx, N):
        return lib.grinqh_gemm_or_gemv(dummy, M, K, ldx, N, 0, dummy, dummy, None, dummy, 2, 128, t,
                                       _lib.MODE_DENSE, ws, 1 << 40, None)

    # fused prefill: 2^31 bytes of x (N = 48: N/16 = 3, never the library path)
    assert call(1 << 18, 4096, 4096, 48) == _lib.GRINQH_ERR_INVALID
    # one decode launch: 2 rows of 2^30 halves each
    assert call(2, 32, 1 << 30, 48) == _lib.GRINQH_ERR_INVALID


def test_noalloc_rejects_mode_and_thresholds_before_device_state(lib):
    """The allocation-free entry point validates the mode and, for graded
    products, the thresholds pointer before it looks up or clears its device
    scratch: without a GPU such a call returns GRINQH_ERR_INVALID, not the
    GRINQH_ERR_HIP a device lookup would give."""
    from grinqh import _lib
    t = _lib.thresholds_f32([0.0] * 4)
    dummy = ctypes.c_void_p(4096)  # never dereferenced: validation fails first
    # an untyped handle of the same library, so that a null thresholds pointer can be passed
    fn = ctypes.CDLL(_lib.library_path()).grinqh_gemm_or_gemv_noalloc
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                   ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]

    def call(mode, thr, M=1):
        tp = ctypes.cast(thr, ctypes.c_void_p) if thr is not None else None
        return fn(dummy, M, 4096, 4096, 4096, 0, dummy, dummy, None, dummy, 8, 128, tp, mode, None)

    assert call(9, t) == _lib.GRINQH_ERR_INVALID
    assert call(-1, t) == _lib.GRINQH_ERR_INVALID
    assert call(_lib.MODE_UNION, None) == _lib.GRINQH_ERR_INVALID            # graded: thresholds required
    assert call(_lib.MODE_REFERENCE, None, M=1) == _lib.GRINQH_ERR_INVALID   # one row is graded
    assert call(_lib.MODE_UNION, t, M=0) == _lib.GRINQH_OK                   # empty batch: nothing to do
