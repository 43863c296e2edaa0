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


def test_workspace_query_library_gemm_path(lib, monkeypatch):
    """A prefill takes the library path (the dense weight, 2*N*K bytes, in
    the workspace) where the dispatch prefers it -- from 513 rows, and at
    512 rows and below for weights under 2^25 elements -- and the library has
    an algorithm for the shape (from 512 rows, from 224 in bf16); the
    large-batch kernel where it applies otherwise (K % 64 == 0,
    N % 128 == 0, from 256 rows: no dense weight, only the split-K counters,
    the statistic, the partial sums of the tiles split over K and the
    activations repacked in MFMA fragment order, 2 bytes per element with
    rows rounded up to 16); the fused kernel, whose partial sums the layout
    also covers, for the rest.  GRINQH_PREFILL=tall or =library forces
    either."""
    dense, union = 2, 1
    q = lambda M, K, N, mode: lib.grinqh_workspace_bytes(M, K, N, 8, mode)
    for mode in (dense, union):
        head = 16384 + (0 if mode == dense else 4096 * 4)
        # the library path by default: the dense weight
        assert q(2048, 4096, 28672, mode) >= 2 * 28672 * 4096
        assert q(1024, 4096, 6144, mode) >= 2 * 6144 * 4096
        assert q(512, 4096, 6144, mode) >= 2 * 6144 * 4096   # qkv: under 2^25 elements
        # gate_up x 512 (2^26.8 elements): the large-batch kernel, 224 tiles
        # of 512 x 128 in one round, x repacked
        assert q(512, 4096, 28672, mode) == head + 512 * 4096 * 2
        # shapes the library has no algorithm for (fewer than 512 rows in fp16
        # and 224 in bf16) take the large-batch kernel from 256 rows
        assert q(256, 4096, 6144, mode) < 2 * 6144 * 4096
        # K % 64 == 32 or N % 128 == 64: the library path's dense weight
        assert q(512, 4128, 6144, mode) >= 2 * 6144 * 4128
        assert q(2048, 4096, 4160, mode) >= 2 * 4160 * 4096
        assert q(224, 4128, 6144, mode) >= 2 * 6144 * 4128 and q(223, 4128, 6144, mode) < 2 * 6144 * 4128
        assert q(4096, 4128, 4112, mode) < 2 * 4112 * 4128
    monkeypatch.setenv("GRINQH_PREFILL", "tall")
    for mode in (dense, union):
        head = 16384 + (0 if mode == dense else 4096 * 4)
        # gate_up x 2048: 896 tiles of 512 x 128, the last 128 in two K ranges
        # (partial sums: 128 tiles x 2 ranges x 256 KiB), then x repacked
        assert q(2048, 4096, 28672, mode) == head + 128 * 2 * 512 * 128 * 4 + 2048 * 4096 * 2
        assert q(2040, 4096, 28672, mode) == q(2048, 4096, 28672, mode)
    # a K split of the large-batch kernel (two 128-column tiles at 512 rows)
    assert q(512, 4096, 256, dense) >= 2 * 512 * 256 * 4
    monkeypatch.setenv("GRINQH_PREFILL", "library")
    assert q(512, 4096, 28672, dense) >= 2 * 28672 * 4096
    # the union layout adds the statistic to the dense one
    assert q(2048, 4096, 6144, union) > q(2048, 4096, 6144, dense)


def test_product_kernel_query(lib, monkeypatch):
    """grinqh_product_kernel names the kernel each row count and shape takes,
    without a GPU: GEMV to 4 rows, decode to 64, the fused prefill below 256
    rows (below 129 for weights of at least 192 blocks of 128 columns), the
    library GEMM or the large-batch kernel above as the dispatch prefers, the large-batch kernel without a workspace (where its repacked
    activations fit the fixed scratch), the fused kernel where neither
    fits."""
    from grinqh import _lib
    f = lambda M, K, N, mode=_lib.MODE_DENSE, noalloc=False, gs=128: _lib.product_kernel(
        M, K, K, N, _lib.DTYPE_F16, 8, gs, mode, noalloc)
    assert f(1, 4096, 4096)[0] == _lib.KERNEL_GEMV
    assert f(64, 4096, 4096)[0] == _lib.KERNEL_DECODE
    assert f(200, 4096, 4096)[0] == _lib.KERNEL_FUSED
    assert f(128, 4096, 28672)[0] == _lib.KERNEL_FUSED
    assert f(129, 4096, 28672)[0] == _lib.KERNEL_TALL           # gate_up: one round of whole tiles
    assert f(255, 14336, 4096)[0] == _lib.KERNEL_FUSED          # down
    assert f(2048, 4096, 28672)[0] == _lib.KERNEL_LIBRARY
    assert f(512, 4096, 6144)[0] == _lib.KERNEL_LIBRARY
    assert f(512, 4096, 28672) == (_lib.KERNEL_TALL, 512, 1)
    assert f(512, 14336, 4096)[0] == _lib.KERNEL_TALL           # down
    assert f(256, 4096, 6144)[0] == _lib.KERNEL_TALL            # no library algorithm in fp16
    # without a workspace: no room for the partial sums of the split tiles
    assert f(2048, 4096, 28672, _lib.MODE_UNION, noalloc=True) == (_lib.KERNEL_TALL, 512, 1)
    assert f(4096, 4096, 4112, noalloc=True)[0] == _lib.KERNEL_FUSED
    # ... and the repacked activations must fit the fixed scratch
    assert f(8192, 4096, 4096, noalloc=True)[0] == _lib.KERNEL_FUSED
    assert f(4096, 4096, 4096, noalloc=True)[0] == _lib.KERNEL_TALL
    monkeypatch.setenv("GRINQH_PREFILL", "tall")
    # 896 tiles: three full rounds whole, the last 128 tiles in two K ranges
    assert f(2048, 4096, 28672) == (_lib.KERNEL_TALL, 512, 2)
    assert f(8192, 4096, 28672) == (_lib.KERNEL_TALL, 512, 1)  # 3584 tiles: 14 full rounds
    assert f(512, 4096, 256)[0] == _lib.KERNEL_TALL and f(512, 4096, 256)[2] > 1
    assert f(512, 4096, 2048, gs=32)[0] == _lib.KERNEL_FUSED
    monkeypatch.setenv("GRINQH_PREFILL", "library")
    assert f(512, 4096, 28672)[0] == _lib.KERNEL_LIBRARY
    with pytest.raises(ValueError):
        f(512, 4016, 4096)  # K % 32 != 0


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
