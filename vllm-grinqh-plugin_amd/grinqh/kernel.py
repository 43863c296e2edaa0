"""``torch.ops.grinqh.gemm_or_gemv`` on gfx950 kernels.

Same op name, schema and dispatch contract as the reference
(grinqh/kernel.py:646-725): pure function of its inputs, output on ``x.device``
in ``x.dtype`` with shape ``x.shape[:-1] + (4*original_n,)``, enqueued on the
current stream without a host synchronisation (graph capturable).  The work is
done by libgrinqh_hip.so through its C ABI; there is no CPU implementation.

Batch grading (``GRINQH_BATCH_GRADING``, read once at import like the
reference's ``GRINQH_*`` tuning variables, grinqh/kernel.py:590-604):

* ``reference`` (default): one row -> graded GEMV (grinqh/kernel.py:681-706),
  more rows -> dense dequantize-then-matmul, thresholds ignored
  (grinqh/kernel.py:663-680).
* ``union``: every batch is graded on ``sigma_k = max_m |x[m,k]|``, the rule of
  grinqh_gemv_batch_union (grinqh/kernel.py:170-360, 607-643).

``use_marlin`` is accepted for schema compatibility and ignored: the build has
one kernel family and no backend dispatch.
"""
from __future__ import annotations

import os
import threading
from typing import List, Optional

import torch

from . import _lib

_BATCH_GRADING = os.environ.get("GRINQH_BATCH_GRADING", "reference").strip().lower()
if _BATCH_GRADING not in ("reference", "union"):
    raise ValueError(f"GRINQH_BATCH_GRADING must be 'reference' or 'union', got {_BATCH_GRADING!r}")

_MODES = {"reference": _lib.MODE_REFERENCE, "union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}


def batch_grading_mode() -> str:
    return _BATCH_GRADING


def set_batch_grading_mode(mode: str) -> None:
    """Set the op's batch grading mode ("reference" or "union") for the calls
    that follow, as GRINQH_BATCH_GRADING does at import.  A HIP graph keeps
    the mode it was captured with."""
    global _BATCH_GRADING
    mode = mode.strip().lower()
    if mode not in ("reference", "union"):
        raise ValueError(f"batch grading mode must be 'reference' or 'union', got {mode!r}")
    _BATCH_GRADING = mode


def _stream_capturing(device: torch.device) -> bool:
    return device.type == "cuda" and torch.cuda.is_current_stream_capturing()


class _Workspaces:
    """Per (device, stream) workspace: split-K counters and partial sums.

    Grown on demand and zero-filled when allocated (the library keeps its
    counters zero between calls).  Calls on one stream are ordered, so they
    may share it; different streams get different buffers.

    Sizes grow in powers of two (at least 1 MiB), so a caller whose batches
    keep growing reallocates O(log size) times.  An outgrown buffer is
    dropped (returned to the allocator) unless a HIP graph was captured while
    it was current: such a graph keeps its address and writes into it on
    every replay, so freeing it would let those replays overwrite whatever
    tensor is placed there next.  Those buffers alone are retired and kept
    alive; their counters are still zero (every call leaves them so), so such
    a replay stays correct.  With power-of-two growth the retired bytes of
    one (device, stream) stay below the size of its current buffer."""

    def __init__(self, capturing=_stream_capturing):
        self._bufs = {}        # key -> [buffer, captured while current]
        self._retired = []
        self._lock = threading.Lock()
        self._capturing = capturing

    @staticmethod
    def _size_for(nbytes: int) -> int:
        return max(1 << 20, 1 << (int(nbytes) - 1).bit_length())

    def get(self, device: torch.device, stream: int, nbytes: int) -> torch.Tensor | None:
        if nbytes == 0:
            return None
        key = (device.type, device.index, stream)
        capturing = self._capturing(device)
        with self._lock:
            entry = self._bufs.get(key)
            if entry is None or entry[0].numel() < nbytes:
                if capturing:
                    raise RuntimeError(
                        "GRINQH: workspace must be allocated before graph capture; run the largest "
                        "batch once eagerly first")
                if entry is not None and entry[1]:
                    self._retired.append(entry[0])
                entry = [torch.zeros(self._size_for(nbytes), dtype=torch.uint8, device=device), False]
                self._bufs[key] = entry
            if capturing:
                entry[1] = True
            return entry[0]

    def retired_bytes(self) -> int:
        """Bytes held by outgrown workspaces (kept alive for captured graphs)."""
        with self._lock:
            return sum(b.numel() for b in self._retired)


_WORKSPACES = _Workspaces()


def _dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float16:
        return _lib.DTYPE_F16
    if dtype == torch.bfloat16:
        return _lib.DTYPE_BF16
    raise ValueError(f"GRINQH supports float16 and bfloat16 activations, got {dtype}")


def run_product(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                bias: Optional[torch.Tensor], max_bits: int, group_size: int, original_n: int,
                thresholds: List[float], mode: str) -> torch.Tensor:
    """Shared host path of every product entry point."""
    if not x.is_cuda:
        raise ValueError(f"GRINQH: x must be on a HIP device (got {x.device}); there is no CPU path")
    dt = _dtype_code(x.dtype)
    K = x.shape[-1]
    N = 4 * int(original_n)
    x2 = x.reshape(-1, K)
    if x2.stride(-1) != 1 or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16 != 0:
        x2 = x2.contiguous()
    M = x2.shape[0]
    Z = max_bits // 2
    if weight_packed.shape[0] != K or weight_packed.shape[1] * weight_packed.element_size() != Z * (N // 16) * 4:
        raise ValueError(f"GRINQH: weight_packed shape {tuple(weight_packed.shape)} does not match "
                         f"K={K}, N={N}, max_bits={max_bits}")
    if weight_packed.device != x.device:
        raise ValueError("GRINQH: weight_packed and x are on different devices")
    scale = weight_scale if weight_scale.dtype == x.dtype else weight_scale.to(x.dtype)
    scale = scale.contiguous()
    if scale.shape[0] * group_size < K or scale.shape[1] != N:
        raise ValueError(f"GRINQH: weight_scale shape {tuple(weight_scale.shape)} does not cover K={K}, N={N}")
    bp = None
    if bias is not None:
        b = bias if bias.dtype == x.dtype else bias.to(x.dtype)
        b = b.contiguous()
        if b.numel() != N:
            raise ValueError(f"GRINQH: bias has {b.numel()} elements, expected {N}")
        bp = b.data_ptr()
    wp = weight_packed.contiguous()
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    lib = _lib.load_library()
    mode_code = _MODES[mode]
    stream = torch.cuda.current_stream(x.device).cuda_stream
    nbytes = lib.grinqh_workspace_bytes(M, K, N, max_bits, mode_code)
    ws = _WORKSPACES.get(x.device, stream, nbytes)
    _lib.check(lib.grinqh_gemm_or_gemv(
        x2.data_ptr(), M, K, x2.stride(0), N, dt, wp.data_ptr(), scale.data_ptr(), bp, y.data_ptr(),
        max_bits, group_size, _lib.thresholds_f32(thresholds), mode_code,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, stream),
        "grinqh_gemm_or_gemv")
    return y.view(*x.shape[:-1], N)


@torch.library.custom_op("grinqh::gemm_or_gemv", mutates_args=())
def grinqh_gemm_or_gemv(
        x: torch.Tensor,
        weight_packed: torch.Tensor,
        weight_scale: torch.Tensor,
        bias: Optional[torch.Tensor],
        max_bits: int,
        group_size: int,
        original_n: int,
        thresholds: List[float],
        use_marlin: bool = False
) -> torch.Tensor:
    """Quantized linear (reference grinqh/kernel.py:646-710)."""
    return run_product(x, weight_packed, weight_scale, bias, max_bits, group_size, original_n, thresholds,
                       _BATCH_GRADING)


@grinqh_gemm_or_gemv.register_fake
def _fake(x, weight_packed, weight_scale, bias, max_bits, group_size, original_n, thresholds, use_marlin=False):
    return torch.empty(x.shape[:-1] + (original_n * 4,), device=x.device, dtype=x.dtype)


def grinqh_gemv_batch_union(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                            bias: Optional[torch.Tensor], max_bits: int, group_size: int, original_n: int,
                            thresholds: List[float]) -> torch.Tensor:
    """Batch-union GEMV (reference grinqh/kernel.py:607-643)."""
    return run_product(x, weight_packed, weight_scale, bias, max_bits, group_size, original_n, thresholds, "union")


def grinqh_prefill_dense(x_flat: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                         group_size: int, original_n: int, max_bits: int) -> torch.Tensor:
    """Dense dequantize-then-matmul for any row count, thresholds ignored
    (reference grinqh_prefill_gemm_compiled, grinqh/kernel.py:561-587; same
    argument order)."""
    return run_product(x_flat, weight_packed, weight_scale, None, max_bits, group_size, original_n,
                       [0.0] * 4, "dense")
