"""Layout utilities of the GRINQH plugin, MI355X build.

Mirrors grinqh/utils.py of the reference: the preshuffle view permutation,
``BitLevel``, and the plane pack / unpack, which here run as gfx950 kernels of
libgrinqh_hip.so instead of Triton.
"""
from __future__ import annotations

from enum import Enum
from typing import Union

import torch

from . import _lib


def grinqh_input_preshuffle(weight: torch.Tensor) -> torch.Tensor:
    """``P[k, 16c + r] = W[k, r*(N/16) + c]`` (reference grinqh/utils.py:17-22)."""
    M, N = weight.shape
    assert N % 16 == 0, "N must be divisible by 16 for this layout."
    return weight.view(M, 16, N // 16).transpose(1, 2).contiguous().view(M, N)


def grinqh_input_postshuffle(weight: torch.Tensor) -> torch.Tensor:
    """Inverse of the preshuffle (reference grinqh/utils.py:25-30)."""
    M, N = weight.shape
    assert N % 16 == 0, "N must be divisible by 16 for this layout."
    return weight.view(M, N // 16, 16).transpose(1, 2).contiguous().view(M, N)


class BitLevel(Enum):
    """Plane count <-> bit width (reference grinqh/utils.py:33-37)."""
    TWO_BIT = 1
    FOUR_BIT = 2
    SIX_BIT = 3
    EIGHT_BIT = 4


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"GRINQH: {name} must be a HIP device tensor (got {t.device}); there is no CPU path")


def pack_planes(A: torch.Tensor, max_bits: int = 8) -> torch.Tensor:
    """Plane pack of already preshuffled + shifted codes.

    Replaces ``pack_triton`` (reference grinqh/utils.py:125-146): ``A`` is a
    uint8 ``[K, N]`` or its uint32 view ``[K, N/4]``; returns uint32
    ``[K, (max_bits/2) * N/16]``.
    """
    _require_gpu(A, "A")
    if A.dtype not in (torch.uint8, torch.uint32, torch.int32):
        raise ValueError("GRINQH pack expects uint8 or uint32 codes")
    A = A.contiguous()
    K = A.shape[0]
    N = A.shape[1] * A.element_size()
    out = torch.empty((K, (max_bits // 2) * (N // 16)), device=A.device, dtype=torch.uint32)
    _lib.check(_lib.load_library().grinqh_pack_planes(A.data_ptr(), out.data_ptr(), K, N, max_bits,
                                                      _stream(A.device)), "grinqh_pack_planes")
    return out


def prepare_weight(w_int8: torch.Tensor, max_bits: int = 8) -> torch.Tensor:
    """Load-time repack of a logical int8 ``W[K, N]`` (preshuffle, shift, plane
    pack in one kernel): the data path of process_weights_after_loading
    (reference grinqh/grinqh.py:200-210)."""
    _require_gpu(w_int8, "weight")
    w = w_int8.contiguous().view(torch.int8)
    K, N = w.shape
    if N % 16 != 0:
        raise AssertionError("N must be divisible by 16 for this layout.")
    out = torch.empty((K, (max_bits // 2) * (N // 16)), device=w.device, dtype=torch.uint32)
    _lib.check(_lib.load_library().grinqh_prepare_weight(w.data_ptr(), out.data_ptr(), K, N, max_bits,
                                                         _stream(w.device)), "grinqh_prepare_weight")
    return out


def unpack_planes(B: torch.Tensor, row: Union[int, torch.Tensor], bit_level: BitLevel,
                  original_n: int) -> torch.Tensor:
    """Unsigned codes of selected rows in preshuffled order, uint32
    ``[rows, original_n]`` (bytes = ``U >> (8-b)``).  Replaces ``unpack_pyt`` /
    ``unpack_triton`` (reference grinqh/utils.py:149-223)."""
    _require_gpu(B, "B")
    if isinstance(row, int):
        rows = torch.tensor([row], device=B.device, dtype=torch.int64)
    else:
        rows = row.to(device=B.device, dtype=torch.int64).reshape(-1).contiguous()
    N = original_n * 4
    if rows.numel() and (int(rows.min()) < 0 or int(rows.max()) >= B.shape[0]):
        raise IndexError(f"GRINQH unpack: row index out of range [0, {B.shape[0]})")
    out = torch.empty((rows.numel(), original_n), device=B.device, dtype=torch.uint32)
    Bc = B.contiguous()
    _lib.check(_lib.load_library().grinqh_unpack_planes(Bc.data_ptr(), rows.data_ptr(), rows.numel(),
                                                        out.data_ptr(), Bc.shape[0], N, int(bit_level.value),
                                                        _stream(B.device)), "grinqh_unpack_planes")
    return out


def dequantize(weight_packed: torch.Tensor, weight_scale: torch.Tensor | None, max_bits: int, group_size: int,
               original_n: int, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """``W * scale`` rounded in ``dtype`` (or the int8 ``W`` when
    ``weight_scale`` is None) in logical column order: the dequantisation of
    grinqh_prefill_gemm_compiled (reference grinqh/kernel.py:568-586)."""
    _require_gpu(weight_packed, "weight_packed")
    K = weight_packed.shape[0]
    N = original_n * 4
    if weight_scale is None:
        out = torch.empty((K, N), device=weight_packed.device, dtype=torch.int8)
        sp, dt = None, _lib.DTYPE_F16
    else:
        dtype = weight_scale.dtype
        out = torch.empty((K, N), device=weight_packed.device, dtype=dtype)
        sp = weight_scale.contiguous().data_ptr()
        dt = _lib.DTYPE_BF16 if dtype == torch.bfloat16 else _lib.DTYPE_F16
    _lib.check(_lib.load_library().grinqh_dequantize(weight_packed.contiguous().data_ptr(), sp, out.data_ptr(), K, N,
                                                     max_bits, group_size, dt, _stream(weight_packed.device)),
               "grinqh_dequantize")
    return out


def grade(x: torch.Tensor, thresholds, max_bits: int):
    """Zone bits (uint8, bit z = zone z active) and midpoint bias (int32) of
    every weight row for ``sigma_k = max_m |x[m, k]|``: the inline grading of
    the reference GEMVs (grinqh/kernel.py:98-114, 249-289), exported."""
    _require_gpu(x, "x")
    x2 = x.reshape(-1, x.shape[-1]).contiguous()
    M, K = x2.shape
    bits = torch.empty(K, device=x.device, dtype=torch.uint8)
    beta = torch.empty(K, device=x.device, dtype=torch.int32)
    dt = _lib.DTYPE_BF16 if x.dtype == torch.bfloat16 else _lib.DTYPE_F16
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("GRINQH activations must be float16 or bfloat16")
    _lib.check(_lib.load_library().grinqh_grade(x2.data_ptr(), M, K, K, dt, max_bits,
                                                _lib.thresholds_f32(thresholds), bits.data_ptr(),
                                                beta.data_ptr(), _stream(x.device)), "grinqh_grade")
    return bits, beta
