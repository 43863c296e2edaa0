"""Producer fusion: RMSNorm and SiLU*mul that also emit the union statistic.

In a Llama-style block the input of qkv_proj and gate_up_proj comes out of an
RMSNorm and the input of down_proj out of SiLU(gate)*up.  These wrappers run
those operations on the GPU (libgrinqh_hip.so: grinqh_rmsnorm_sigma,
grinqh_silu_mul_sigma) and return, next to y, the column maxima of |y| per
chunk of 16 rows; ``gemv_batch_union_sigma`` grades a union product from them
instead of reading x once more for the statistic (grinqh/kernel.py:249 in the
reference computes it inside the GEMV).  No reference counterpart: vLLM's
RMSNorm / SiluAndMul and the reference's op are separate.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _lib
from .kernel import _WORKSPACES, _dtype_code


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


def _chunks(M: int) -> int:
    return (M + _lib.SIGMA_CHUNK_ROWS - 1) // _lib.SIGMA_CHUNK_ROWS


def rmsnorm_sigma(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-5,
                  residual: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, Optional[torch.Tensor]]:
    """``y = RNE(h * rsqrt(mean(h^2) + eps)) * weight`` with ``h = x`` or, given
    ``residual``, ``h = RNE(x + residual)``; returns ``(y, sigma_chunks,
    h or None)``."""
    if not x.is_cuda:
        raise ValueError("GRINQH: x must be on a HIP device; there is no CPU path")
    K = x.shape[-1]
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    w = weight.to(x.dtype).contiguous()
    y = torch.empty_like(x2)
    sig = torch.empty((_chunks(M), K), dtype=torch.float32, device=x.device)
    r_in = r_out = None
    if residual is not None:
        r_in = residual.reshape(-1, K).to(x.dtype).contiguous()
        r_out = torch.empty_like(r_in)
    lib = _lib.load_library()
    _lib.check(lib.grinqh_rmsnorm_sigma(x2.data_ptr(), M, K, K, r_in.data_ptr() if r_in is not None else None,
                                        r_out.data_ptr() if r_out is not None else None, w.data_ptr(), float(eps),
                                        y.data_ptr(), sig.data_ptr(), _dtype_code(x.dtype), _stream(x.device)),
               "grinqh_rmsnorm_sigma")
    return y.view(x.shape), sig, (r_out.view(x.shape) if r_out is not None else None)


def silu_mul_sigma(gate_up: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """``y = RNE(silu(g)) * u`` for ``gate_up = [g | u]`` along the last
    dimension; returns ``(y, sigma_chunks)``."""
    if not gate_up.is_cuda:
        raise ValueError("GRINQH: gate_up must be on a HIP device; there is no CPU path")
    F2 = gate_up.shape[-1]
    if F2 % 2:
        raise ValueError("gate_up must hold [gate | up] halves of equal width")
    F = F2 // 2
    g2 = gate_up.reshape(-1, F2).contiguous()
    M = g2.shape[0]
    y = torch.empty((M, F), dtype=gate_up.dtype, device=gate_up.device)
    sig = torch.empty((_chunks(M), F), dtype=torch.float32, device=gate_up.device)
    lib = _lib.load_library()
    _lib.check(lib.grinqh_silu_mul_sigma(g2.data_ptr(), M, F, F2, y.data_ptr(), sig.data_ptr(),
                                         _dtype_code(gate_up.dtype), _stream(gate_up.device)),
               "grinqh_silu_mul_sigma")
    return y.view(*gate_up.shape[:-1], F), sig


def gemv_batch_union_sigma(x: torch.Tensor, weight_packed: torch.Tensor, weight_scale: torch.Tensor,
                           bias: Optional[torch.Tensor], max_bits: int, group_size: int, original_n: int,
                           thresholds: List[float], sigma_chunks: torch.Tensor) -> torch.Tensor:
    """Union-graded product (grinqh_gemv_batch_union) graded from the
    ``sigma_chunks`` a producer returned for this ``x``."""
    if not x.is_cuda:
        raise ValueError("GRINQH: x must be on a HIP device; there is no CPU path")
    K = x.shape[-1]
    N = 4 * int(original_n)
    x2 = x.reshape(-1, K).contiguous()
    M = x2.shape[0]
    if sigma_chunks.dtype != torch.float32 or tuple(sigma_chunks.shape) != (_chunks(M), K):
        raise ValueError(f"sigma_chunks must be float32 [{_chunks(M)}, {K}], got {tuple(sigma_chunks.shape)}")
    sc = sigma_chunks.contiguous()
    # inputs kept referenced until the call is enqueued (a temporary freed
    # earlier could be handed to y below)
    scale = weight_scale.to(x.dtype).contiguous()
    b = bias.to(x.dtype).contiguous() if bias is not None else None
    wp = weight_packed.contiguous()
    y = torch.empty((M, N), dtype=x.dtype, device=x.device)
    lib = _lib.load_library()
    stream = _stream(x.device)
    nbytes = lib.grinqh_workspace_bytes(M, K, N, max_bits, _lib.MODE_UNION)
    ws = _WORKSPACES.get(x.device, stream, nbytes)
    _lib.check(lib.grinqh_gemv_batch_union_sigma(
        x2.data_ptr(), M, K, K, N, _dtype_code(x.dtype), wp.data_ptr(), scale.data_ptr(),
        b.data_ptr() if b is not None else None,
        y.data_ptr(), max_bits, group_size, _lib.thresholds_f32(thresholds), sc.data_ptr(),
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0, stream),
        "grinqh_gemv_batch_union_sigma")
    return y.view(*x.shape[:-1], N)
