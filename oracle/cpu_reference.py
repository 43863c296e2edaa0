"""The reference's pure-PyTorch math, restated for the CPU, as the timed CPU
baseline of bench.py.

TEST / MEASUREMENT INFRASTRUCTURE ONLY: imported by bench.py's cpu_baseline
leg (and tests), never by the product.  It works from the same packed planes
the GPU kernels read, with torch CPU ops:

* ``dense_prefill``: grinqh_prefill_gemm_compiled (grinqh/kernel.py:561-587) --
  unpack every plane the way ``unpack_pyt`` does (grinqh/utils.py:149-177),
  sign-extend, postshuffle (utils.py:25-30), multiply by the group scale in the
  activation dtype, then ``x @ W``.
* ``graded``: the reference test oracle's masked effective weights
  (tests/test_grinqh_ops.py:28-55) with the batch-union statistic
  (grinqh/kernel.py:249) and an fp32 matmul (tests/test_grinqh_ops.py:221, 276).
"""
from __future__ import annotations

import torch

_SHIFTS = torch.tensor([6, 4, 2, 0], dtype=torch.int32)


def unpack_codes(planes: torch.Tensor, max_bits: int) -> torch.Tensor:
    """``unpack_pyt`` over all rows -> uint8 codes ``[K, N]`` in preshuffled order."""
    K = planes.shape[0]
    Z = max_bits // 2
    nz = planes.shape[1] // Z
    pz = planes.view(torch.int32).reshape(K, Z, nz)
    bits = (pz.unsqueeze(-1) >> _SHIFTS) & 0x03030303
    merge = (torch.arange(Z, dtype=torch.int32) * 2).flip(0).view(1, Z, 1, 1)
    res = (bits << merge).sum(dim=1, dtype=torch.int32)
    return res.reshape(K, nz * 4).view(torch.uint8)


def weight_int8(planes: torch.Tensor, max_bits: int) -> torch.Tensor:
    """Sign-extended, postshuffled int8 ``W[K, N]`` (grinqh/kernel.py:568-576)."""
    sh = 8 - max_bits
    w = (unpack_codes(planes, max_bits).view(torch.int8) << sh) >> sh
    K, N = w.shape
    return w.view(K, N // 16, 16).transpose(1, 2).contiguous().view(K, N)


def dense_prefill(x: torch.Tensor, planes: torch.Tensor, scale: torch.Tensor, group_size: int,
                  max_bits: int) -> torch.Tensor:
    w = weight_int8(planes, max_bits)
    K, N = w.shape
    ws = (w.view(K // group_size, group_size, N).to(x.dtype) * scale.view(-1, 1, N)).view(K, N)
    return x @ ws


def graded(x: torch.Tensor, planes: torch.Tensor, scale: torch.Tensor, thresholds, group_size: int,
           max_bits: int) -> torch.Tensor:
    sh = 8 - max_bits
    w = weight_int8(planes, max_bits)
    x_abs = x.abs().float().amax(0)
    w_u8 = (w << sh).view(torch.uint8)
    row_mask = torch.zeros_like(x_abs, dtype=torch.uint8)
    bias = torch.zeros_like(x_abs, dtype=torch.float32)
    base = 1 << (max_bits - 1)
    prev = 0
    for zone in range(max_bits // 2):
        active = x_abs > float(thresholds[zone])
        row_mask |= active.to(torch.uint8) * (0xC0 >> 2 * zone)
        cur = base >> (2 * zone + 2)
        bias += active * (cur - prev)
        prev = cur
    masked = (w_u8 & row_mask[:, None]).view(torch.int8).float() / 2 ** sh + bias[:, None]
    return (x.float() @ (masked * scale.float().repeat_interleave(group_size, 0))).to(x.dtype)
