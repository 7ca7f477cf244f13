"""Canonical group-wise signed Q4 codec (host side, for writing packs).

Same format and API as the reference's src/uma_qmoe/q4.py:
  * codes are symmetric in [-7, 7]; the -8 code is reserved and rejected on
    unpack (q4.py:12-14, 117-133), although the HIP kernels decode it;
  * two's-complement nibbles, low nibble = even element (q4.py:96-114);
  * one float32 scale per `group_size` elements of the flattened tensor,
    scale = absmax / 7, an all-zero group gets scale 1.0, codes are
    clip(round_half_even(w / scale)) (q4.py:136-165).

``quantize_q4_tensor`` is the bulk path used to stage synthetic layers: it
runs the same arithmetic with torch on whichever device holds the weights.
"""

from __future__ import annotations

from dataclasses import dataclass
import math
from typing import Any

import numpy as np

Q4_BITS = 4
Q4_MIN = -7
Q4_MAX = 7
DEFAULT_GROUP_SIZE = 128
DEFAULT_ALIGNMENT = 64


class ContractError(ValueError):
    """Invalid codec input or layout (the reference's ContractError, a ValueError)."""


def align_up(value: int, alignment: int) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value < 0:
        raise ContractError("alignment input must be a non-negative integer")
    if isinstance(alignment, bool) or not isinstance(alignment, int) or alignment <= 0 or alignment & (alignment - 1):
        raise ContractError("alignment must be a positive power of two")
    return -(-value // alignment) * alignment


@dataclass(frozen=True)
class Q4Layout:
    element_count: int
    group_size: int
    group_count: int
    packed_bytes: int
    scale_bytes: int
    unpadded_bytes: int
    storage_bytes: int
    alignment_bytes: int
    effective_bits_per_weight: float


@dataclass(frozen=True)
class Q4Tensor:
    shape: tuple[int, ...]
    group_size: int
    packed: bytes
    scales: bytes

    @property
    def element_count(self) -> int:
        return math.prod(self.shape)

    @property
    def layout(self) -> Q4Layout:
        return q4_layout(self.element_count, self.group_size)


def q4_layout(element_count: int, group_size: int = DEFAULT_GROUP_SIZE, alignment_bytes: int = DEFAULT_ALIGNMENT) -> Q4Layout:
    for value, what in ((element_count, "element_count"), (group_size, "group_size")):
        if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
            raise ContractError(f"Q4 {what} must be a positive integer")
    groups = -(-element_count // group_size)
    packed = -(-element_count // 2)
    scale_bytes = 4 * groups
    storage = align_up(packed + scale_bytes, alignment_bytes)
    return Q4Layout(
        element_count=element_count,
        group_size=group_size,
        group_count=groups,
        packed_bytes=packed,
        scale_bytes=scale_bytes,
        unpadded_bytes=packed + scale_bytes,
        storage_bytes=storage,
        alignment_bytes=alignment_bytes,
        effective_bits_per_weight=storage * 8 / element_count,
    )


def pack_int4(values: Any) -> bytes:
    """Pack signed codes in [-7, 7], low nibble first, two's complement."""
    codes = np.asarray(values).reshape(-1)
    if codes.size == 0:
        raise ContractError("cannot pack an empty Q4 array")
    if not np.issubdtype(codes.dtype, np.integer):
        raise ContractError("Q4 nibble input must be integer")
    wide = codes.astype(np.int16)
    if wide.min() < Q4_MIN or wide.max() > Q4_MAX:
        raise ContractError("Q4 nibble input is outside [-7, 7]")
    nib = np.zeros(codes.size + (codes.size & 1), dtype=np.uint8)
    nib[: codes.size] = (wide & 0xF).astype(np.uint8)
    return (nib[0::2] | (nib[1::2] << 4)).tobytes()


def unpack_int4(payload: bytes | bytearray | memoryview, element_count: int) -> np.ndarray:
    layout = q4_layout(element_count)
    raw = np.frombuffer(payload, dtype=np.uint8)
    if raw.size != layout.packed_bytes:
        raise ContractError("Q4 packed byte count does not match element count")
    both = np.stack((raw & 0xF, raw >> 4), axis=1).reshape(-1).astype(np.int8)
    signed = np.where(both >= 8, both - 16, both).astype(np.int8)
    values = signed[:element_count]
    if np.any(values == -8):
        raise ContractError("Q4 payload contains the reserved -8 code")
    if element_count % 2 and both[-1] != 0:
        raise ContractError("Q4 odd tail padding nibble must be zero")
    return values


def quantize_q4(values: Any, *, group_size: int = DEFAULT_GROUP_SIZE) -> Q4Tensor:
    source = np.asarray(values)
    if source.size == 0:
        raise ContractError("cannot quantize an empty tensor")
    if not np.issubdtype(source.dtype, np.number) or not np.all(np.isfinite(source)):
        raise ContractError("Q4 source must contain only finite numeric values")
    shape = tuple(int(d) for d in source.shape)
    flat = source.astype(np.float32).reshape(-1)
    layout = q4_layout(int(flat.size), group_size)
    padded = np.zeros(layout.group_count * group_size, dtype=np.float32)
    padded[: flat.size] = flat
    groups = padded.reshape(layout.group_count, group_size)
    scales = (np.abs(groups).max(axis=1) / np.float32(Q4_MAX)).astype("<f4")
    scales[scales == 0] = np.float32(1.0)
    codes = np.clip(np.rint(groups / scales[:, None]), Q4_MIN, Q4_MAX).astype(np.int8).reshape(-1)[: flat.size]
    return Q4Tensor(shape=shape, group_size=group_size, packed=pack_int4(codes), scales=scales.tobytes())


def dequantize_q4(tensor: Q4Tensor) -> np.ndarray:
    layout = q4_layout(tensor.element_count, tensor.group_size)
    if len(tensor.packed) != layout.packed_bytes or len(tensor.scales) != layout.scale_bytes:
        raise ContractError("Q4 tensor payload lengths do not match layout")
    codes = unpack_int4(tensor.packed, tensor.element_count).astype(np.float32)
    scales = np.frombuffer(tensor.scales, dtype="<f4")
    if not np.all(np.isfinite(scales)) or np.any(scales <= 0):
        raise ContractError("Q4 scales must be finite and positive")
    return (codes * np.repeat(scales, tensor.group_size)[: tensor.element_count]).reshape(tensor.shape)


def quantize_groups_tensor(weights, qmax: int, group_size: int = DEFAULT_GROUP_SIZE):
    """Symmetric group quantization of each leading-dim tensor with torch.

    ``weights`` is [..., n] per tensor; groups run along the last (flattened
    per-tensor) dimension, which must be a multiple of ``group_size``.
    Returns (codes int8 [..., n], scales float32 [..., n / group_size]).
    """
    import torch

    w = weights.to(torch.float32)
    n = w.shape[-1]
    if n % group_size:
        raise ContractError("bulk quantization needs the tensor size to be a multiple of the group size")
    g = w.reshape(*w.shape[:-1], n // group_size, group_size)
    scales = g.abs().amax(dim=-1) / float(qmax)
    scales = torch.where(scales == 0, torch.ones_like(scales), scales)
    codes = torch.clamp(torch.round(g / scales.unsqueeze(-1)), -qmax, qmax).to(torch.int8)
    return codes.reshape(w.shape), scales


def pack_codes_tensor(codes):
    """Pack int8 codes [..., n] (n even) into uint8 [..., n/2], low nibble first."""
    import torch

    nib = (codes.to(torch.int16) & 0xF).to(torch.uint8)
    return nib[..., 0::2] | (nib[..., 1::2] << 4)


def quantize_q4_tensor(weights, group_size: int = DEFAULT_GROUP_SIZE):
    """Bulk Q4: (packed uint8 [..., n/2], scales float32 [..., n/group])."""
    codes, scales = quantize_groups_tensor(weights, Q4_MAX, group_size)
    return pack_codes_tensor(codes), scales


__all__ = [
    "DEFAULT_ALIGNMENT",
    "DEFAULT_GROUP_SIZE",
    "ContractError",
    "Q4Layout",
    "Q4Tensor",
    "align_up",
    "dequantize_q4",
    "pack_int4",
    "q4_layout",
    "quantize_q4",
    "quantize_q4_tensor",
    "unpack_int4",
]
