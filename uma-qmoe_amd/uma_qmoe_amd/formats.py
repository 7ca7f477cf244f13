"""Tensor encodings of the packed-expert formats (host side, offline).

Every routed-expert matrix of a pack is stored in one of three encodings,
named per tensor and never inferred from byte counts (the formats of
src/uma_qmoe/q4.py:96-179 and src/uma_qmoe/target_pack.py:78-176):

  q4_group128  signed 4-bit codes in [-7, 7] (the code -8 is reserved), two
               per byte, element 2i in the low nibble, two's complement; one
               float32 scale per 128 consecutive elements of the flattened
               tensor: scale = max|w| / 7 (1.0 for an all-zero group), code =
               clamp(round_half_even(w / scale), -7, 7). An ExpertPack may
               declare another group size; TargetPacks always use 128.
  q8_group128  int8 codes in [-127, 127], same grouping, scale = max|w| / 127.
  bf16_le      the float32 value rounded to the nearest bf16 (ties to even),
               little-endian words, no scales.

A tail group shorter than the group size is quantized as if zero-padded, and
an odd Q4 element count leaves a zero high nibble in the last byte.

The arithmetic is written once, vectorised with torch over any leading
dimensions, so the same functions encode one tensor on the CPU for a pack
writer or a whole [E, rows, cols] projection on the GPU for the seeded
benchmark layers. The HIP kernels read the resulting bytes as they are.
"""

from __future__ import annotations

from dataclasses import dataclass
import math
from typing import Any

import numpy as np

GROUP_SIZE = 128


class ContractError(ValueError):
    """A tensor, payload or pack violates the format contract."""


@dataclass(frozen=True)
class TargetTensor:
    """One encoded tensor as a TargetPack stores it (bytes + optional scales)."""

    shape: tuple[int, ...]
    encoding: str
    data: bytes
    scales: bytes = b""
    group_size: int | None = None

    @property
    def element_count(self) -> int:
        return math.prod(self.shape)


@dataclass(frozen=True)
class Q4Tensor:
    """One Q4 tensor as an ExpertPack hands it out (``tensor_q4``)."""

    shape: tuple[int, ...]
    group_size: int
    packed: bytes
    scales: bytes

    @property
    def element_count(self) -> int:
        return math.prod(self.shape)


@dataclass(frozen=True)
class Encoding:
    """Byte layout and code range of one encoding."""

    name: str
    bits: int
    qmax: int  # largest code magnitude; 0 for the unquantized bf16

    @property
    def grouped(self) -> bool:
        return self.qmax > 0

    def data_bytes(self, elements: int) -> int:
        return -(-elements * self.bits // 8)

    def scale_bytes(self, elements: int, group: int = GROUP_SIZE) -> int:
        return 4 * -(-elements // group) if self.grouped else 0


Q4 = Encoding("q4_group128", 4, 7)
Q8 = Encoding("q8_group128", 8, 127)
BF16 = Encoding("bf16_le", 16, 0)
ENCODINGS: dict[str, Encoding] = {e.name: e for e in (Q4, Q8, BF16)}


def encoding(name: str) -> Encoding:
    try:
        return ENCODINGS[name]
    except KeyError:
        raise ContractError(f"unsupported TargetPack encoding {name!r}") from None


# ------------------------------------------------------- vectorised core --
def group_codes(weights: Any, qmax: int, group: int = GROUP_SIZE):
    """Symmetric group quantization along the last dimension.

    ``weights`` [..., n] (any float dtype and device) -> (codes int8 [..., n],
    scales float32 [..., ceil(n / group)]). The float32 division and the
    half-to-even rounding are the reference's (q4.py:155-159,
    target_pack.py:92-112).
    """
    import torch

    w = weights.to(torch.float32)
    n = w.shape[-1]
    groups = -(-n // group)
    if groups * group != n:
        w = torch.nn.functional.pad(w, (0, groups * group - n))
    g = w.reshape(*w.shape[:-1], groups, group)
    scales = g.abs().amax(dim=-1) / float(qmax)
    scales = torch.where(scales == 0, torch.ones_like(scales), scales)
    codes = torch.round(g / scales.unsqueeze(-1)).clamp_(-qmax, qmax).to(torch.int8)
    return codes.reshape(*w.shape[:-1], groups * group)[..., :n], scales


def nibbles(codes: Any):
    """int8 codes [..., n] -> uint8 [..., ceil(n / 2)], element 2i in the low nibble."""
    import torch

    c = (codes.to(torch.int16) & 0xF).to(torch.uint8)
    if c.shape[-1] % 2:
        c = torch.nn.functional.pad(c, (0, 1))
    return c[..., 0::2] | (c[..., 1::2] << 4)


def from_nibbles(packed: Any, n: int):
    """uint8 [..., m] -> signed int8 codes [..., n] (no range checks)."""
    import torch

    p = packed.to(torch.int16)
    both = torch.stack((p & 0xF, p >> 4), dim=-1).reshape(*p.shape[:-1], -1)
    return torch.where(both >= 8, both - 16, both).to(torch.int8)[..., :n]


def bf16_words(weights: Any):
    """Round-to-nearest-even bf16 bit patterns (int16) of float values."""
    import torch

    return weights.to(torch.float32).to(torch.bfloat16).view(torch.int16)


def encode_projection(weights: Any, name: str, group: int = GROUP_SIZE):
    """Encode [..., rows, cols] float weights tensor by tensor (groups run
    along each flattened [rows, cols] matrix) -> (data, scales or None):
    Q4 uint8 [..., rows, cols/2], Q8 int8 [..., rows, cols], BF16 bfloat16
    [..., rows, cols]; scales float32 [..., rows*cols/group]."""
    import torch

    enc = encoding(name)
    if not enc.grouped:
        return weights.to(torch.bfloat16).contiguous(), None
    *lead, rows, cols = weights.shape
    if enc is Q4 and cols % 2:
        raise ContractError("bulk Q4 encoding needs an even column count")
    codes, scales = group_codes(weights.reshape(*lead, rows * cols), enc.qmax, group)
    data = nibbles(codes).reshape(*lead, rows, cols // 2) if enc is Q4 else codes.reshape(*lead, rows, cols)
    return data.contiguous(), scales.contiguous()


# ---------------------------------------------------------- one tensor --
def _source(values: Any):
    import torch

    if isinstance(values, torch.Tensor):
        src = values.detach().to("cpu", torch.float32)
    else:
        arr = np.asarray(values)
        if arr.size == 0 or not np.issubdtype(arr.dtype, np.number):
            raise ContractError("TargetPack source must be a non-empty numeric tensor")
        src = torch.from_numpy(np.ascontiguousarray(arr, dtype=np.float32))
    if src.numel() == 0:
        raise ContractError("TargetPack source must be a non-empty numeric tensor")
    if not bool(torch.isfinite(src).all()):
        raise ContractError("TargetPack source must contain only finite values")
    return src


def encode(values: Any, name: str, *, group_size: int = GROUP_SIZE) -> TargetTensor:
    """Encode one tensor (numpy or torch, any shape) into ``name``."""
    enc = encoding(name)
    src = _source(values)
    shape = tuple(int(d) for d in src.shape)
    flat = src.reshape(-1)
    if not enc.grouped:
        return TargetTensor(shape, enc.name, bf16_words(flat).numpy().tobytes())
    codes, scales = group_codes(flat, enc.qmax, group_size)
    data = nibbles(codes) if enc is Q4 else codes
    return TargetTensor(shape, enc.name, data.numpy().tobytes(), scales.numpy().astype("<f4").tobytes(), group_size)


def check_payload(name: str, data: Any, scales: Any, elements: int, group: int = GROUP_SIZE, what: str = "tensor") -> None:
    """Length and value checks of one stored tensor: payload sizes, the
    reserved Q4 code, the Q4 tail nibble, finite positive scales."""
    enc = encoding(name)
    raw = np.frombuffer(data, dtype=np.uint8)
    if raw.size != enc.data_bytes(elements) or len(scales) != enc.scale_bytes(elements, group):
        raise ContractError(f"{what} payload lengths do not match its {name} layout")
    if enc is Q4:
        if bool(np.any(((raw & 0x0F) == 8) | ((raw >> 4) == 8))):
            raise ContractError(f"{what} contains the reserved Q4 -8 code")
        if elements % 2 and raw[-1] >> 4:
            raise ContractError(f"{what} has non-zero Q4 odd tail padding")
    if enc.grouped:
        s = np.frombuffer(scales, dtype="<f4")
        if not bool(np.all(np.isfinite(s) & (s > 0))):
            raise ContractError(f"{what} scales must be finite and positive")


def decode(tensor: TargetTensor) -> np.ndarray:
    """Float32 values of one stored tensor (host-side inspection and the
    correctness checks; the GPU path never expands weights)."""
    import torch

    enc = encoding(tensor.encoding)
    n = tensor.element_count
    if enc.grouped:
        if tensor.group_size is None or tensor.group_size <= 0:
            raise ContractError("TargetTensor group size is invalid")
        check_payload(enc.name, tensor.data, tensor.scales, n, tensor.group_size, "TargetTensor")
    elif len(tensor.data) != 2 * n or tensor.scales or tensor.group_size is not None:
        raise ContractError("BF16 TargetTensor layout is invalid")
    raw = torch.frombuffer(bytearray(tensor.data), dtype=torch.uint8)
    if not enc.grouped:
        return raw.view(torch.bfloat16).float().numpy().reshape(tensor.shape)
    codes = from_nibbles(raw, n) if enc is Q4 else raw.view(torch.int8)
    scales = torch.frombuffer(bytearray(tensor.scales), dtype=torch.float32)
    per_element = scales.repeat_interleave(tensor.group_size)[:n]
    return (codes.to(torch.float32) * per_element).numpy().reshape(tensor.shape)


# ------------------------------------ reference-named codec entry points --
def quantize_q4(values: Any, *, group_size: int = GROUP_SIZE) -> Q4Tensor:
    """Canonical Q4 of one tensor (src/uma_qmoe/q4.py:136-165)."""
    if isinstance(group_size, bool) or not isinstance(group_size, int) or group_size <= 0:
        raise ContractError("Q4 group_size must be a positive integer")
    t = encode(values, Q4.name, group_size=group_size)
    return Q4Tensor(t.shape, group_size, t.data, t.scales)


def dequantize_q4(tensor: Q4Tensor) -> np.ndarray:
    """Float32 values of a Q4 tensor (src/uma_qmoe/q4.py:168-179)."""
    return decode(TargetTensor(tuple(tensor.shape), Q4.name, tensor.packed, tensor.scales, tensor.group_size))


def pack_int4(values: Any) -> bytes:
    """Codes in [-7, 7] -> packed bytes (src/uma_qmoe/q4.py:96-114)."""
    import torch

    codes = np.asarray(values).reshape(-1)
    if codes.size == 0:
        raise ContractError("cannot pack an empty Q4 array")
    if not np.issubdtype(codes.dtype, np.integer):
        raise ContractError("Q4 nibble input must be integer")
    if codes.min() < -Q4.qmax or codes.max() > Q4.qmax:
        raise ContractError("Q4 nibble input is outside [-7, 7]")
    return nibbles(torch.from_numpy(codes.astype(np.int8))).numpy().tobytes()


def unpack_int4(payload: Any, element_count: int) -> np.ndarray:
    """Packed bytes -> int8 codes, rejecting the reserved -8 and a non-zero
    odd tail nibble (src/uma_qmoe/q4.py:117-133)."""
    import torch

    if isinstance(element_count, bool) or not isinstance(element_count, int) or element_count <= 0:
        raise ContractError("Q4 element_count must be a positive integer")
    raw = np.frombuffer(payload, dtype=np.uint8)
    if raw.size != Q4.data_bytes(element_count):
        raise ContractError("Q4 packed byte count does not match element count")
    codes = from_nibbles(torch.from_numpy(raw.copy()), element_count).numpy()
    if bool(np.any(codes == -8)):
        raise ContractError("Q4 payload contains the reserved -8 code")
    if element_count % 2 and raw[-1] >> 4:
        raise ContractError("Q4 odd tail padding nibble must be zero")
    return codes


def encode_target_tensor(values: Any, encoding_name: str, *, group_size: int = GROUP_SIZE) -> TargetTensor:
    """One tensor in a TargetPack encoding (src/uma_qmoe/target_pack.py:115-141)."""
    encoding(encoding_name)
    if group_size != GROUP_SIZE:
        raise ContractError("TargetPack v1 requires group size 128")
    return encode(values, encoding_name)


def decode_target_tensor(tensor: TargetTensor) -> np.ndarray:
    """Float32 values of a TargetPack tensor (src/uma_qmoe/target_pack.py:144-176)."""
    if encoding(tensor.encoding).grouped and tensor.group_size != GROUP_SIZE:
        raise ContractError("TargetTensor group size is invalid")
    return decode(tensor)


__all__ = [
    "BF16",
    "ENCODINGS",
    "GROUP_SIZE",
    "Q4",
    "Q8",
    "ContractError",
    "Encoding",
    "Q4Tensor",
    "TargetTensor",
    "bf16_words",
    "check_payload",
    "decode",
    "decode_target_tensor",
    "dequantize_q4",
    "encode",
    "encode_projection",
    "encode_target_tensor",
    "encoding",
    "from_nibbles",
    "group_codes",
    "nibbles",
    "pack_int4",
    "quantize_q4",
    "unpack_int4",
]
