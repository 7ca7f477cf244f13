"""TargetPack tensor encodings and an in-memory pack with the reader interface.

Encodings (explicit per tensor, never inferred from byte lengths), as in the
reference's src/uma_qmoe/target_pack.py:27-176:
  q4_group128  canonical Q4 (see q4.py)
  q8_group128  int8 codes in [-127, 127], scale = absmax/127 per 128 elements
  bf16_le      raw little-endian bf16, round-to-nearest-even from float32

``MemoryTargetPack`` implements the reader methods the operator boundary and
the backend call (``mapping_count``, ``tensor_views``, ``tensor``,
``tensor_q4``, ``layer_encoding``, ``close``), as src/uma_qmoe/target_pack.py:
695-796 does for an mmap'd file.
"""

from __future__ import annotations

from dataclasses import dataclass, field
import math
from typing import Any, Iterable, Mapping

import numpy as np

from .q4 import DEFAULT_GROUP_SIZE, ContractError, Q4Tensor, dequantize_q4, quantize_q4

ENCODINGS = frozenset({"q4_group128", "q8_group128", "bf16_le"})


@dataclass(frozen=True)
class TargetTensor:
    shape: tuple[int, ...]
    encoding: str
    data: bytes
    scales: bytes = b""
    group_size: int | None = None

    @property
    def element_count(self) -> int:
        return math.prod(self.shape)


def _finite_source(values: Any) -> np.ndarray:
    if hasattr(values, "detach"):
        values = values.detach().float().cpu().numpy()
    src = np.asarray(values)
    if src.size == 0 or not np.issubdtype(src.dtype, np.number):
        raise ContractError("TargetPack source must be a non-empty numeric tensor")
    src = src.astype(np.float32)
    if not np.all(np.isfinite(src)):
        raise ContractError("TargetPack source must contain only finite values")
    return src


def float32_to_bf16_bits(values: Any) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    words = np.ascontiguousarray(np.asarray(values, dtype="<f4")).view("<u4")
    return ((words + (np.uint32(0x7FFF) + ((words >> 16) & 1))) >> 16).astype("<u2")


def bf16_bits_to_float32(bits: Any, shape: tuple[int, ...] | None = None) -> np.ndarray:
    out = (np.asarray(bits, dtype="<u2").astype("<u4") << 16).view("<f4")
    return out.reshape(shape) if shape is not None else out


def quantize_q8(values: Any, group_size: int = DEFAULT_GROUP_SIZE) -> TargetTensor:
    src = _finite_source(values)
    flat = src.reshape(-1)
    groups_n = -(-flat.size // group_size)
    padded = np.zeros(groups_n * group_size, dtype=np.float32)
    padded[: flat.size] = flat
    groups = padded.reshape(groups_n, group_size)
    scales = (np.abs(groups).max(axis=1) / np.float32(127.0)).astype("<f4")
    scales[scales == 0] = np.float32(1.0)
    codes = np.clip(np.rint(groups / scales[:, None]), -127, 127).astype(np.int8).reshape(-1)[: flat.size]
    return TargetTensor(tuple(int(d) for d in src.shape), "q8_group128", codes.tobytes(), scales.tobytes(), group_size)


def encode_target_tensor(values: Any, encoding: str, *, group_size: int = DEFAULT_GROUP_SIZE) -> TargetTensor:
    if encoding not in ENCODINGS:
        raise ContractError(f"unsupported TargetPack encoding {encoding!r}")
    if group_size != DEFAULT_GROUP_SIZE:
        raise ContractError("TargetPack v1 requires group size 128")
    src = _finite_source(values)
    shape = tuple(int(d) for d in src.shape)
    if encoding == "bf16_le":
        return TargetTensor(shape, encoding, float32_to_bf16_bits(src).tobytes())
    if encoding == "q8_group128":
        return quantize_q8(src, group_size)
    q = quantize_q4(src, group_size=group_size)
    return TargetTensor(q.shape, encoding, q.packed, q.scales, group_size)


def decode_target_tensor(tensor: TargetTensor) -> np.ndarray:
    """Float32 view of one tensor (host-side inspection; the GPU path never
    materialises this)."""
    if tensor.encoding == "bf16_le":
        if len(tensor.data) != 2 * tensor.element_count or tensor.scales or tensor.group_size is not None:
            raise ContractError("BF16 TargetTensor layout is invalid")
        return bf16_bits_to_float32(np.frombuffer(tensor.data, dtype="<u2"), tensor.shape)
    if tensor.group_size != DEFAULT_GROUP_SIZE:
        raise ContractError("TargetTensor group size is invalid")
    if tensor.encoding == "q4_group128":
        return dequantize_q4(Q4Tensor(tensor.shape, tensor.group_size, tensor.data, tensor.scales))
    if tensor.encoding == "q8_group128":
        groups = -(-tensor.element_count // tensor.group_size)
        if len(tensor.data) != tensor.element_count or len(tensor.scales) != 4 * groups:
            raise ContractError("Q8 TargetTensor payload lengths are invalid")
        scales = np.frombuffer(tensor.scales, dtype="<f4")
        if not np.all(np.isfinite(scales)) or np.any(scales <= 0):
            raise ContractError("Q8 TargetTensor scales must be finite and positive")
        codes = np.frombuffer(tensor.data, dtype=np.int8).astype(np.float32)
        return (codes * np.repeat(scales, tensor.group_size)[: tensor.element_count]).reshape(tensor.shape)
    raise ContractError(f"unsupported TargetTensor encoding {tensor.encoding!r}")


@dataclass
class MemoryTargetPack:
    """An in-memory pack holding already-encoded tensors.

    ``layer_encodings`` maps layer index -> encoding of that layer's routed
    experts. ``model`` carries the fixed-model shape (num_layers, num_experts,
    top_k, hidden_size, intermediate_size) for callers that need it.
    """

    tensors: dict[str, TargetTensor]
    layer_encodings: dict[int, str]
    model: dict[str, Any] = field(default_factory=dict)
    mapping_count: int = 1
    closed: bool = False

    @property
    def header(self) -> dict[str, Any]:
        return {"quantization": {"group_size": DEFAULT_GROUP_SIZE}, "model": dict(self.model)}

    def _get(self, name: str) -> TargetTensor:
        if self.closed:
            raise ContractError("TargetPack is closed")
        try:
            return self.tensors[name]
        except KeyError as exc:
            raise ContractError(f"TargetPack has no tensor {name!r}") from exc

    def tensor(self, name: str) -> TargetTensor:
        return self._get(name)

    def tensor_views(self, name: str) -> tuple[memoryview, memoryview, dict[str, Any]]:
        t = self._get(name)
        meta = {"shape": list(t.shape), "encoding": t.encoding, "group_size": t.group_size}
        return memoryview(t.data), memoryview(t.scales), meta

    def tensor_q4(self, name: str) -> Q4Tensor:
        t = self._get(name)
        if t.encoding != "q4_group128":
            raise ContractError(f"tensor {name!r} is {t.encoding}, not Q4")
        return Q4Tensor(t.shape, int(t.group_size or DEFAULT_GROUP_SIZE), t.data, t.scales)

    def layer_encoding(self, layer_index: int) -> str:
        try:
            return self.layer_encodings[int(layer_index)]
        except KeyError as exc:
            raise ContractError(f"TargetPack has no layer {layer_index}") from exc

    def names(self) -> Iterable[str]:
        return self.tensors.keys()

    def close(self) -> None:
        self.closed = True


def memory_pack(tensors: Mapping[str, TargetTensor], layer_encodings: Mapping[int, str], **model: Any) -> MemoryTargetPack:
    for name, t in tensors.items():
        if t.encoding not in ENCODINGS:
            raise ContractError(f"tensor {name!r} has unsupported encoding {t.encoding!r}")
    return MemoryTargetPack(dict(tensors), {int(k): v for k, v in layer_encodings.items()}, dict(model))


__all__ = [
    "ENCODINGS",
    "MemoryTargetPack",
    "TargetTensor",
    "bf16_bits_to_float32",
    "decode_target_tensor",
    "encode_target_tensor",
    "float32_to_bf16_bits",
    "memory_pack",
    "quantize_q8",
]
