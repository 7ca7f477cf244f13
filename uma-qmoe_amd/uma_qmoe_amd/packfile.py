"""ExpertPack / TargetPack files: writer, one-mmap reader, in-memory pack.

Both pack kinds share one container (src/uma_qmoe/expert_pack.py:166-300,
src/uma_qmoe/target_pack.py:394-489); only the header's fields differ:

  prefix   96 bytes, little endian: magic[8] ("UQMOEPK1" ExpertPack, all Q4;
           "UQMOTPK1" TargetPack, one encoding per layer), version u32 (1),
           header length u32, payload offset u64, payload length u64,
           SHA-256 of the header [32], SHA-256 of the payload [32];
  header   canonical JSON (sorted keys, separators "," and ":", UTF-8), then
           zero bytes up to the payload offset, a multiple of 4096;
  payload  the tensors in header order; each starts at a multiple of the
           tensor alignment (64), holds its data, zero bytes up to a multiple
           of 4, its float32 scales, and zero bytes up to the next multiple of
           the alignment. Nothing else is in the payload.

The header lists every tensor with its offsets (relative to the payload),
byte counts, shape and the SHA-256 of its data followed by its scales. The
model identity is the SHA-256 of the canonical JSON of {model_id,
model_revision, model_manifest_sha256}; a TargetPack's policy identity is the
SHA-256 of {policy_id, layer_encodings, policy_evidence_sha256}.

``PackReader`` is the library's C++ reader (csrc/uqm_pack.cpp): it maps the
file once (the custom operator requires exactly one mapping per pack) and
validates it completely before use: prefix, both hashes, canonical JSON,
identities, the layout of every tensor, zero padding, per-tensor hashes and
the payload semantics (no reserved Q4 code, zero Q4 tail nibble, finite
positive scales), on worker threads. Tensor views are zero-copy slices of the
mapping; the HIP backend stages a layer's experts straight from the mapping
through pinned buffers to the device (``stage_projection``).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
import hashlib
import json
import os
from pathlib import Path
import re
import struct
import tempfile
from typing import Any, Iterable, Iterator, Mapping
import weakref


from .formats import (
    ENCODINGS,
    GROUP_SIZE,
    Q4,
    ContractError,
    Q4Tensor,
    TargetTensor,
    check_payload,
    encode,
    encoding,
)

VERSION = 1
HEADER_ALIGNMENT = 4096
TENSOR_ALIGNMENT = 64
PREFIX = struct.Struct("<8sIIQQ32s32s")
EXPERT_MAGIC = b"UQMOEPK1"
TARGET_MAGIC = b"UQMOTPK1"
QWEN_MODEL_ID = "Qwen/Qwen1.5-MoE-A2.7B"
_SAFE_NAME = re.compile(r"^[A-Za-z0-9_.-]+$")
_EXPERT_NAME = re.compile(r"^model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight$")
_HEX40 = re.compile(r"^[0-9a-f]{40}$")
_HEX64 = re.compile(r"^[0-9a-f]{64}$")

# Header constants of the two formats.
Q4_CONTRACT = {
    "bits": 4,
    "nibble_order": "low_first_twos_complement",
    "rounding": "nearest_even",
    "scale_dtype": "float32_le",
    "signed_range": [-7, 7],
    "zero_point": None,
}
TARGET_ENCODINGS = {
    "q4_group128": {**Q4_CONTRACT, "group_size": GROUP_SIZE},
    "q8_group128": {"bits": 8, "group_size": GROUP_SIZE, "rounding": "nearest_even", "scale_dtype": "float32_le",
                    "signed_range": [-127, 127], "zero_point": None},
    "bf16_le": {"bits": 16, "byte_order": "little"},
}


def canonical_json(value: Any) -> bytes:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False).encode("utf-8")


def _sha256_json(value: Any) -> str:
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":")).encode("utf-8")).hexdigest()


def model_identity(model_id: str, model_revision: str, manifest_sha256: str) -> str:
    return _sha256_json({"model_id": model_id, "model_revision": model_revision,
                         "model_manifest_sha256": manifest_sha256})


def fixed_model_dims(model_id: str) -> tuple[str, int, int]:
    """(name, layers, experts) of the two fixed models a TargetPack targets."""
    return ("Qwen", 24, 60) if model_id == QWEN_MODEL_ID else ("OLMoE", 16, 64)


def policy_block(policy_id: str, layer_encodings: Mapping[int, str], evidence_sha256: str, layers: int,
                 model_name: str) -> dict[str, Any]:
    """The TargetPack ``policy`` header object, validated."""
    if not isinstance(policy_id, str) or not policy_id:
        raise ContractError("TargetPack policy id must be non-empty")
    if set(layer_encodings) != set(range(layers)):
        raise ContractError(f"TargetPack policy must assign every {model_name} layer exactly once")
    if any(v not in ENCODINGS for v in layer_encodings.values()):
        raise ContractError("TargetPack policy contains an unsupported encoding")
    if not isinstance(evidence_sha256, str) or not _HEX64.fullmatch(evidence_sha256):
        raise ContractError("TargetPack policy evidence identity must be SHA-256")
    by_layer = {str(i): layer_encodings[i] for i in range(layers)}
    return {
        "policy_id": policy_id,
        "layer_encodings": by_layer,
        "policy_evidence_sha256": evidence_sha256,
        "policy_identity_sha256": _sha256_json({"policy_id": policy_id, "layer_encodings": by_layer,
                                                "policy_evidence_sha256": evidence_sha256}),
    }


def _align(v: int, a: int) -> int:
    return -(-v // a) * a


def _check_alignment(a: Any) -> int:
    if isinstance(a, bool) or not isinstance(a, int) or a <= 0 or a & (a - 1):
        raise ContractError("alignment must be a positive power of two")
    return a


@dataclass(frozen=True)
class _Kind:
    magic: bytes
    label: str
    data_field: str  # "packed" (ExpertPack) or "data" (TargetPack)


EXPERT_PACK = _Kind(EXPERT_MAGIC, "ExpertPack", "packed")
TARGET_PACK = _Kind(TARGET_MAGIC, "TargetPack", "data")
_KINDS = {k.magic: k for k in (EXPERT_PACK, TARGET_PACK)}


# ------------------------------------------------------------------ writer --
def _identity_fields(kind: _Kind, model_id: str, model_revision: str, manifest: str) -> dict[str, Any]:
    if not isinstance(model_revision, str) or not _HEX40.fullmatch(model_revision):
        raise ContractError(f"{kind.label} model revision must be a lowercase git SHA")
    if not isinstance(manifest, str) or not _HEX64.fullmatch(manifest):
        raise ContractError(f"{kind.label} model manifest identity must be SHA-256")
    return {"model_id": model_id, "model_revision": model_revision, "model_manifest_sha256": manifest,
            "model_identity_sha256": model_identity(model_id, model_revision, manifest)}


def _write(kind: _Kind, destination: str | Path, items: Iterator[tuple[str, TargetTensor, dict[str, Any]]],
           header_fields: dict[str, Any], alignment: int) -> Path:
    """Streams the payload into a temporary file beside the destination,
    then writes prefix + header + payload. ``items`` yields (name, encoded
    tensor, extra header fields of that tensor)."""
    target = Path(destination)
    target.parent.mkdir(parents=True, exist_ok=True)
    if target.exists():
        raise ContractError(f"refusing to overwrite existing {kind.label} {target}")
    entries: list[dict[str, Any]] = []
    names: set[str] = set()
    digest = hashlib.sha256()
    fd, tmp_name = tempfile.mkstemp(prefix=f".{target.name}.", suffix=".payload", dir=target.parent)
    tmp = Path(tmp_name)
    try:
        with os.fdopen(fd, "wb") as payload:
            size = 0

            def put(b: bytes) -> None:
                nonlocal size
                payload.write(b)
                digest.update(b)
                size += len(b)

            for name, t, extra in items:
                if not isinstance(name, str) or not _SAFE_NAME.fullmatch(name):
                    raise ContractError(f"invalid {kind.label} tensor name {name!r}")
                if name in names:
                    raise ContractError(f"duplicate {kind.label} tensor name {name!r}")
                names.add(name)
                start = _align(size, alignment)
                put(bytes(start - size))
                put(t.data)
                scale_at = _align(size, 4)
                put(bytes(scale_at - size))
                put(t.scales)
                end = _align(size, alignment)
                put(bytes(end - size))
                n = t.element_count
                group = t.group_size or GROUP_SIZE
                entry = {
                    "name": name,
                    "shape": list(t.shape),
                    "element_count": n,
                    f"{kind.data_field}_offset": start,
                    f"{kind.data_field}_bytes": len(t.data),
                    "scale_offset": scale_at,
                    "scale_bytes": len(t.scales),
                    "storage_end_offset": end,
                    "group_count": -(-n // group) if t.scales else 0,
                    "effective_bits_per_weight": (end - start) * 8 / n,
                    "tensor_payload_sha256": hashlib.sha256(t.data + t.scales).hexdigest(),
                    **extra,
                }
                entries.append(entry)
        if not entries:
            raise ContractError(f"{kind.label} must contain at least one tensor")
        header = {**header_fields, "schema_version": VERSION, "tensor_alignment_bytes": alignment,
                  "tensor_count": len(entries), "tensors": entries}
        if kind is TARGET_PACK:
            header["encoding_tensor_counts"] = {e: sum(x["encoding"] == e for x in entries) for e in sorted(ENCODINGS)}
        hb = canonical_json(header)
        payload_offset = _align(PREFIX.size + len(hb), HEADER_ALIGNMENT)
        prefix = PREFIX.pack(kind.magic, VERSION, len(hb), payload_offset, size, hashlib.sha256(hb).digest(),
                             digest.digest())
        with target.open("xb") as out, tmp.open("rb") as src:
            out.write(prefix)
            out.write(hb)
            out.write(bytes(payload_offset - PREFIX.size - len(hb)))
            while chunk := src.read(1 << 23):
                out.write(chunk)
        return target
    except BaseException:
        if target.exists():
            target.unlink()
        raise
    finally:
        tmp.unlink(missing_ok=True)


def write_expert_pack(destination: str | Path, tensors: Iterable[tuple[str, Any]], *, model_id: str,
                      model_revision: str, model_manifest_sha256: str, group_size: int = GROUP_SIZE,
                      tensor_alignment_bytes: int = TENSOR_ALIGNMENT) -> dict[str, Any]:
    """Writes an all-Q4 ExpertPack (values are quantized as they stream in;
    a ``Q4Tensor`` is stored as it is) and returns its inspection record."""
    _check_alignment(tensor_alignment_bytes)
    header = {"format": "canonical_q4_symmetric_grouped",
              "model": _identity_fields(EXPERT_PACK, model_id, model_revision, model_manifest_sha256),
              "quantization": {**Q4_CONTRACT, "group_size": group_size}}

    def items():
        for name, values in tensors:
            if isinstance(values, TargetTensor):
                if values.encoding != Q4.name:
                    raise ContractError(f"ExpertPack tensor {name!r} is {values.encoding}, not Q4")
                values = Q4Tensor(values.shape, values.group_size or GROUP_SIZE, values.data, values.scales)
            if isinstance(values, Q4Tensor):
                if values.group_size != group_size:
                    raise ContractError("pre-encoded Q4 tensor group size differs from the pack's")
                t = TargetTensor(tuple(values.shape), Q4.name, values.packed, values.scales, group_size)
                check_payload(Q4.name, t.data, t.scales, t.element_count, group_size, f"tensor {name!r}")
            else:
                t = encode(values, Q4.name, group_size=group_size)
            yield name, t, {}

    return inspect_pack(_write(EXPERT_PACK, destination, items(), header, tensor_alignment_bytes))


def write_target_pack(destination: str | Path, tensors: Iterable[tuple[str, Any]], *, model_id: str,
                      model_revision: str, model_manifest_sha256: str, policy_id: str,
                      layer_encodings: Mapping[int, str], policy_evidence_sha256: str,
                      tensor_alignment_bytes: int = TENSOR_ALIGNMENT) -> dict[str, Any]:
    """Writes a TargetPack: each expert tensor in its layer's encoding (a
    ``TargetTensor`` must already be in it) and returns its inspection record."""
    _check_alignment(tensor_alignment_bytes)
    model_name, layers, experts = fixed_model_dims(model_id)
    header = {"format": "mixed_precision_target_pack",
              "model": _identity_fields(TARGET_PACK, model_id, model_revision, model_manifest_sha256),
              "policy": policy_block(policy_id, layer_encodings, policy_evidence_sha256, layers, model_name),
              "encodings": TARGET_ENCODINGS}

    def items():
        for name, values in tensors:
            m = _EXPERT_NAME.fullmatch(name) if isinstance(name, str) else None
            if m is None:
                raise ContractError(f"unexpected TargetPack tensor name {name!r}")
            layer, expert = int(m.group(1)), int(m.group(2))
            if layer >= layers or expert >= experts:
                raise ContractError(f"TargetPack tensor identity is out of range: {name!r}")
            enc = layer_encodings[layer]
            if isinstance(values, TargetTensor):
                t = values
                if t.encoding != enc:
                    raise ContractError("pre-encoded TargetTensor does not match its layer policy")
                if not t.shape or any(isinstance(d, bool) or not isinstance(d, int) or d <= 0 for d in t.shape):
                    raise ContractError("pre-encoded TargetTensor shape is invalid")
                if encoding(enc).grouped and t.group_size != GROUP_SIZE:
                    raise ContractError("pre-encoded TargetTensor requires group size 128")
                if not encoding(enc).grouped and (t.scales or t.group_size is not None):
                    raise ContractError("pre-encoded BF16 TargetTensor layout is invalid")
                check_payload(enc, t.data, t.scales, t.element_count, GROUP_SIZE, "pre-encoded TargetTensor")
            else:
                t = encode(values, enc)
            yield name, t, {"layer_index": layer, "expert_index": expert, "projection": m.group(3),
                            "encoding": enc, "group_size": t.group_size}

    return inspect_pack(_write(TARGET_PACK, destination, items(), header, tensor_alignment_bytes))


# ------------------------------------------------------------------ reader --
_ENCODING_NAMES = {0: "q4_group128", 1: "q8_group128", 2: "bf16_le"}  # UQM_Q4 / UQM_Q8 / UQM_BF16
_PACK_KINDS = {0: EXPERT_PACK, 1: TARGET_PACK}  # UQM_PACK_EXPERT / UQM_PACK_TARGET
_PROJECTION_IDS = {"gate_proj": 0, "up_proj": 1, "down_proj": 2}


class PackReader:
    """A validated pack file, read by the library's C++ reader
    (csrc/uqm_pack.cpp, ``uqm_pack_open``): one read-only mapping, every
    check of the format made before the constructor returns, and the first
    violation raised as ``ContractError`` with the reference reader's
    message. ``tensor_views`` are zero-copy views of the mapping; after
    ``close()`` the mapping lives on until the last view handed out is
    released."""

    kind: _Kind | None = None  # set by the kind-specific subclasses

    def __init__(self, path: str | Path, *, expected_model_id: str | None = None,
                 expected_model_revision: str | None = None, expected_model_manifest_sha256: str | None = None,
                 expected_policy_id: str | None = None) -> None:
        from . import _native

        self.path = Path(path)
        self._lib = _native.library()
        self._handle = None
        self._closed = False
        self._live_views = 0
        want_kind = -1 if self.kind is None else (0 if self.kind is EXPERT_PACK else 1)

        def c(v: str | None):
            return None if v is None else str(v).encode("utf-8")

        handle = ctypes.c_void_p()
        rc = self._lib.uqm_pack_open(os.fsencode(self.path), want_kind, c(expected_model_id),
                                     c(expected_model_revision), c(expected_model_manifest_sha256),
                                     c(expected_policy_id), ctypes.byref(handle))
        self._check(rc, "uqm_pack_open")
        self._handle = handle
        self.mapping_count = 1
        kind, poff, plen, group = ctypes.c_int32(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_int32()
        self._check(self._lib.uqm_pack_info(handle, ctypes.byref(kind), ctypes.byref(poff), ctypes.byref(plen),
                                            ctypes.byref(group)), "uqm_pack_info")
        self.kind = _PACK_KINDS[kind.value]
        self.payload_offset, self.payload_length, self.group_size = poff.value, plen.value, group.value
        text, length = ctypes.c_char_p(), ctypes.c_size_t()
        self._check(self._lib.uqm_pack_header(handle, ctypes.byref(text), ctypes.byref(length)), "uqm_pack_header")
        self.header = json.loads(ctypes.string_at(text, length.value))
        self._index = {t["name"]: t for t in self.header["tensors"]}

    def _check(self, rc: int, what: str) -> None:
        from . import _native

        if rc == _native.UQM_ERR_PACK:
            raise ContractError(self._lib.uqm_last_error().decode("utf-8", "replace"))
        _native.check(rc, what)

    # -- access ----------------------------------------------------------------
    def _entry(self, name: str) -> dict[str, Any]:
        if self._closed:
            raise ContractError(f"{self.kind.label} is closed")
        try:
            return self._index[name]
        except KeyError:
            raise ContractError(f"{self.kind.label} has no tensor {name!r}") from None

    def _lookup(self, name: str):
        from . import _native

        self._entry(name)
        info = _native.PackTensor()
        self._check(self._lib.uqm_pack_lookup(self._handle, name.encode("utf-8"), ctypes.byref(info)),
                    "uqm_pack_lookup")
        return info

    def _view(self, address: int, nbytes: int) -> memoryview:

        if nbytes == 0 or not address:
            return memoryview(b"")
        array = (ctypes.c_ubyte * nbytes).from_address(address)
        self._live_views += 1
        weakref.finalize(array, self._view_released)
        return memoryview(array).cast("B")

    def _view_released(self) -> None:
        self._live_views -= 1
        if self._closed and self._live_views == 0:
            self._release()

    def tensor_views(self, name: str) -> tuple[memoryview, memoryview, Mapping[str, Any]]:
        """Zero-copy (data, scales, header entry) of one tensor; the entry
        carries ``shape`` and ``encoding`` (and ``group_size``)."""
        t = self._entry(name)
        info = self._lookup(name)
        meta = t if self.kind is TARGET_PACK else {**t, "encoding": Q4.name, "group_size": self.group_size}
        return (self._view(info.data or 0, info.data_bytes), self._view(info.scales or 0, info.scale_bytes), meta)

    def tensor(self, name: str) -> TargetTensor:
        data, scales, meta = self.tensor_views(name)
        try:
            return TargetTensor(tuple(meta["shape"]), meta["encoding"], bytes(data), bytes(scales),
                                meta["group_size"] if ENCODINGS[meta["encoding"]].grouped else None)
        finally:
            data.release()
            scales.release()

    def tensor_q4(self, name: str) -> Q4Tensor:
        t = self.tensor(name)
        if t.encoding != Q4.name:
            raise ContractError(f"tensor {name!r} is {t.encoding}, not Q4")
        return Q4Tensor(t.shape, int(t.group_size), t.data, t.scales)

    def layer_encoding(self, layer_index: int) -> str:
        if self._closed:
            raise ContractError(f"{self.kind.label} is closed")
        enc = ctypes.c_int32()
        self._check(self._lib.uqm_pack_layer_encoding(self._handle, int(layer_index), ctypes.byref(enc)),
                    "uqm_pack_layer_encoding")
        return _ENCODING_NAMES[enc.value]

    def names(self) -> list[str]:
        return list(self._index)

    def stage_projection(self, layer_index: int, projection: str, num_experts: int, data_dst: int,
                         scales_dst: int, stream: int) -> None:
        """Copies ``projection`` of experts 0..num_experts-1 of one layer to
        the device addresses given (data expert-major, scales expert-major)
        through the reader's pinned buffers; returns when the copies are done."""
        if self._closed:
            raise ContractError(f"{self.kind.label} is closed")
        self._check(self._lib.uqm_pack_stage_projection(self._handle, int(layer_index), _PROJECTION_IDS[projection],
                                                        int(num_experts), data_dst, scales_dst or None, stream),
                    "uqm_pack_stage_projection")

    def _release(self) -> None:
        if self._handle is not None:
            self._lib.uqm_pack_close(self._handle)
            self._handle = None

    def close(self) -> None:
        """Closes the pack; the mapping is released now, or when the last
        view handed out is released."""
        if self._closed:
            return
        self._closed = True
        if self._live_views == 0:
            self._release()

    def __del__(self) -> None:
        if getattr(self, "_handle", None) is not None and getattr(self, "_live_views", 0) == 0:
            self._release()

    def __enter__(self):
        return self

    def __exit__(self, *_exc: Any) -> None:
        self.close()


class ExpertPackReader(PackReader):
    """A validated all-Q4 ExpertPack (src/uma_qmoe/expert_pack.py:317-556)."""

    kind = EXPERT_PACK


class TargetPackReader(PackReader):
    """A validated mixed TargetPack (src/uma_qmoe/target_pack.py:493-812)."""

    kind = TARGET_PACK


def open_pack(path: str | Path, **expected: Any) -> PackReader:
    """Opens either kind, chosen by the file's magic."""
    with Path(path).open("rb") as f:
        magic = f.read(8)
    cls = {EXPERT_MAGIC: ExpertPackReader, TARGET_MAGIC: TargetPackReader}.get(magic)
    if cls is None:
        raise ContractError("pack magic/version mismatch")
    if cls is ExpertPackReader:
        expected.pop("expected_policy_id", None)
    return cls(path, **expected)


def inspect_pack(path: str | Path) -> dict[str, Any]:
    """Verified manifest record of a pack file (src/uma_qmoe/expert_pack.py:559-582)."""
    source = Path(path)
    with source.open("rb") as f:
        prefix = PREFIX.unpack(f.read(PREFIX.size))
    with open_pack(source) as reader:
        header = reader.header
        kind = reader.kind
        poff, plen = reader.payload_offset, reader.payload_length
    digest = hashlib.sha256()
    with source.open("rb") as f:
        while chunk := f.read(1 << 23):
            digest.update(chunk)
    return {
        "schema_version": 1,
        "kind": "expert_pack_manifest" if kind is EXPERT_PACK else "target_pack_manifest",
        "status": "verified",
        "artifact": {"path": source.name, "size_bytes": source.stat().st_size, "sha256": digest.hexdigest()},
        "header_sha256": prefix[5].hex(),
        "payload_sha256": prefix[6].hex(),
        "payload_offset": poff,
        "payload_length": plen,
        "header": header,
    }


# ----------------------------------------------------------- in memory --
@dataclass
class MemoryTargetPack:
    """Encoded tensors held in memory behind the pack-reader interface
    (``mapping_count``, ``tensor_views``, ``tensor``, ``tensor_q4``,
    ``layer_encoding``, ``close``); ``layer_encodings`` maps a layer index to
    the encoding of its routed experts."""

    tensors: dict[str, TargetTensor]
    layer_encodings: dict[int, str]
    model: dict[str, Any] = field(default_factory=dict)
    mapping_count: int = 1
    closed: bool = False

    @property
    def header(self) -> dict[str, Any]:
        return {"model": dict(self.model)}

    def _get(self, name: str) -> TargetTensor:
        if self.closed:
            raise ContractError("TargetPack is closed")
        try:
            return self.tensors[name]
        except KeyError:
            raise ContractError(f"TargetPack has no tensor {name!r}") from None

    def tensor(self, name: str) -> TargetTensor:
        return self._get(name)

    def tensor_views(self, name: str) -> tuple[memoryview, memoryview, dict[str, Any]]:
        t = self._get(name)
        return memoryview(t.data), memoryview(t.scales), {"shape": list(t.shape), "encoding": t.encoding,
                                                          "group_size": t.group_size}

    def tensor_q4(self, name: str) -> Q4Tensor:
        t = self._get(name)
        if t.encoding != Q4.name:
            raise ContractError(f"tensor {name!r} is {t.encoding}, not Q4")
        return Q4Tensor(t.shape, int(t.group_size or GROUP_SIZE), t.data, t.scales)

    def layer_encoding(self, layer_index: int) -> str:
        try:
            return self.layer_encodings[int(layer_index)]
        except KeyError:
            raise ContractError(f"TargetPack has no layer {layer_index}") from None

    def names(self) -> list[str]:
        return list(self.tensors)

    def close(self) -> None:
        self.closed = True


def memory_pack(tensors: Mapping[str, TargetTensor], layer_encodings: Mapping[int, str], **model: Any) -> MemoryTargetPack:
    for name, t in tensors.items():
        encoding(t.encoding)
    return MemoryTargetPack(dict(tensors), {int(k): v for k, v in layer_encodings.items()}, dict(model))


__all__ = [
    "EXPERT_MAGIC",
    "HEADER_ALIGNMENT",
    "PREFIX",
    "TARGET_MAGIC",
    "TENSOR_ALIGNMENT",
    "ExpertPackReader",
    "MemoryTargetPack",
    "PackReader",
    "TargetPackReader",
    "canonical_json",
    "inspect_pack",
    "memory_pack",
    "model_identity",
    "open_pack",
    "write_expert_pack",
    "write_target_pack",
]
