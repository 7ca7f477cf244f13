"""TEST INFRASTRUCTURE ONLY: ctypes wrapper over the oracle's C codec (codec.c).

Restates src/uma_qmoe/q4.py:96-179 and src/uma_qmoe/target_pack.py:78-175 of
the reference. The product never imports this module.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "liboracle_codec.so"
_LIB = None

ERRORS = {
    1: "value outside the codec range or reserved -8 code",
    2: "nonzero odd tail padding nibble",
    3: "scales must be finite and positive",
    4: "invalid argument",
}


class CodecError(ValueError):
    pass


def build() -> Path:
    """Compile codec.c with the committed Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def _lib():
    global _LIB
    if _LIB is None:
        if not _LIB_PATH.is_file():
            build()
        lib = ctypes.CDLL(str(_LIB_PATH))
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        for name, args in {
            "orc_q4_pack": (p, i64, p),
            "orc_q4_unpack": (p, i64, p),
            "orc_q4_quantize": (p, i64, i64, p, p, p),
            "orc_q4_dequantize": (p, p, i64, i64, p, p),
            "orc_q8_quantize": (p, i64, i64, p, p),
            "orc_q8_dequantize": (p, p, i64, i64, p),
        }.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        for name in ("orc_f32_to_bf16", "orc_bf16_to_f32"):
            fn = getattr(lib, name)
            fn.argtypes = (p, i64, p)
            fn.restype = None
        _LIB = lib
    return _LIB


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _check(rc: int) -> None:
    if rc:
        raise CodecError(ERRORS.get(rc, f"codec error {rc}"))


def q4_pack(values) -> bytes:
    v = np.ascontiguousarray(np.asarray(values).reshape(-1).astype(np.int8))
    out = np.zeros((v.size + 1) // 2, dtype=np.uint8)
    _check(_lib().orc_q4_pack(_ptr(v), v.size, _ptr(out)))
    return out.tobytes()


def q4_unpack(payload, n: int) -> np.ndarray:
    raw = np.frombuffer(bytes(payload), dtype=np.uint8)
    if raw.size != (n + 1) // 2:
        raise CodecError("Q4 packed byte count does not match element count")
    out = np.empty(n, dtype=np.int8)
    _check(_lib().orc_q4_unpack(_ptr(raw), n, _ptr(out)))
    return out


def q4_quantize(values, group: int = 128) -> tuple[bytes, bytes]:
    """Return (packed bytes, little-endian f32 scale bytes)."""
    src = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
    n = src.size
    q = np.empty(n, dtype=np.int8)
    packed = np.empty((n + 1) // 2, dtype=np.uint8)
    scales = np.empty((n + group - 1) // group, dtype="<f4")
    _check(_lib().orc_q4_quantize(_ptr(src), n, group, _ptr(q), _ptr(packed), _ptr(scales)))
    return packed.tobytes(), scales.tobytes()


def q4_dequantize(packed, scales, shape, group: int = 128) -> np.ndarray:
    n = int(np.prod(shape))
    raw = np.frombuffer(bytes(packed), dtype=np.uint8)
    sc = np.frombuffer(bytes(scales), dtype="<f4")
    if raw.size != (n + 1) // 2 or sc.size != (n + group - 1) // group:
        raise CodecError("Q4 tensor payload lengths do not match layout")
    q = np.empty(n, dtype=np.int8)
    out = np.empty(n, dtype=np.float32)
    _check(_lib().orc_q4_dequantize(_ptr(raw), _ptr(sc), n, group, _ptr(q), _ptr(out)))
    return out.reshape(shape)


def q8_quantize(values, group: int = 128) -> tuple[bytes, bytes]:
    src = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
    n = src.size
    q = np.empty(n, dtype=np.int8)
    scales = np.empty((n + group - 1) // group, dtype="<f4")
    _check(_lib().orc_q8_quantize(_ptr(src), n, group, _ptr(q), _ptr(scales)))
    return q.tobytes(), scales.tobytes()


def q8_dequantize(data, scales, shape, group: int = 128) -> np.ndarray:
    n = int(np.prod(shape))
    q = np.frombuffer(bytes(data), dtype=np.int8)
    sc = np.frombuffer(bytes(scales), dtype="<f4")
    if q.size != n or sc.size != (n + group - 1) // group:
        raise CodecError("Q8 TargetTensor payload lengths are invalid")
    out = np.empty(n, dtype=np.float32)
    _check(_lib().orc_q8_dequantize(_ptr(np.ascontiguousarray(q)), _ptr(sc), n, group, _ptr(out)))
    return out.reshape(shape)


def f32_to_bf16_bits(values) -> np.ndarray:
    src = np.ascontiguousarray(np.asarray(values, dtype=np.float32).reshape(-1))
    out = np.empty(src.size, dtype=np.uint16)
    _lib().orc_f32_to_bf16(_ptr(src), src.size, _ptr(out))
    return out


def bf16_bits_to_f32(bits, shape=None) -> np.ndarray:
    src = np.ascontiguousarray(np.asarray(bits, dtype=np.uint16).reshape(-1))
    out = np.empty(src.size, dtype=np.float32)
    _lib().orc_bf16_to_f32(_ptr(src), src.size, _ptr(out))
    return out.reshape(shape) if shape is not None else out


def decode_tensor(data, scales, metadata) -> np.ndarray:
    """Decode one stored tensor to float32 by its explicit encoding.

    Follows decode_target_tensor, src/uma_qmoe/target_pack.py:144-176.
    """
    shape = tuple(int(v) for v in metadata["shape"])
    encoding = metadata["encoding"]
    if encoding == "q4_group128":
        return q4_dequantize(data, scales, shape, int(metadata.get("group_size", 128)))
    if encoding == "q8_group128":
        return q8_dequantize(data, scales, shape, int(metadata.get("group_size", 128)))
    if encoding == "bf16_le":
        if len(bytes(scales)):
            raise CodecError("BF16 TargetTensor layout is invalid")
        bits = np.frombuffer(bytes(data), dtype="<u2")
        if bits.size != int(np.prod(shape)):
            raise CodecError("BF16 TargetTensor layout is invalid")
        return bf16_bits_to_f32(bits, shape)
    raise CodecError(f"unsupported TargetTensor encoding {encoding!r}")
