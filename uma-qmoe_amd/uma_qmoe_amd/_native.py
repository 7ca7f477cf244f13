"""ctypes binding of libuma_qmoe_hip.so (the C ABI in include/uma_qmoe_hip.h and
include/uma_qmoe_pack.h).

Loading never falls back to anything: if the library is missing or was built
for another ABI, :func:`library` raises. Build it with
``python -m uma_qmoe_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from .build import LIB_PATH

ABI_VERSION = 1

UQM_Q4 = 0
UQM_Q8 = 1
UQM_BF16 = 2

UQM_OPT_FUSED_DECODE = 1
UQM_OPT_MFMA_MIN_TOKENS = 3
NOALLOC_SCRATCH_BYTES = 16 << 20  # UQM_NOALLOC_SCRATCH_BYTES
UQM_OPT_OVERLAP_SHARED = 4
UQM_OPT_STREAM_MAX_ROUTES = 5
UQM_OPT_FUSED_WAIT_US = 6  # fused kernel's wait budget in microseconds (0: every wait gives up at once)
FUSED_WAIT_US_DEFAULT = 2000

ENCODING_IDS = {"q4_group128": UQM_Q4, "q8_group128": UQM_Q8, "bf16_le": UQM_BF16}

UQM_ERR_PACK = 5
ERROR_NAMES = {1: "argument", 2: "hip", 3: "device", 4: "workspace", UQM_ERR_PACK: "pack"}

_LOCK = threading.Lock()
_LIB = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32


class ExpertWeights(ctypes.Structure):
    """uqm_expert_weights."""

    _fields_ = [
        ("encoding", _i32),
        ("group_size", _i32),
        ("num_experts", _i64),
        ("hidden_size", _i64),
        ("intermediate_size", _i64),
        ("gate", _vp),
        ("gate_scales", _vp),
        ("up", _vp),
        ("up_scales", _vp),
        ("down", _vp),
        ("down_scales", _vp),
    ]


class LayerWeights(ctypes.Structure):
    """uqm_layer_weights."""

    _fields_ = [
        ("experts", ExpertWeights),
        ("router", _vp),
        ("top_k", _i64),
        ("norm_topk_prob", _i32),
        ("has_shared", _i32),
        ("shared_intermediate_size", _i64),
        ("shared_gate", _vp),
        ("shared_up", _vp),
        ("shared_down", _vp),
        ("shared_expert_gate", _vp),
    ]


class PackTensor(ctypes.Structure):
    """uqm_pack_tensor."""

    _fields_ = [
        ("data", _vp),
        ("data_bytes", ctypes.c_uint64),
        ("scales", _vp),
        ("scale_bytes", ctypes.c_uint64),
        ("element_count", _i64),
        ("shape", _i64 * 4),
        ("ndim", _i32),
        ("encoding", _i32),
        ("group_size", _i32),
        ("reserved", _i32),
    ]


_cp = ctypes.c_char_p
_u64p = ctypes.POINTER(ctypes.c_uint64)
_i32p = ctypes.POINTER(_i32)

# name -> (restype, argtypes)
SIGNATURES = {
    "uqm_abi_version": (ctypes.c_int, ()),
    "uqm_last_error": (ctypes.c_char_p, ()),
    "uqm_device_arch": (ctypes.c_int, (ctypes.c_int, ctypes.c_char_p, ctypes.c_int)),
    "uqm_moe_workspace_bytes": (ctypes.c_size_t, (_i64, _i64, _i64, _i64, _i64, _i64)),
    "uqm_q4_linear": (ctypes.c_int, (_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp)),
    "uqm_q8_linear": (ctypes.c_int, (_vp, _i64, _vp, _vp, _i64, _i64, _i64, _vp, _vp)),
    "uqm_bf16_linear": (ctypes.c_int, (_vp, _i64, _vp, _i64, _i64, _vp, _vp)),
    "uqm_route_permute": (ctypes.c_int, (_vp, _i64, _i64, _i64, _vp, _vp, _vp, ctypes.c_size_t, _vp)),
    "uqm_router_topk": (
        ctypes.c_int,
        (_vp, _i64, _i64, _vp, _i64, _i64, _i32, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp),
    ),
    "uqm_moe_forward": (
        ctypes.c_int,
        (ctypes.POINTER(ExpertWeights), _vp, _i64, _vp, _vp, _i64, _vp, _vp, ctypes.c_size_t, _vp),
    ),
    "uqm_moe_layer": (
        ctypes.c_int,
        (ctypes.POINTER(LayerWeights), _vp, _i64, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp),
    ),
    "uqm_moe_layer_noalloc": (
        ctypes.c_int,
        (ctypes.POINTER(LayerWeights), _vp, _i64, _vp, _vp, _vp, _vp, _vp),
    ),
    "uqm_norm_moe_layer": (
        ctypes.c_int,
        (ctypes.POINTER(LayerWeights), _vp, _i64, _vp, ctypes.c_float, _vp, _vp, _vp, _vp, _vp, ctypes.c_size_t, _vp),
    ),
    "uqm_rmsnorm": (ctypes.c_int, (_vp, _i64, _i64, _vp, ctypes.c_float, _vp, _vp)),
    "uqm_dequantize": (ctypes.c_int, (_i32, _vp, _vp, _i64, _i64, _vp, _vp)),
    "uqm_set_option": (ctypes.c_int, (ctypes.c_int, _i64)),
    "uqm_workspace_status": (ctypes.c_int, (_vp, ctypes.c_size_t, _vp)),
    "uqm_noalloc_status": (ctypes.c_int, (_vp,)),
    "uqm_pack_open": (ctypes.c_int, (_cp, _i32, _cp, _cp, _cp, _cp, ctypes.POINTER(_vp))),
    "uqm_pack_close": (ctypes.c_int, (_vp,)),
    "uqm_pack_info": (ctypes.c_int, (_vp, _i32p, _u64p, _u64p, _i32p)),
    "uqm_pack_header": (ctypes.c_int, (_vp, ctypes.POINTER(_cp), ctypes.POINTER(ctypes.c_size_t))),
    "uqm_pack_lookup": (ctypes.c_int, (_vp, _cp, ctypes.POINTER(PackTensor))),
    "uqm_pack_layer_encoding": (ctypes.c_int, (_vp, _i64, _i32p)),
    "uqm_pack_stage_projection": (ctypes.c_int, (_vp, _i64, _i32, _i64, _vp, _vp, _vp)),
}


class NativeError(RuntimeError):
    """A nonzero status from the HIP library (surfaced as RuntimeError, like the
    reference binding's TORCH_CHECK)."""


def library_path() -> Path:
    return LIB_PATH


def library():
    """Load (once) and return the ctypes handle; raises if unavailable."""
    global _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        path = library_path()
        if not path.is_file():
            raise RuntimeError(
                f"libuma_qmoe_hip.so is not built ({path}); run python -m uma_qmoe_amd.build"
            )
        lib = ctypes.CDLL(str(path))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.uqm_abi_version()
        if version != ABI_VERSION:
            raise RuntimeError(f"libuma_qmoe_hip ABI {version} does not match the host's {ABI_VERSION}")
        _LIB = lib
        return lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        message = library().uqm_last_error().decode("utf-8", "replace")
        kind = ERROR_NAMES.get(rc, str(rc))
        raise NativeError(f"{what} failed ({kind} error): {message}")


def exported_symbols() -> list[str]:
    return sorted(SIGNATURES)
