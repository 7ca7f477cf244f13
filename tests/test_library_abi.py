"""The C-ABI library loads and exports every entry point include/*.h declares
(no compute calls: this runs without a GPU)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

from uma_qmoe_amd import _native

INCLUDE = Path(__file__).resolve().parent.parent / "include"
HEADER = INCLUDE / "uma_qmoe_hip.h"


def declared_functions() -> list[str]:
    text = "".join(h.read_text() for h in sorted(INCLUDE.glob("*.h")))
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(uqm_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_bound_functions():
    declared = declared_functions()
    assert declared, "no uqm_* declarations found"
    assert sorted(_native.SIGNATURES) == declared


def test_library_loads_and_exports_every_declared_symbol():
    lib = _native.library()
    for name in declared_functions():
        assert hasattr(lib, name), name
        assert ctypes.cast(getattr(lib, name), ctypes.c_void_p).value
    assert lib.uqm_abi_version() == _native.ABI_VERSION


def test_workspace_query_is_host_only_and_validates():
    lib = _native.library()
    n = lib.uqm_moe_workspace_bytes(1, 2048, 1408, 5632, 60, 4)
    assert n > 0 and n % 256 == 0
    assert lib.uqm_moe_workspace_bytes(-1, 2048, 1408, 0, 60, 4) == 0
    assert lib.uqm_moe_workspace_bytes(512, 2048, 1408, 5632, 60, 4) > n


def test_struct_layouts_match_header():
    # uqm_expert_weights: 2 x int32, 3 x int64, 6 pointers
    assert ctypes.sizeof(_native.ExpertWeights) == 8 + 3 * 8 + 6 * 8
    assert ctypes.sizeof(_native.LayerWeights) == ctypes.sizeof(_native.ExpertWeights) + 8 + 8 + 4 + 4 + 8 + 4 * 8


def header_enum_values(header: Path = HEADER) -> dict[str, int]:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    values = {}
    for body in re.findall(r"enum\s*\{(.*?)\}", text, flags=re.S):
        for name, value in re.findall(r"\b(UQM_[A-Z0-9_]+)\s*=\s*(\d+)", body):
            values[name] = int(value)
    return values


def test_python_constants_match_header_enums():
    values = header_enum_values()
    for name in ("UQM_Q4", "UQM_Q8", "UQM_BF16", "UQM_OPT_FUSED_DECODE",
                 "UQM_OPT_MFMA_MIN_TOKENS", "UQM_OPT_OVERLAP_SHARED", "UQM_OPT_STREAM_MAX_ROUTES",
                 "UQM_OPT_FUSED_WAIT_US", "UQM_ERR_PACK"):
        assert values[name] == getattr(_native, name), name
    pack_enums = header_enum_values(INCLUDE / "uma_qmoe_pack.h")
    assert (pack_enums["UQM_PACK_EXPERT"], pack_enums["UQM_PACK_TARGET"]) == (0, 1)
    assert (pack_enums["UQM_PROJ_GATE"], pack_enums["UQM_PROJ_UP"], pack_enums["UQM_PROJ_DOWN"]) == (0, 1, 2)


def test_pack_tensor_struct_layout():
    # uqm_pack_tensor: 2 pointers, 2 x uint64, int64, int64[4], 4 x int32
    assert ctypes.sizeof(_native.PackTensor) == 2 * 8 + 2 * 8 + 8 + 4 * 8 + 4 * 4


def test_set_option_is_host_only_and_validates():
    lib = _native.library()
    assert lib.uqm_set_option(_native.UQM_OPT_OVERLAP_SHARED, 0) == 0
    assert lib.uqm_set_option(_native.UQM_OPT_OVERLAP_SHARED, 1) == 0
    assert lib.uqm_set_option(99, 1) != 0
    assert b"unknown option" in lib.uqm_last_error()
    assert lib.uqm_set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, -1) != 0
    assert lib.uqm_set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, -1) != 0
    assert lib.uqm_set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, 32) == 0  # the default


def test_noalloc_limit_is_checked_on_the_host():
    """UQM_NOALLOC_SCRATCH_BYTES matches the Python constant, and a call whose
    workspace would exceed it is refused before anything touches a device."""
    import ctypes

    text = HEADER.read_text()
    m = re.search(r"#define\s+UQM_NOALLOC_SCRATCH_BYTES\s+\(\(size_t\)(\d+)\s*<<\s*(\d+)\)", text)
    assert m and int(m.group(1)) << int(m.group(2)) == _native.NOALLOC_SCRATCH_BYTES
    lib = _native.library()
    experts = _native.ExpertWeights(_native.UQM_Q4, 128, 60, 2048, 1408, 16, 16, 16, 16, 16, 16)
    layer = _native.LayerWeights(experts, 16, 4, 0, 1, 5632, 16, 16, 16, 16)
    need = lib.uqm_moe_workspace_bytes(1000, 2048, 1408, 5632, 60, 4)
    assert need > _native.NOALLOC_SCRATCH_BYTES
    rc = lib.uqm_moe_layer_noalloc(ctypes.byref(layer), 16, 1000, 16, None, None, None, None)
    assert rc == 4  # UQM_ERR_WORKSPACE
    assert b"uqm_moe_layer_noalloc" in lib.uqm_last_error() and b"workspace" in lib.uqm_last_error()
    assert lib.uqm_moe_layer_noalloc(None, 16, 1, 16, None, None, None, None) == 1
