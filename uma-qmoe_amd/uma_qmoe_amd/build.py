"""Builds libuma_qmoe_hip.so for gfx950 with hipcc (in-tree, no JIT cache).

Each ``csrc/*.hip`` translation unit (hipcc) and each host-only
``csrc/*.cpp`` one (g++) is compiled in parallel to an object under
``_build/`` and linked into ``uma-qmoe_amd/lib/libuma_qmoe_hip.so``;
each ``csrc/timeline/NAME.hip`` (the per-phase timeline of the fused kernel
and the grouped-GEMM counter program, both used to take rocprofv3 counters
on a few hundred dispatches) becomes the program ``uma-qmoe_amd/lib/NAME``.
Run as ``python -m uma_qmoe_amd.build`` with ``uma-qmoe_amd`` on sys.path.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent.parent  # uma-qmoe_amd/
CSRC = PACKAGE_ROOT / "csrc"
BUILD_DIR = PACKAGE_ROOT / "_build"
LIB_DIR = PACKAGE_ROOT / "lib"
LIB_PATH = LIB_DIR / "libuma_qmoe_hip.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Keep the compiler from emitting packed FP32 (v_pk_*_f32) instructions.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


CXX = os.environ.get("CXX", "g++")
# Host-only translation units (the pack reader): plain C++ against the HIP
# runtime API, linked with OpenSSL's libcrypto for SHA-256.
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include"]
LINK_LIBS = ["-lcrypto", "-lpthread"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    if src.suffix == ".cpp":
        cmd = [CXX, *HOST_FLAGS, "-c", str(src), "-o", str(obj)]
    else:
        cmd = [HIPCC, *COMMON_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compilation failed for {src.name}:\n{proc.stderr}")
    return obj


PROGRAMS = CSRC / "timeline"
# Programs that call the library through its C ABI (linked against it, so
# built after it); the others include the kernel sources they measure.
LINKED_PROGRAMS = {"grouped_counters"}


def _compile_program(src: Path) -> Path:
    """A stand-alone counter program (csrc/timeline/NAME.hip) -> lib/NAME."""
    out = LIB_DIR / src.stem
    tmp = out.with_suffix(".tmp")
    cmd = [HIPCC, *[f for f in COMMON_FLAGS if f != "-fPIC"], str(src), "-o", str(tmp)]
    if src.stem in LINKED_PROGRAMS:
        cmd += [f"-L{LIB_DIR}", "-luma_qmoe_hip", "-Wl,-rpath,$ORIGIN"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> Path:
    """Compile every HIP source, link the shared library and build the
    counter programs. Always rebuilds."""
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = min(len(srcs) + 1, max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        programs = sorted(PROGRAMS.glob("*.hip"))
        extras = [pool.submit(_compile_program, p) for p in programs if p.stem not in LINKED_PROGRAMS]
        objs = list(pool.map(_compile, srcs))
        for e in extras:
            e.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), *LINK_LIBS, "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    for p in programs:
        if p.stem in LINKED_PROGRAMS:
            _compile_program(p)
    if verbose:
        print(f"built {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
