"""The C++ pack reader under AddressSanitizer and UBSan (host code, CPU):
tests/pack_reader_harness.cpp and csrc/uqm_pack.cpp built with g++
-fsanitize=address,undefined open a valid pack and several hundred corrupted
copies (random byte edits anywhere in the file, truncations, headers with
valid hashes and random edits), read every byte of every tensor they accept,
and must finish without a sanitizer report; each file is accepted or refused
exactly as the library build decides."""

from __future__ import annotations

import hashlib
import json
import os
from pathlib import Path
import random
import shutil
import subprocess

import numpy as np
import pytest

from uma_qmoe_amd.formats import ContractError
from uma_qmoe_amd.packfile import PREFIX, ExpertPackReader, write_expert_pack, write_target_pack

ROOT = Path(__file__).resolve().parent.parent
OLMOE = "allenai/OLMoE-1B-7B-0125"


def _build(tmp: Path) -> Path:
    if shutil.which("g++") is None or not Path("/opt/rocm/lib/libamdhip64.so").exists():
        pytest.skip("g++ or the HIP runtime library is not available")
    exe = tmp / "harness"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-omit-frame-pointer",
           "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include", str(ROOT / "tests" / "pack_reader_harness.cpp"),
           str(ROOT / "uma-qmoe_amd" / "csrc" / "uqm_pack.cpp"), "-o", str(exe), "-L/opt/rocm/lib", "-lamdhip64",
           "-lcrypto", "-lpthread", "-Wl,-rpath,/opt/rocm/lib"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        pytest.skip(f"sanitizer build unavailable: {proc.stderr[-400:]}")
    return exe


def _corpus(tmp: Path, seed: int = 5) -> list[Path]:
    rng = random.Random(seed)
    base = tmp / "valid.uqep"
    write_expert_pack(base, [("a.gate", np.linspace(-2, 2, 257, dtype=np.float32).reshape(1, 257)),
                             ("b.down", np.linspace(1, -1, 129, dtype=np.float32))],
                      model_id=OLMOE, model_revision="a" * 40, model_manifest_sha256="b" * 64)
    target = tmp / "valid.uqtp"
    write_target_pack(target, [("model.layers.8.mlp.experts.1.up_proj.weight", np.ones((1, 257), np.float32))],
                      model_id=OLMOE, model_revision="a" * 40, model_manifest_sha256="b" * 64, policy_id="p",
                      layer_encodings={i: "q8_group128" if i == 8 else "bf16_le" for i in range(16)},
                      policy_evidence_sha256="c" * 64)
    files = [base, target]
    raw = base.read_bytes()
    hlen, poff = PREFIX.unpack_from(raw)[2:4]
    for i in range(120):  # random byte edits anywhere
        b = bytearray(raw)
        for _ in range(rng.randint(1, 6)):
            b[rng.randrange(len(b))] = rng.randrange(256)
        files.append(tmp / f"edit{i}.uqep")
        files[-1].write_bytes(b)
    for i, cut in enumerate((0, 1, 95, 96, 100, poff - 1, poff, len(raw) - 1)):  # truncations
        files.append(tmp / f"cut{i}.uqep")
        files[-1].write_bytes(raw[:cut])
    for i in range(200):  # header edits with valid header hash (the parser sees them)
        hb = bytearray(raw[96:96 + hlen])
        for _ in range(rng.randint(1, 4)):
            at = rng.randrange(len(hb))
            if rng.random() < 0.5:
                hb[at] = rng.choice(b'{}[]",:0123456789-.eE \\tnulrfasu' + bytes([rng.randrange(256)]))
            elif rng.random() < 0.5:
                del hb[at]
            else:
                hb.insert(at, rng.randrange(256))
        fields = list(PREFIX.unpack_from(raw))
        fields[2], fields[5] = len(hb), hashlib.sha256(hb).digest()
        if 96 + len(hb) > poff:
            continue
        out = bytes(PREFIX.pack(*fields)) + bytes(hb) + bytes(poff - 96 - len(hb)) + raw[poff:]
        files.append(tmp / f"hdr{i}.uqep")
        files[-1].write_bytes(out)
    # deep nesting and long strings in an otherwise valid header
    header = json.loads(raw[96:96 + hlen])
    for i, extra in enumerate(([[[[[[[[[[1]]]]]]]]]], "x" * 900, {"é\U0001F600": [1.5e300, -0.0, 5e-324]})):
        hb = json.dumps({**header, "extra": extra}, sort_keys=True, separators=(",", ":")).encode()
        fields = list(PREFIX.unpack_from(raw))
        fields[2], fields[5] = len(hb), hashlib.sha256(hb).digest()
        files.append(tmp / f"deep{i}.uqep")
        files[-1].write_bytes(bytes(PREFIX.pack(*fields)) + hb + bytes(poff - 96 - len(hb)) + raw[poff:])
    return files


def test_reader_under_sanitizers(tmp_path):
    exe = _build(tmp_path)
    files = _corpus(tmp_path)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", UBSAN_OPTIONS="halt_on_error=1")
    proc = subprocess.run([str(exe), *map(str, files)], capture_output=True, text=True, env=env, timeout=600)
    assert proc.returncode == 0, proc.stderr[-2000:]
    assert "Sanitizer" not in proc.stderr, proc.stderr[-2000:]
    lines = proc.stdout.splitlines()
    assert len(lines) == len(files)
    accepted = 0
    for path, line in zip(files, lines):
        try:
            ExpertPackReader(path).close() if path.suffix == ".uqep" else None
            lib_ok = True
        except ContractError:
            lib_ok = False
        if path.suffix == ".uqep":
            assert line.startswith("ok") == lib_ok, (path.name, line)
        accepted += line.startswith("ok")
    assert lines[0].startswith("ok 2") and lines[1].startswith("ok 1")
    assert accepted >= 5  # the valid files and the well-formed extras
