"""The C++ pack reader on arbitrary input (CPU): random JSON values and
random byte edits of a valid header, with the header hash rewritten so the
parser sees them. The reader must accept exactly the headers that are
Python's canonical JSON of their own value (and otherwise valid), and refuse
everything else with ContractError, never crash."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import HealthCheck, given, settings, strategies as st  # noqa: E402

from uma_qmoe_amd.formats import ContractError  # noqa: E402
from uma_qmoe_amd.packfile import PREFIX, ExpertPackReader, write_expert_pack  # noqa: E402

OLMOE = "allenai/OLMoE-1B-7B-0125"


@pytest.fixture(scope="module")
def pack(tmp_path_factory) -> Path:
    path = tmp_path_factory.mktemp("fuzz") / "experts.uqep"
    write_expert_pack(path, [("a.gate", np.linspace(-2, 2, 257, dtype=np.float32).reshape(1, 257))],
                      model_id=OLMOE, model_revision="a" * 40, model_manifest_sha256="b" * 64)
    return path


def with_header(path: Path, hb: bytes, name: str) -> Path:
    raw = bytearray(path.read_bytes())
    fields = list(PREFIX.unpack_from(raw))
    poff = fields[3]
    assert 96 + len(hb) <= poff
    fields[2], fields[5] = len(hb), hashlib.sha256(hb).digest()
    out = path.with_name(name)
    out.write_bytes(bytes(PREFIX.pack(*fields)) + hb + bytes(poff - 96 - len(hb)) + bytes(raw[poff:]))
    return out


def canonical(value) -> bytes:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False).encode()


json_values = st.recursive(
    st.none() | st.booleans() | st.integers(min_value=-(2 ** 63), max_value=2 ** 63 - 1)
    | st.floats(allow_nan=False, allow_infinity=False) | st.text(max_size=12),
    lambda children: st.lists(children, max_size=4) | st.dictionaries(st.text(max_size=6), children, max_size=4),
    max_leaves=12,
)


@settings(max_examples=150, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(extra=json_values)
def test_any_canonical_value_is_accepted(pack, extra):
    """Extra header content in Python's canonical form reads back equal."""
    header = json.loads(pack.read_bytes()[96:96 + PREFIX.unpack_from(pack.read_bytes())[2]])
    header["extra"] = extra
    path = with_header(pack, canonical(header), "canon.uqep")
    with ExpertPackReader(path) as reader:
        assert reader.header["extra"] == json.loads(canonical(extra))


@settings(max_examples=300, deadline=None, suppress_health_check=[HealthCheck.function_scoped_fixture])
@given(data=st.data())
def test_random_header_edits_never_crash(pack, data):
    raw = pack.read_bytes()
    hlen = PREFIX.unpack_from(raw)[2]
    hb = bytearray(raw[96:96 + hlen])
    for _ in range(data.draw(st.integers(1, 4))):
        op = data.draw(st.sampled_from(["flip", "insert", "delete"]))
        at = data.draw(st.integers(0, len(hb) - 1))
        if op == "flip":
            hb[at] = data.draw(st.integers(0, 255))
        elif op == "insert":
            hb.insert(at, data.draw(st.integers(0, 255)))
        elif len(hb) > 1:
            del hb[at]
    path = with_header(pack, bytes(hb), "edit.uqep")
    try:
        value = json.loads(bytes(hb))
        is_canonical = isinstance(value, dict) and canonical(value) == bytes(hb)
    except (ValueError, UnicodeDecodeError):
        is_canonical = False
    try:
        with ExpertPackReader(path) as reader:
            accepted = reader.header
    except ContractError as exc:
        accepted = None
        if not is_canonical:
            assert "canonical" in str(exc)
    if accepted is not None:
        assert is_canonical and accepted == json.loads(bytes(hb))
