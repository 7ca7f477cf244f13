"""The C++ pack reader (csrc/uqm_pack.cpp) on the CPU: every check of the
format, each provoked on its own with every hash rewritten so that only that
check can catch it, against the message the reference's readers raise
(src/uma_qmoe/expert_pack.py:317-556, src/uma_qmoe/target_pack.py:493-812);
the order in which violations are reported; and the canonical-JSON rule,
checked against Python's own json.dumps on values that exercise every
formatting case (float forms, escapes, key order)."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
import struct

import numpy as np
import pytest

from uma_qmoe_amd.formats import ContractError
from uma_qmoe_amd.packfile import PREFIX, ExpertPackReader, TargetPackReader, open_pack, write_expert_pack, write_target_pack

OLMOE = "allenai/OLMoE-1B-7B-0125"
IDS = dict(model_revision="a" * 40, model_manifest_sha256="b" * 64)
POLICY = {layer: ("q4_group128" if layer == 15 else "q8_group128" if layer == 8 else "bf16_le") for layer in range(16)}


def canonical(value) -> bytes:
    return json.dumps(value, sort_keys=True, separators=(",", ":"), allow_nan=False).encode("utf-8")


@pytest.fixture
def expert_pack(tmp_path):
    path = tmp_path / "experts.uqep"
    write_expert_pack(path, [("a.gate", np.linspace(-2, 2, 257, dtype=np.float32).reshape(1, 257)),
                             ("b.down", np.linspace(1, -1, 129, dtype=np.float32))], model_id=OLMOE, **IDS)
    return path


@pytest.fixture
def target_pack(tmp_path):
    path = tmp_path / "experts.uqtp"
    write_target_pack(path, [("model.layers.0.mlp.experts.0.gate_proj.weight", np.ones((2, 129), np.float32)),
                             ("model.layers.8.mlp.experts.1.up_proj.weight", np.ones((1, 257), np.float32)),
                             ("model.layers.15.mlp.experts.2.down_proj.weight", np.ones((1, 129), np.float32))],
                      model_id=OLMOE, **IDS, policy_id="p", layer_encodings=POLICY, policy_evidence_sha256="c" * 64)
    return path


def rewrite(path: Path, *, header=None, header_bytes=None, payload=None, prefix=None, rehash=True) -> Path:
    """A copy of the pack with the header (a dict, or raw bytes), payload or
    prefix fields replaced; the header and payload hashes are recomputed
    unless ``rehash`` is False."""
    raw = bytearray(path.read_bytes())
    fields = list(PREFIX.unpack_from(raw))
    hlen, poff = fields[2], fields[3]
    hb = bytes(raw[96:96 + hlen])
    body = bytes(raw[poff:])
    if header is not None:
        hb = canonical(header(json.loads(hb)))
    if header_bytes is not None:
        hb = header_bytes(hb)
    if payload is not None:
        body = bytes(payload(bytearray(body), json.loads(hb)))
    assert 96 + len(hb) <= poff, "the test header no longer fits before the payload"
    fields[2], fields[4] = len(hb), len(body)
    if rehash:
        fields[5], fields[6] = hashlib.sha256(hb).digest(), hashlib.sha256(body).digest()
    if prefix is not None:
        fields = prefix(fields)
    out = bytearray(PREFIX.pack(*fields)) + hb + bytes(poff - 96 - len(hb)) + body
    dest = path.with_name("rewritten" + path.suffix)
    dest.write_bytes(out)
    return dest


def tensor_hash(payload, t, field="packed"):
    data = payload[t[f"{field}_offset"]:t[f"{field}_offset"] + t[f"{field}_bytes"]]
    scales = payload[t["scale_offset"]:t["scale_offset"] + t["scale_bytes"]]
    return hashlib.sha256(bytes(data) + bytes(scales)).hexdigest()


def set_tensor(i, **fields):
    def f(h):
        h["tensors"][i].update(fields)
        return h
    return f


@pytest.mark.parametrize("mutation,message", [
    (dict(prefix=lambda f: [b"UQMOXPK1", *f[1:]]), "ExpertPack magic/version mismatch"),
    (dict(prefix=lambda f: [f[0], 2, *f[2:]]), "ExpertPack magic/version mismatch"),
    (dict(prefix=lambda f: [*f[:3], f[3] + 8, *f[4:]]), "payload offset/alignment is invalid"),
    (dict(prefix=lambda f: [*f[:4], f[4] - 1, *f[5:]]), "payload length does not match file size"),
    (dict(prefix=lambda f: [*f[:5], bytes(32), f[6]]), "ExpertPack header hash mismatch"),
    (dict(prefix=lambda f: [*f[:6], bytes(32)]), "ExpertPack payload hash mismatch"),
    (dict(header_bytes=lambda hb: hb[:-1]), "ExpertPack header is not canonical JSON"),
    (dict(header_bytes=lambda hb: hb.replace(b'"bits":4', b'"bits": 4')), "ExpertPack header JSON is not canonical"),
    (dict(header_bytes=lambda hb: b"[" + hb + b"]"), "ExpertPack header JSON is not canonical"),
    (dict(header_bytes=lambda hb: hb[:-1] + b',"format":"x"}'), "ExpertPack header JSON is not canonical"),
    (dict(header=lambda h: {**h, "schema_version": 2}), "ExpertPack header schema is unsupported"),
    (dict(header=lambda h: {**h, "format": "mixed_precision_target_pack"}), "ExpertPack header schema is unsupported"),
    (dict(header=lambda h: {k: v for k, v in h.items() if k != "tensors"}), "ExpertPack header is incomplete"),
    (dict(header=lambda h: {**h, "model": {**h["model"], "model_id": "other"}}), "model identity hash mismatch"),
    (dict(header=lambda h: {**h, "quantization": {**h["quantization"], "group_size": True}}),
     "ExpertPack quantization contract mismatch"),
    (dict(header=lambda h: {**h, "quantization": {**h["quantization"], "rounding": "away"}}),
     "ExpertPack quantization contract mismatch"),
    (dict(header=lambda h: {**h, "tensor_alignment_bytes": 48}), "alignment must be a positive power of two"),
    (dict(header=lambda h: {**h, "tensor_count": 3}), "ExpertPack tensor count is inconsistent"),
    (dict(header=set_tensor(1, name="a b")), "ExpertPack tensor names must be unique and safe"),
    (dict(header=set_tensor(1, name="a.gate")), "ExpertPack tensor names must be unique and safe"),
    (dict(header=set_tensor(0, shape=[1, 0])), "ExpertPack tensor 'a.gate' has invalid shape"),
    (dict(header=set_tensor(0, shape=[1, True])), "ExpertPack tensor 'a.gate' has invalid shape"),
    (dict(header=set_tensor(0, element_count=258)), "ExpertPack tensor 'a.gate' layout is invalid"),
    (dict(header=set_tensor(0, group_count=2)), "ExpertPack tensor 'a.gate' layout is invalid"),
    (dict(header=set_tensor(0, scale_offset=136)), "ExpertPack tensor 'a.gate' layout is invalid"),
    (dict(header=set_tensor(1, packed_offset=64)), "ExpertPack tensor 'b.down' layout is invalid"),
    (dict(header=set_tensor(0, effective_bits_per_weight=4.5)), "ExpertPack tensor 'a.gate' effective bpw is invalid"),
    (dict(header=set_tensor(0, tensor_payload_sha256="0" * 64)), "ExpertPack tensor 'a.gate' hash mismatch"),
])
def test_expert_pack_checks(expert_pack, mutation, message):
    with pytest.raises(ContractError, match=message):
        ExpertPackReader(rewrite(expert_pack, **mutation))


def test_numeric_fields_compare_as_python_numbers(expert_pack):
    # a float equal to the integer passes where Python's == says equal
    ok = rewrite(expert_pack, header=set_tensor(0, element_count=257.0))
    with ExpertPackReader(ok) as reader:
        assert reader.tensor("a.gate").element_count == 257


def test_payload_semantics_and_padding(expert_pack):
    # each payload change is rehashed at tensor and payload level
    raw = bytearray(expert_pack.read_bytes())
    hlen, poff = PREFIX.unpack_from(raw)[2:4]
    header = json.loads(raw[96:96 + hlen])
    payload_bytes = bytearray(raw[poff:])
    t = header["tensors"][0]
    for at, value, message in ((3, 0x80, "reserved Q4 -8 code"), (128, 0x10, "non-zero Q4 odd tail padding")):
        p = bytearray(payload_bytes)
        p[t["packed_offset"] + at] = value
        h = json.loads(json.dumps(header))
        h["tensors"][0]["tensor_payload_sha256"] = tensor_hash(p, t)
        with pytest.raises(ContractError, match=f"ExpertPack tensor 'a.gate' (contains the|has) {message}"):
            ExpertPackReader(rewrite(expert_pack, header=lambda _h, h=h: h, payload=lambda _p, _h, p=p: p))
    for scale in (0.0, -1.0, float("inf"), float("nan")):
        p = bytearray(payload_bytes)
        struct.pack_into("<f", p, t["scale_offset"] + 4, scale)
        h = json.loads(json.dumps(header))
        h["tensors"][0]["tensor_payload_sha256"] = tensor_hash(p, t)
        with pytest.raises(ContractError, match="scales must be finite and positive"):
            ExpertPackReader(rewrite(expert_pack, header=lambda _h, h=h: h, payload=lambda _p, _h, p=p: p))
    for at, where in ((t["packed_bytes"], "data-to-scale"), (t["storage_end_offset"] - t["packed_offset"] - 1, "trailing")):
        p = bytearray(payload_bytes)
        p[t["packed_offset"] + at] = 1
        with pytest.raises(ContractError, match=f"tensor 'a.gate' {where} padding must be zero"):
            ExpertPackReader(rewrite(expert_pack, payload=lambda _p, _h, p=p: p))
    # payload bytes no tensor claims
    with pytest.raises(ContractError, match="payload has unclaimed trailing bytes"):
        ExpertPackReader(rewrite(expert_pack, payload=lambda p, _h: p + bytes(64)))
    # header padding is outside both hashes
    bad = bytearray(expert_pack.read_bytes())
    bad[96 + hlen] = 1
    (expert_pack.parent / "pad.uqep").write_bytes(bad)
    with pytest.raises(ContractError, match="ExpertPack header padding must be zero"):
        ExpertPackReader(expert_pack.parent / "pad.uqep")


def test_violations_are_reported_in_the_reference_order(expert_pack):
    # payload hash before an unparsable header
    with pytest.raises(ContractError, match="payload hash mismatch"):
        ExpertPackReader(rewrite(expert_pack, header_bytes=lambda hb: hb[:-1], prefix=lambda f: [*f[:6], bytes(32)]))
    # tensor 0's hash before tensor 1's layout
    with pytest.raises(ContractError, match="tensor 'a.gate' hash mismatch"):
        ExpertPackReader(rewrite(expert_pack, header=lambda h: set_tensor(1, element_count=1)(
            set_tensor(0, tensor_payload_sha256="0" * 64)(h))))
    # a short file
    short = expert_pack.parent / "short.uqep"
    short.write_bytes(expert_pack.read_bytes()[:95])
    with pytest.raises(ContractError, match="pack is shorter than its fixed prefix"):
        ExpertPackReader(short)
    # the wrong kind for the reader class
    with pytest.raises(ContractError, match="TargetPack magic/version mismatch"):
        TargetPackReader(expert_pack)


@pytest.mark.parametrize("mutation,message", [
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "policy_id": ""}}), "TargetPack policy id must be non-empty"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "layer_encodings": {
        k: v for k, v in h["policy"]["layer_encodings"].items() if k != "3"}}}),
     "TargetPack policy must assign every OLMoE layer exactly once"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "layer_encodings": {
        **h["policy"]["layer_encodings"], "3": "fp8"}}}), "TargetPack policy contains an unsupported encoding"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "layer_encodings": {
        **{k: v for k, v in h["policy"]["layer_encodings"].items() if k != "3"}, "x": "bf16_le"}}}),
     "TargetPack layer policy is invalid"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "layer_encodings": {
        **{k: v for k, v in h["policy"]["layer_encodings"].items() if k != "3"}, "03": "bf16_le"}}}),
     "TargetPack policy identity hash mismatch"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "policy_evidence_sha256": "C" * 64}}),
     "TargetPack policy evidence identity must be SHA-256"),
    (dict(header=lambda h: {**h, "policy": {**h["policy"], "policy_identity_sha256": "0" * 64}}),
     "TargetPack policy identity hash mismatch"),
    (dict(header=lambda h: {**h, "encodings": {**h["encodings"], "bf16_le": {"bits": 16}}}),
     "TargetPack encoding contract mismatch"),
    (dict(header=set_tensor(0, layer_index=1)), "TargetPack tensor 'model.layers.0.mlp.experts.0.gate_proj.weight' "
                                               "policy identity is invalid"),
    (dict(header=set_tensor(0, encoding="q8_group128")), "policy identity is invalid"),
    (dict(header=set_tensor(0, name="model.layers.16.mlp.experts.0.gate_proj.weight")), "policy identity is invalid"),
    (dict(header=set_tensor(0, name="model.layers.0.mlp.experts.0.gate.weight")),
     "TargetPack tensor names must be unique fixed expert tensors"),
    (dict(header=set_tensor(0, group_size=128)), "layout is invalid"),  # BF16 has no group
    (dict(header=set_tensor(1, group_size=64)), "layout is invalid"),
    (dict(header=lambda h: {**h, "encoding_tensor_counts": {"bf16_le": 1, "q4_group128": 1, "q8_group128": 2}}),
     "TargetPack encoding tensor counts are inconsistent"),
])
def test_target_pack_checks(target_pack, mutation, message):
    with pytest.raises(ContractError, match=message):
        TargetPackReader(rewrite(target_pack, **mutation))


def test_expected_identities(target_pack):
    for kw, what in ((dict(expected_model_id="x"), "model id"), (dict(expected_model_revision="c" * 40), "model revision"),
                     (dict(expected_model_manifest_sha256="d" * 64), "model manifest"),
                     (dict(expected_policy_id="q"), "policy id")):
        with pytest.raises(ContractError, match=f"TargetPack {what} mismatch"):
            TargetPackReader(target_pack, **kw)
    with open_pack(target_pack, expected_model_id=OLMOE, expected_policy_id="p") as reader:
        assert reader.layer_encoding(8) == "q8_group128" and reader.layer_encoding(0) == "bf16_le"
        with pytest.raises(ContractError, match=r"TargetPack layer index must be in \[0, 15\]"):
            reader.layer_encoding(16)


EXTRA = {
    "floats": [1e-05, 0.0001, 1e16, 1e17, 0.1, 1.5, 2.0, 5e-324, 1.7976931348623157e308, -0.0, 12345678901234567.0,
               123456789.123, 1 / 3, 6.02214076e23, -2.5e-7, 100.0, 1e22],
    "ints": [0, -1, 2 ** 63 - 1, -(2 ** 63)],
    "strings": ["plain", "quote\" backslash\\ slash/", "\b\f\n\r\t\x00\x1f\x7f", "é", " ", "\U0001F600", "\ud800"],
    "nested": {"b": [True, False, None], "a": {"é": 1, "e": 2, "z": {}}, "": []},
}


def test_canonical_json_matches_python(expert_pack):
    """Extra header content in every formatting case json.dumps produces is
    accepted as canonical; the same values written another way are not."""
    path = rewrite(expert_pack, header=lambda h: {**h, "extra": EXTRA})
    with ExpertPackReader(path) as reader:
        assert reader.header["extra"] == json.loads(json.dumps(EXTRA))
    for old, new in ((b"1e-05", b"1E-05"), (b"1e-05", b"1e-5"), (b"1e+16", b"1e16"), (b"0.0001", b"1e-04"),
                     (b"100.0", b"100.00"), (b"\\u00e9", "é".encode()), (b"\\u00e9", b"\\u00E9"),
                     (b"\\ud83d\\ude00", "\U0001F600".encode()), (b"slash/", b"slash\\/"), (b'"a":{', b'"a" :{'),
                     (b'"b":[true', b'"b": [true')):
        hb = canonical({**json.loads(rewrite_header_bytes(expert_pack)), "extra": EXTRA})
        assert old in hb, old
        bad = rewrite(expert_pack, header_bytes=lambda _hb, hb=hb, old=old, new=new: hb.replace(old, new, 1))
        with pytest.raises(ContractError, match="ExpertPack header (JSON is not canonical|is not canonical JSON)"):
            ExpertPackReader(bad)
    # keys out of order
    hb = canonical({**json.loads(rewrite_header_bytes(expert_pack)), "extra": {"a": 1, "b": 2}})
    bad = rewrite(expert_pack, header_bytes=lambda _hb: hb.replace(b'"a":1,"b":2', b'"b":2,"a":1'))
    with pytest.raises(ContractError, match="ExpertPack header JSON is not canonical"):
        ExpertPackReader(bad)


def rewrite_header_bytes(path: Path) -> bytes:
    raw = path.read_bytes()
    hlen = PREFIX.unpack_from(raw)[2]
    return raw[96:96 + hlen]


def test_views_outlive_close(expert_pack):
    reader = ExpertPackReader(expert_pack)
    data, scales, meta = reader.tensor_views("a.gate")
    want = bytes(data)
    reader.close()
    with pytest.raises(ContractError, match="closed"):
        reader.tensor_views("a.gate")
    assert bytes(data) == want and len(scales) == meta["scale_bytes"]
    data.release()
    scales.release()
    with pytest.raises(ContractError, match="has no tensor 'missing'"):
        ExpertPackReader(expert_pack).tensor_views("missing")
