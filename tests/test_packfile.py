"""Pack files (CPU): the cases of the reference's tests/unit/test_expert_pack.py
and tests/unit/test_target_pack.py for this build's writer and reader, plus
independent checks of what the format fixes (prefix fields, hashes, model and
policy identities, alignment), the stored bytes against the oracle's C codec,
and a write -> read -> stage round trip of a synthetic layer."""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
import struct

import numpy as np
import pytest
import torch

from oracle import codec as oc
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.formats import ContractError, TargetTensor, decode_target_tensor, dequantize_q4
from uma_qmoe_amd.native_backend import stage_experts
from uma_qmoe_amd.packfile import (
    PREFIX,
    ExpertPackReader,
    TargetPackReader,
    inspect_pack,
    open_pack,
    write_expert_pack,
    write_target_pack,
)

OLMOE = "allenai/OLMoE-1B-7B-0125"
QWEN = "Qwen/Qwen1.5-MoE-A2.7B"
POLICY_ID = "olmoe-layer15-awq-q4-q8-bf16-v1"
LAYER_ENCODINGS = {layer: ("q4_group128" if layer == 15 else "q8_group128" if layer in {8, 11, 12, 13, 14}
                           else "bf16_le") for layer in range(16)}
IDS = dict(model_revision="a" * 40, model_manifest_sha256="b" * 64)


def _expert_pack(path: Path):
    # the two tensors of tests/unit/test_expert_pack.py:21-36
    tensors = {
        "model.layers.2.experts.7.gate_up_proj": np.linspace(-2, 2, 257, dtype=np.float32).reshape(1, 257),
        "model.layers.2.experts.7.down_proj": np.linspace(1, -1, 129, dtype=np.float32),
    }
    return write_expert_pack(path, tensors.items(), model_id=OLMOE, **IDS), tensors


def _target_pack(path: Path):
    # the three tensors of tests/unit/test_target_pack.py:32-55
    tensors = {
        "model.layers.0.mlp.experts.0.gate_proj.weight": np.linspace(-2.0, 2.0, 258, dtype=np.float32).reshape(2, 129),
        "model.layers.8.mlp.experts.1.up_proj.weight": np.linspace(-1.0, 1.0, 257, dtype=np.float32).reshape(1, 257),
        "model.layers.15.mlp.experts.2.down_proj.weight": np.linspace(1.0, -1.0, 129, dtype=np.float32).reshape(1, 129),
    }
    manifest = write_target_pack(path, tensors.items(), model_id=OLMOE, **IDS, policy_id=POLICY_ID,
                                 layer_encodings=LAYER_ENCODINGS, policy_evidence_sha256="c" * 64)
    return manifest, tensors


def _sha(obj) -> str:
    return hashlib.sha256(json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def _check_container(path: Path, magic: bytes, data_field: str):
    """What the format fixes, recomputed from the raw file."""
    raw = path.read_bytes()
    mag, version, hlen, poff, plen, hsha, psha = struct.unpack_from("<8sIIQQ32s32s", raw)
    assert PREFIX.size == 96 and mag == magic and version == 1
    assert poff % 4096 == 0 and poff + plen == len(raw) and poff >= 96 + hlen
    header_bytes = raw[96:96 + hlen]
    assert hashlib.sha256(header_bytes).digest() == hsha
    assert hashlib.sha256(raw[poff:]).digest() == psha
    assert not any(raw[96 + hlen:poff])
    header = json.loads(header_bytes)
    assert json.dumps(header, sort_keys=True, separators=(",", ":")).encode() == header_bytes
    m = header["model"]
    assert m["model_identity_sha256"] == _sha({k: m[k] for k in ("model_id", "model_revision",
                                                                  "model_manifest_sha256")})
    payload = raw[poff:]
    end = 0
    for t in header["tensors"]:
        start = t[f"{data_field}_offset"]
        assert start % 64 == 0 and start >= end and not any(payload[end:start])
        data = payload[start:start + t[f"{data_field}_bytes"]]
        scales = payload[t["scale_offset"]:t["scale_offset"] + t["scale_bytes"]]
        assert t["scale_offset"] == -(-(start + len(data)) // 4) * 4
        assert hashlib.sha256(data + scales).hexdigest() == t["tensor_payload_sha256"]
        end = t["storage_end_offset"]
        assert end % 64 == 0 and t["effective_bits_per_weight"] == (end - start) * 8 / t["element_count"]
    assert end == plen
    return header, payload


def test_expert_pack_layout_identity_and_single_mapping(tmp_path):
    path = tmp_path / "experts.uqep"
    manifest, tensors = _expert_pack(path)
    header, payload = _check_container(path, b"UQMOEPK1", "packed")
    assert manifest["header"] == header and manifest["payload_offset"] % 4096 == 0
    assert header["tensor_count"] == 2 and header["quantization"]["group_size"] == 128
    with ExpertPackReader(path, expected_model_id=OLMOE, expected_model_revision="a" * 40,
                          expected_model_manifest_sha256="b" * 64) as reader:
        assert reader.mapping_count == 1
        for name, src in tensors.items():
            restored = dequantize_q4(reader.tensor_q4(name))
            assert restored.shape == src.shape
            # the stored bytes are the oracle codec's encoding of the same values
            packed, scales = oc.q4_quantize(src, 128)
            t = reader.tensor_q4(name)
            assert t.packed == packed and t.scales == scales
        data, scales, meta = reader.tensor_views("model.layers.2.experts.7.gate_up_proj")
        assert len(data) == meta["packed_bytes"] == 129 and len(scales) == meta["scale_bytes"] == 12
        data.release()
        scales.release()
    assert inspect_pack(path) == manifest
    assert manifest["artifact"]["sha256"] == hashlib.sha256(path.read_bytes()).hexdigest()


def test_expert_pack_rejects_payload_corruption_and_model_mismatch(tmp_path):
    path = tmp_path / "experts.uqep"
    _expert_pack(path)
    raw = bytearray(path.read_bytes())
    raw[-1] ^= 0x01
    bad = tmp_path / "corrupted.uqep"
    bad.write_bytes(raw)
    with pytest.raises(ContractError, match="payload hash"):
        ExpertPackReader(bad)
    with pytest.raises(ContractError, match="model revision"):
        ExpertPackReader(path, expected_model_revision="c" * 40)
    with pytest.raises(ContractError, match="magic/version"):
        TargetPackReader(path)


def _rehashed(path: Path, mutate, field: str = "packed") -> Path:
    """Applies ``mutate(payload, first tensor entry)`` and rewrites every hash
    so that only the semantic checks can catch it (test_expert_pack.py:39-62)."""
    raw = bytearray(path.read_bytes())
    prefix = list(PREFIX.unpack_from(raw))
    hlen, poff = prefix[2], prefix[3]
    header = json.loads(raw[96:96 + hlen])
    t = header["tensors"][0]
    payload = bytearray(raw[poff:])
    mutate(payload, t)
    data = payload[t[f"{field}_offset"]:t[f"{field}_offset"] + t[f"{field}_bytes"]]
    scales = payload[t["scale_offset"]:t["scale_offset"] + t["scale_bytes"]]
    t["tensor_payload_sha256"] = hashlib.sha256(data + scales).hexdigest()
    hb = json.dumps(header, sort_keys=True, separators=(",", ":"), allow_nan=False).encode()
    assert len(hb) == hlen
    prefix[5], prefix[6] = hashlib.sha256(hb).digest(), hashlib.sha256(payload).digest()
    raw[:96] = PREFIX.pack(*prefix)
    raw[96:96 + hlen] = hb
    raw[poff:] = payload
    out = path.with_name("semantic.uqep")
    out.write_bytes(raw)
    return out


@pytest.mark.parametrize("mutate,message", [
    (lambda p, t: p.__setitem__(t["packed_offset"], 0x08), "reserved Q4 -8"),
    (lambda p, t: struct.pack_into("<f", p, t["scale_offset"], float("nan")), "finite and positive"),
    (lambda p, t: p.__setitem__(t["packed_offset"] + t["packed_bytes"] - 1,
                                p[t["packed_offset"] + t["packed_bytes"] - 1] | 0x10), "tail padding"),
    (lambda p, t: p.__setitem__(t["packed_offset"] + t["packed_bytes"], 1), "padding must be zero"),
])
def test_expert_pack_rejects_semantically_invalid_rehashed_payload(tmp_path, mutate, message):
    path = tmp_path / "experts.uqep"
    _expert_pack(path)
    with pytest.raises(ContractError, match=message):
        ExpertPackReader(_rehashed(path, mutate))


def test_target_pack_mixed_encodings_identity_and_single_mapping(tmp_path):
    path = tmp_path / "experts.uqtp"
    manifest, tensors = _target_pack(path)
    header, _ = _check_container(path, b"UQMOTPK1", "data")
    assert header["encoding_tensor_counts"] == {"bf16_le": 1, "q4_group128": 1, "q8_group128": 1}
    pol = header["policy"]
    assert pol["policy_identity_sha256"] == _sha({"policy_id": POLICY_ID, "layer_encodings": pol["layer_encodings"],
                                                  "policy_evidence_sha256": "c" * 64})
    with TargetPackReader(path, expected_model_id=OLMOE, expected_model_revision="a" * 40,
                          expected_model_manifest_sha256="b" * 64, expected_policy_id=POLICY_ID) as reader:
        assert reader.mapping_count == 1
        assert reader.layer_encoding(0) == "bf16_le"
        assert reader.layer_encoding(8) == "q8_group128"
        assert reader.layer_encoding(15) == "q4_group128"
        for name, src in tensors.items():
            t = reader.tensor(name)
            restored = decode_target_tensor(t)
            assert restored.shape == src.shape and np.all(np.isfinite(restored))
            # stored bytes == the oracle codec's encoding, decoded values == the oracle's decode
            if t.encoding == "q4_group128":
                ref = oc.q4_quantize(src, 128)
            elif t.encoding == "q8_group128":
                ref = oc.q8_quantize(src, 128)
            else:
                ref = (oc.f32_to_bf16_bits(src.reshape(-1)).astype("<u2").tobytes(), b"")
            assert (t.data, t.scales) == ref
            assert np.array_equal(restored, oc.decode_tensor(t.data, t.scales, {"shape": list(t.shape),
                                                                               "encoding": t.encoding,
                                                                               "group_size": t.group_size}))
        bf16 = "model.layers.0.mlp.experts.0.gate_proj.weight"
        assert np.max(np.abs(decode_target_tensor(reader.tensor(bf16)) - tensors[bf16])) < 0.01
    assert inspect_pack(path) == manifest


def test_target_pack_rejects_policy_and_payload_mismatch(tmp_path):
    path = tmp_path / "experts.uqtp"
    _target_pack(path)
    with pytest.raises(ContractError, match="policy id"):
        TargetPackReader(path, expected_policy_id="different")
    raw = bytearray(path.read_bytes())
    raw[-1] ^= 1
    bad = tmp_path / "corrupted.uqtp"
    bad.write_bytes(raw)
    with pytest.raises(ContractError, match="payload hash"):
        TargetPackReader(bad)


def test_target_pack_rejects_tampered_header(tmp_path):
    path = tmp_path / "experts.uqtp"
    _target_pack(path)
    raw = bytearray(path.read_bytes())
    _, _, hlen, poff, _, _, _ = PREFIX.unpack_from(raw)
    header = json.loads(raw[96:96 + hlen])
    header["encoding_tensor_counts"]["q4_group128"] += 1
    hb = json.dumps(header, sort_keys=True, separators=(",", ":")).encode()
    assert len(hb) == hlen
    prefix = list(PREFIX.unpack_from(raw))
    prefix[5] = hashlib.sha256(hb).digest()
    raw[:96] = PREFIX.pack(*prefix)
    raw[96:96 + hlen] = hb
    bad = tmp_path / "tampered.uqtp"
    bad.write_bytes(raw)
    with pytest.raises(ContractError, match="encoding tensor counts"):
        TargetPackReader(bad)
    raw[100] ^= 1  # a header byte without rehashing
    bad.write_bytes(raw)
    with pytest.raises(ContractError, match="header hash"):
        TargetPackReader(bad)


def test_target_pack_requires_complete_layer_policy(tmp_path):
    policy = dict(LAYER_ENCODINGS)
    policy.pop(0)
    with pytest.raises(ContractError, match="every OLMoE layer"):
        write_target_pack(tmp_path / "invalid.uqtp",
                          [("model.layers.15.mlp.experts.0.down_proj.weight", np.ones((1, 128), np.float32))],
                          model_id=OLMOE, **IDS, policy_id=POLICY_ID, layer_encodings=policy,
                          policy_evidence_sha256="c" * 64)
    assert not (tmp_path / "invalid.uqtp").exists()


def test_target_pack_preserves_validated_preencoded_tensor(tmp_path):
    path = tmp_path / "preencoded.uqtp"
    name = "model.layers.8.mlp.experts.0.gate_proj.weight"
    tensor = TargetTensor((1, 2), "q8_group128", bytes((1, 255)), np.asarray([0.25], "<f4").tobytes(), 128)
    write_target_pack(path, [(name, tensor)], model_id=OLMOE, **IDS, policy_id=POLICY_ID,
                      layer_encodings=LAYER_ENCODINGS, policy_evidence_sha256="c" * 64)
    with TargetPackReader(path) as reader:
        assert reader.tensor(name) == tensor
        assert np.array_equal(decode_target_tensor(reader.tensor(name)), np.asarray([[0.25, -0.25]], np.float32))
    with pytest.raises(ContractError, match="does not match its layer policy"):
        write_target_pack(tmp_path / "mismatch.uqtp", [("model.layers.0.mlp.experts.0.gate_proj.weight", tensor)],
                          model_id=OLMOE, **IDS, policy_id=POLICY_ID, layer_encodings=LAYER_ENCODINGS,
                          policy_evidence_sha256="c" * 64)


def test_target_pack_qwen_policy_bounds(tmp_path):
    policy = {layer: "q8_group128" for layer in range(24)}
    path = tmp_path / "qwen.uqtp"
    write_target_pack(path, [("model.layers.23.mlp.experts.59.down_proj.weight", np.ones((1, 128), np.float32))],
                      model_id=QWEN, **IDS, policy_id="qwen-q8", layer_encodings=policy,
                      policy_evidence_sha256="d" * 64)
    with open_pack(path) as reader:
        assert isinstance(reader, TargetPackReader) and reader.layer_encoding(23) == "q8_group128"
        with pytest.raises(ContractError, match=r"\[0, 23\]"):
            reader.layer_encoding(24)
    with pytest.raises(ContractError, match="out of range"):
        write_target_pack(tmp_path / "oob.uqtp",
                          [("model.layers.0.mlp.experts.60.down_proj.weight", np.ones((1, 128), np.float32))],
                          model_id=QWEN, **IDS, policy_id="qwen-q8", layer_encodings=policy,
                          policy_evidence_sha256="d" * 64)


def test_writer_refuses_overwrite_and_duplicates(tmp_path):
    path = tmp_path / "experts.uqep"
    _expert_pack(path)
    with pytest.raises(ContractError, match="overwrite"):
        _expert_pack(path)
    with pytest.raises(ContractError, match="duplicate"):
        write_expert_pack(tmp_path / "dup.uqep", [("a", np.ones(4)), ("a", np.ones(4))], model_id=OLMOE, **IDS)
    assert not (tmp_path / "dup.uqep").exists()


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
def test_pack_round_trip_stages_the_synthetic_bytes(tmp_path, encoding):
    """A synthetic layer written into a pack, read back and staged
    expert-major equals the layer it came from, byte for byte."""
    shape = syn.MoEShape(f"pack_rt_{encoding}", 256, 5, 2, 128, encoding=encoding)
    layer = syn.build_experts(shape, seed=5)
    path = tmp_path / "layer3.uqtp"
    policy = {i: encoding for i in range(16)}
    tensors = [(n.replace("layers.0.", "layers.3."), t) for n, t in syn.pack_tensors({0: layer})]
    write_target_pack(path, tensors, model_id=OLMOE, **IDS, policy_id="rt", layer_encodings=policy,
                      policy_evidence_sha256="e" * 64)
    with TargetPackReader(path) as reader:
        staged = stage_experts(reader, 3, "cpu")
    assert (staged.encoding, staged.num_experts, staged.hidden_size, staged.intermediate_size) == (
        encoding, 5, 256, 128)
    for a, b in zip(layer.tensors, staged.tensors):
        assert a.shape == b.shape and torch.equal(a.view(torch.uint8), b.reshape(a.shape).view(torch.uint8))
