"""Qwen host integration (load_fixed_qwen) on the CPU: a tiny Qwen2MoE
checkpoint written to disk loads with the routed experts from a Q4
ExpertPack, every MoE block replaced, no expert parameter; with
performance_mode=False the blocks run the registered reference (the oracle)
and the model's logits match Transformers' own model with the pack's
dequantized experts. The loader's refusals follow the reference's
(qwen_compressed_loader.py:143-299)."""

from __future__ import annotations

import json

import pytest
import torch

from oracle import moe as om
from qwen_tiny import ARCH, MANIFEST, prompt, reference_model, write_checkpoint
from uma_qmoe_amd.custom_op import (
    clear_reference_implementations,
    register_moe_forward,
    register_reference_implementation,
)
from uma_qmoe_amd.formats import ContractError
from uma_qmoe_amd.qwen_host import is_qwen_expert_tensor_name, load_fixed_qwen


def _oracle_block(hidden, router, sg, su, sd, seg, top_k, norm, layer_index, reader):
    layer = {"router": router, "shared_gate": sg, "shared_up": su, "shared_down": sd, "shared_expert_gate": seg,
             "top_k": int(top_k), "num_experts": router.shape[0], "norm_topk_prob": bool(norm)}
    return om.qwen_block(hidden, layer, reader, layer_index)


def _oracle_routed(hidden, indices, weights, layer_index, reader):
    return om.streaming_reference(hidden, indices, weights, layer_index, reader, num_experts=60)


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("qwen_tiny")
    pack, model, q4 = write_checkpoint(d)
    return d, pack, model, q4


@pytest.fixture(autouse=True)
def _references():
    register_moe_forward()
    register_reference_implementation("block", _oracle_block)
    register_reference_implementation("qwen", _oracle_routed)
    yield
    clear_reference_implementations()


def _close(got, ref, what, rel=2e-2):
    r = om.rel_l2(got.float(), ref.float())
    assert torch.isfinite(got).all(), what
    assert r <= rel, f"{what}: rel-L2 {r}"


@pytest.mark.parametrize("fused_block", [True, False])
def test_host_matches_transformers_with_dequantized_experts(checkpoint, fused_block):
    d, pack, model, q4 = checkpoint
    ref = reference_model(model, q4)
    ids = prompt(6)
    with load_fixed_qwen(d, pack, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH,
                         fused_block=fused_block) as host:
        ev = host.evidence
        assert ev["quantized_moe_block_count"] == 2 and ev["expert_parameter_count"] == 0
        assert ev["skipped_expert_tensor_count"] == 2 * 60 * 3 and ev["expert_pack_mapping_count"] == 1
        assert not any(".mlp.experts." in n for n, _ in host.model.named_parameters())
        with torch.no_grad():
            got = host.model(input_ids=ids).logits
            want = ref(input_ids=ids).logits
        _close(got, want, f"logits fused_block={fused_block}")
        assert torch.equal(got[0, -1].argmax(), want[0, -1].argmax())


def test_expert_tensor_names():
    assert is_qwen_expert_tensor_name("model.layers.3.mlp.experts.59.down_proj.weight")
    assert not is_qwen_expert_tensor_name("model.layers.3.mlp.shared_expert.down_proj.weight")
    assert not is_qwen_expert_tensor_name("model.layers.3.mlp.experts.gate_up_proj")


def test_loader_refusals(checkpoint, tmp_path):
    d, pack, _model, _q4 = checkpoint
    with pytest.raises(ContractError, match="unexpected fixed Qwen architecture"):
        load_fixed_qwen(d, pack, model_manifest_sha256=MANIFEST, device="cpu")  # the 24-layer default
    with pytest.raises(ContractError, match="ExpertPack cannot satisfy a TargetPack policy id"):
        load_fixed_qwen(d, pack, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH,
                        target_policy_id="p")
    with pytest.raises(ContractError, match="manifest"):
        load_fixed_qwen(d, pack, model_manifest_sha256="3" * 64, device="cpu", architecture=ARCH)
    # an index missing a dense tensor, and one with an expert tensor too many
    import shutil

    for mutate, message in ((lambda m: m.pop("lm_head.weight"), "dense checkpoint set mismatch"),
                            (lambda m: m.__setitem__("model.layers.0.mlp.experts.60.up_proj.weight", "x"),
                             "expected to skip 360")):
        e = tmp_path / message.split()[0]
        shutil.copytree(d, e)
        index = json.loads((e / "model.safetensors.index.json").read_text())
        mutate(index["weight_map"])
        (e / "model.safetensors.index.json").write_text(json.dumps(index))
        with pytest.raises(ContractError, match=message):
            load_fixed_qwen(e, e / "experts.uqep", model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH)


def _target_pack(path, q4, keep=lambda name: True):
    """The tiny model's routed experts as a Q4 TargetPack (policy
    "qwen-tiny-q4", every layer Q4), holding the tensors ``keep`` accepts."""
    from uma_qmoe_amd.formats import TargetTensor
    from uma_qmoe_amd.packfile import write_target_pack
    from uma_qmoe_amd.qwen_host import QWEN_MODEL_ID, QWEN_MODEL_REVISION

    tensors = [(n, TargetTensor(tuple(t.shape), "q4_group128", t.packed, t.scales, t.group_size))
               for n, t in sorted(q4.items()) if keep(n)]
    write_target_pack(path, tensors, model_id=QWEN_MODEL_ID, model_revision=QWEN_MODEL_REVISION,
                      model_manifest_sha256=MANIFEST, policy_id="qwen-tiny-q4",
                      layer_encodings={i: "q4_group128" for i in range(24)}, policy_evidence_sha256="4" * 64)
    return path


def test_target_pack_loads_and_incomplete_one_is_refused(checkpoint, tmp_path):
    """A complete TargetPack loads (one mapping, one VMA); one missing a
    layer, or holding a tensor at the wrong shape, is refused before the model
    is built (target_pack.py:738-775 via qwen_compressed_loader.py:187)."""
    d, _pack, _model, q4 = checkpoint
    full = _target_pack(tmp_path / "full.uqtp", q4)
    with load_fixed_qwen(d, full, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH,
                         target_policy_id="qwen-tiny-q4") as host:
        assert host.evidence["expert_pack_mapping_count"] == 1
        assert host.evidence["expert_pack_vma_count"] == 1
        assert host.evidence["quantized_moe_block_count"] == 2
    host.close()  # a second close does nothing
    partial = _target_pack(tmp_path / "partial.uqtp", q4, keep=lambda n: not n.startswith("model.layers.1."))
    with pytest.raises(ContractError, match=r"tensor set mismatch: missing=\['model\.layers\.1\.mlp\.experts\.0\."):
        load_fixed_qwen(d, partial, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH,
                        target_policy_id="qwen-tiny-q4")
    with pytest.raises(ContractError, match="Qwen TargetPack loading requires a policy id"):
        load_fixed_qwen(d, full, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH)


def test_reader_with_more_than_one_mapping_is_refused(checkpoint):
    from uma_qmoe_amd.packfile import ExpertPackReader

    d, pack, _model, _q4 = checkpoint
    reader = ExpertPackReader(pack, expected_model_manifest_sha256=MANIFEST)
    try:
        reader.mapping_count = 2
        with pytest.raises(ContractError, match="mapped ExpertPack more than once"):
            load_fixed_qwen(d, reader, model_manifest_sha256=MANIFEST, device="cpu", architecture=ARCH)
    finally:
        reader.close()


def test_incomplete_target_pack_counts_are_checked():
    """The completeness check on an in-memory pack: the exact tensor set at
    the model's shapes passes; a policy that disagrees with the stored
    encodings is refused."""
    from uma_qmoe_amd.formats import encode
    from uma_qmoe_amd.packfile import memory_pack
    from uma_qmoe_amd.qwen_host import expected_expert_tensors, require_complete_target_pack

    import numpy as np

    shapes = expected_expert_tensors(2, 3, 256, 128)
    assert len(shapes) == 2 * 3 * 3 and shapes["model.layers.1.mlp.experts.2.down_proj.weight"] == (256, 128)
    tensors = {n: encode(np.zeros(s, np.float32), "q4_group128") for n, s in shapes.items()}
    require_complete_target_pack(memory_pack(tensors, {0: "q4_group128", 1: "q4_group128"}),
                                 layers=2, experts=3, hidden=256, intermediate=128)
    with pytest.raises(ContractError, match="policy counts are inconsistent"):
        require_complete_target_pack(memory_pack(tensors, {0: "q4_group128", 1: "q8_group128"}),
                                     layers=2, experts=3, hidden=256, intermediate=128)
    bad = dict(tensors)
    bad["model.layers.0.mlp.experts.0.up_proj.weight"] = encode(np.zeros((128, 128), np.float32), "q4_group128")
    with pytest.raises(ContractError, match=r"wrong_shape=\['model\.layers\.0\.mlp\.experts\.0\.up_proj"):
        require_complete_target_pack(memory_pack(bad, {0: "q4_group128", 1: "q4_group128"}),
                                     layers=2, experts=3, hidden=256, intermediate=128)
