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
