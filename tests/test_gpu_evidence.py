"""The packed-Q4 validation run on the GPU (uma_qmoe_amd.validate_kernel, the
reference's benchmarks/runners/validate_packed_q4_kernel.py:95-221): on a
written OLMoE-shaped ExpertPack (layer 0, 64 experts, H = 2048, I = 1024) it
produces a ``packed_q4_kernel_evidence`` document that passes the schema's
structural rules with every gate passed: the three projections against
F.linear on the dequantised weight, moe_forward at 1 and 32 tokens in
performance mode against correctness mode, timing samples, the compressed
cache with no dequantised cache. The command-line entry refuses to overwrite
its output. Acceptance (the reference's): max-abs <= 1.0, cosine >= 0.99."""

from __future__ import annotations

import json

import pytest
import torch

from test_gpu_kernels import DEV, note
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd import validate_kernel as vk
from uma_qmoe_amd.custom_op import REGISTRY
from uma_qmoe_amd.evidence import validate_kernel_evidence
from uma_qmoe_amd.packfile import write_expert_pack

pytestmark = pytest.mark.gpu
MANIFEST = "5" * 64


@pytest.fixture(scope="module")
def olmoe_pack(tmp_path_factory):
    path = tmp_path_factory.mktemp("evidence") / "olmoe_l0.uqep"
    layer = syn.build_experts(syn.C1, device=DEV, seed=303)
    write_expert_pack(path, syn.pack_tensors({0: layer}), model_id=vk.MODEL_ID, model_revision=vk.MODEL_REVISION,
                      model_manifest_sha256=MANIFEST)
    return path


def test_validation_run_passes_every_gate(olmoe_pack):
    note("evidence: validate_kernel.run on an OLMoE ExpertPack (layer 0)")
    try:
        doc = vk.run(olmoe_pack, model_manifest_sha256=MANIFEST, warmup=2, measured=5)
    finally:
        REGISTRY.uninstall("hip_gfx950")
    validate_kernel_evidence(doc)
    assert doc["status"] == "passed" and doc["gates"]["overall_passed"], doc["gates"]
    assert doc["kernel"]["platform"] == "hip_gfx950" and doc["target_id"] == "mi355x"
    c = doc["correctness"]
    assert [r["name"] for r in c["projection_results"]] == ["gate_proj", "up_proj", "down_proj"]
    assert [r["shape"] for r in c["projection_results"]] == [[1024, 2048], [1024, 2048], [2048, 1024]]
    for r in c["projection_results"] + [c["moe_forward"], c["prefill_moe_forward"]]:
        assert r["finite"] and r["cosine_similarity"] > 0.999 and r["max_absolute_error"] < 0.05, r
    p = doc["performance"]
    assert len(p["samples_milliseconds"]) == 5 and len(p["prefill_samples_milliseconds"]) == 5
    # the staged layer (64 experts x 3 projections) plus the three projections
    # q4_linear cached on their own: 65 expert-sized sets of 3,342,336 bytes
    assert p["compressed_cache_tensor_count"] == 3 * 64 + 3 and p["compressed_cache_bytes"] == 65 * 3_342_336
    assert p["dequantized_weight_cache_bytes"] == 0
    print(json.dumps({"median_ms": p["median_milliseconds"], "prefill_median_ms": p["prefill_median_milliseconds"],
                      "moe_forward": c["moe_forward"], "prefill": c["prefill_moe_forward"]}), flush=True)


def test_command_line_writes_once(olmoe_pack, tmp_path):
    out = tmp_path / "evidence.json"
    try:
        assert vk.main(["--expert-pack", str(olmoe_pack), "--model-manifest-sha256", MANIFEST,
                        "--warmup-iterations", "1", "--measured-iterations", "3", "--output", str(out)]) == 0
    finally:
        REGISTRY.uninstall("hip_gfx950")
    validate_kernel_evidence(json.loads(out.read_text()))
    with pytest.raises(SystemExit, match="refusing to overwrite"):
        vk.main(["--expert-pack", str(olmoe_pack), "--model-manifest-sha256", MANIFEST, "--output", str(out)])
    torch.cuda.synchronize()
