"""The library's pack reader staging a layer from a pack file onto the GPU
(``uqm_pack_stage_projection``, through ``stage_experts``): the device bytes
equal the synthetic layer the file was written from, byte for byte, for each
encoding; the Q4 case is a full c2 layer (60 experts, 86.5 MB per
projection), several times the reader's pinned buffers, so pieces split
across buffer fills and both buffers alternate. A staged layer then runs a
block against the same layer staged by the reference's route (copies of the
tensor views)."""

from __future__ import annotations

import pytest
import torch

from test_gpu_kernels import DEV, note
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.native_backend import load_native_extension, stage_experts
from uma_qmoe_amd.packfile import TargetPackReader, write_target_pack

pytestmark = pytest.mark.gpu

QWEN = "Qwen/Qwen1.5-MoE-A2.7B"
IDS = dict(model_revision="a" * 40, model_manifest_sha256="b" * 64)


def _write(tmp_path, shape, layer_index, seed):
    layer = syn.build_experts(shape, layer=layer_index, seed=seed, device=DEV)
    tensors = [(n.replace("layers.0.", f"layers.{layer_index}."), t) for n, t in syn.pack_tensors({0: layer})]
    path = tmp_path / f"{shape.name}.uqtp"
    write_target_pack(path, tensors, model_id=QWEN, **IDS, policy_id="staging",
                      layer_encodings={i: shape.encoding for i in range(24)}, policy_evidence_sha256="e" * 64)
    return path, layer


@pytest.mark.parametrize("encoding,experts,inter", [("q4_group128", 60, 1408), ("q8_group128", 7, 256),
                                                    ("bf16_le", 5, 128)])
def test_staged_bytes_equal_the_written_layer(tmp_path, encoding, experts, inter):
    shape = syn.MoEShape(f"staging_{encoding}", 2048, experts, 4, inter, encoding=encoding)
    note(f"pack staging {encoding} E={experts} I={inter}")
    path, layer = _write(tmp_path, shape, 3, seed=11)
    with TargetPackReader(path) as reader:
        staged = stage_experts(reader, 3, DEV)
        torch.cuda.synchronize()
    assert (staged.encoding, staged.num_experts, staged.hidden_size, staged.intermediate_size) == (
        encoding, experts, 2048, inter)
    for want, got in zip(layer.tensors, staged.tensors):
        assert want.shape == got.shape
        assert torch.equal(want.view(torch.uint8), got.reshape(want.shape).view(torch.uint8))


def test_staged_layer_runs_like_the_synthetic_one(tmp_path):
    shape = syn.C2
    note("pack staging c2 block")
    path, layer = _write(tmp_path, shape, 0, seed=syn.SEED)
    _, ext = load_native_extension()
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, 1).to(DEV)
    with TargetPackReader(path) as reader:
        staged = stage_experts(reader, 0, DEV)
    want = ext.moe_layer(layer, dense, x, shape.top_k)
    got = ext.moe_layer(staged, dense, x, shape.top_k)
    for a, b in zip(want, got):
        assert torch.equal(a, b)
