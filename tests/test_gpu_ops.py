"""The reference's operator API end to end on the GPU.

Each case is the drop-in flow of src/uma_qmoe/custom_op.py:509-628 and
src/uma_qmoe/native_backend.py:482-552,1141-1154: register the ops, install a
backend, register a pack reader, call ``torch.ops.uma_qmoe.*(..., True)`` on
cuda tensors, and compare with the oracle reading the same pack:

  c1  OLMoE shapes, all-Q4 ExpertPack file, ``moe_forward``
  c2  Qwen shapes, all-Q4 TargetPack file, ``qwen_moe_forward`` and ``moe_block``
  c3  Qwen layers 0 (BF16) and 16 (Q8) in an in-memory TargetPack, mixed
      backend, ``moe_block`` and ``qwen_moe_forward``

Also: the backend's cache summary equals the staged compressed bytes with no
dequantized cache, unregistering empties the caches, ``q4_linear`` through a
pack handle, correctness mode (the library's transient-dequantisation path, or a
registered implementation in its place), the HIP dequantisation bit for bit
against the oracle codec, and the
multi-token routing weights equal softmax(logits) at the selected experts.
Tolerance (north star): rel-L2 <= 1e-2, max-abs <= 2e-2; indices bit-exact
given the logits.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe as om
from test_gpu_kernels import DEV, assert_close, assert_weights_follow_logits, note
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.custom_op import (
    REGISTRY,
    clear_reference_implementations,
    register_expert_pack,
    register_moe_forward,
    register_reference_implementation,
    register_target_pack,
    unregister_expert_pack,
)
from uma_qmoe_amd.formats import decode_target_tensor
from uma_qmoe_amd.native_backend import install_mixed_target_backend, install_packed_q4_backend
from uma_qmoe_amd.packfile import ExpertPackReader, TargetPackReader, memory_pack, write_expert_pack, write_target_pack

pytestmark = pytest.mark.gpu

IDS = dict(model_revision="0" * 40, model_manifest_sha256="1" * 64)
QWEN = "Qwen/Qwen1.5-MoE-A2.7B"
OLMOE = "allenai/OLMoE-1B-7B-0125"


@pytest.fixture(autouse=True)
def _ops():
    register_moe_forward()
    yield
    clear_reference_implementations()
    REGISTRY.uninstall("hip_gfx950")


def _renamed(layer, index):
    """The synthetic layer's tensors, named as layer ``index`` of a pack."""
    for name, t in syn.pack_tensors({0: layer}):
        yield name.replace("model.layers.0.", f"model.layers.{index}."), t


def _dense_cpu(dense):
    return {k: (None if v is None else v.cpu()) for k, v in
            (("router", dense.router), ("shared_gate", dense.shared_gate), ("shared_up", dense.shared_up),
             ("shared_down", dense.shared_down), ("shared_expert_gate", dense.shared_expert_gate))}


def _expected_cache(layer) -> int:
    return layer.num_experts * layer.bytes_per_expert()


# ------------------------------------------------------------------ c1 --
def test_c1_moe_forward_from_expert_pack_file(tmp_path):
    note("ops c1: ExpertPack file -> install_packed_q4_backend -> moe_forward")
    L = 5
    layer = syn.build_experts(syn.C1, device=DEV, seed=101)
    path = tmp_path / "olmoe_l5.uqep"
    write_expert_pack(path, _renamed(layer, L), model_id=OLMOE, **IDS)
    reader = ExpertPackReader(path, expected_model_id=OLMOE)
    handle = register_expert_pack(reader)
    backend = install_packed_q4_backend()
    try:
        dense = syn.build_dense(syn.C1, seed=101)
        for t in (1, 3, 40):
            x = syn.hidden_states(syn.C1, t, seed=t)
            _logits, w, idx = om.router(x, dense.router, 8)
            out = torch.ops.uma_qmoe.moe_forward(x.to(DEV), idx.to(DEV), w.to(DEV), L, handle, True)
            torch.cuda.synchronize()
            assert out.shape == x.shape and out.dtype == torch.bfloat16 and out.device.type == "cuda"
            ref = om.olmoe_streaming_reference(x, idx, w, L, reader)
            assert_close(out, ref, f"c1 moe_forward T={t}")
            # int32 routes are accepted as well (custom_op.py:195-198)
            out32 = torch.ops.uma_qmoe.moe_forward(x.to(DEV), idx.to(DEV, torch.int32), w.to(DEV), L, handle, True)
            assert torch.equal(out32.cpu().view(torch.int16), out.cpu().view(torch.int16))
        summary = backend.cache_summary()
        assert summary == {"tensor_count": 3 * 64, "device_storage_bytes": 64 * 3_342_336,
                           "dequantized_weight_bytes": 0}
        assert summary["device_storage_bytes"] == _expected_cache(layer)
        # a single projection through the handle (native_backend.py:300-317)
        name = f"model.layers.{L}.mlp.experts.9.gate_proj.weight"
        xs = syn.hidden_states(syn.C1, 2, seed=77)
        got = backend.q4_linear(xs.to(DEV), handle, name)
        wt = torch.from_numpy(decode_target_tensor(reader.tensor(name)))
        assert_close(got, torch.nn.functional.linear(xs.float(), wt), "c1 q4_linear via handle")
    finally:
        unregister_expert_pack(handle)
        reader.close()
    assert backend.cache_summary() == {"tensor_count": 0, "device_storage_bytes": 0, "dequantized_weight_bytes": 0}


# ------------------------------------------------------------------ c2 --
def _qwen_q4_pack(tmp_path, layer, L):
    path = tmp_path / "qwen_q4.uqtp"
    write_target_pack(path, _renamed(layer, L), model_id=QWEN, **IDS, policy_id="qwen-all-q4",
                      layer_encodings={i: "q4_group128" for i in range(24)}, policy_evidence_sha256="2" * 64)
    return TargetPackReader(path, expected_model_id=QWEN, expected_policy_id="qwen-all-q4")


@pytest.mark.parametrize("norm", [False, True])
def test_c2_qwen_ops_from_target_pack_file(tmp_path, norm):
    note(f"ops c2: TargetPack file -> qwen_moe_forward / moe_block (norm_topk_prob={norm})")
    L = 7
    shape = syn.C2
    layer = syn.build_experts(shape, device=DEV, seed=202)
    dense = syn.build_dense(shape, device=DEV, seed=202)
    dc = _dense_cpu(dense)
    lay = {**dc, "top_k": 4, "num_experts": 60, "norm_topk_prob": norm}
    reader = _qwen_q4_pack(tmp_path, layer, L)
    handle = register_target_pack(reader)
    backend = install_packed_q4_backend()
    try:
        for t in (1, 2, 5, 32):
            x = syn.hidden_states(shape, t, seed=10 + t)
            xd = x.to(DEV)
            # the routed op with routes from the (oracle) router
            _l, w, idx = om.router(x, dc["router"], 4, norm)
            out = torch.ops.uma_qmoe.qwen_moe_forward(xd, idx.to(DEV), w.to(DEV), L, handle, True)
            ref = om.qwen_streaming_reference(x, idx, w, L, reader)
            assert_close(out, ref, f"c2 qwen_moe_forward T={t}")
            # the whole block: router + routed + gated shared expert in one op
            out, logits, weights, indices = torch.ops.uma_qmoe.moe_block(
                xd, dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate,
                4, norm, L, handle, True)
            torch.cuda.synchronize()
            assert logits.shape == (t, 60) and weights.shape == (t, 4) and indices.dtype == torch.int64
            assert_close(logits, torch.nn.functional.linear(x.float(), dc["router"].float()), f"c2 logits T={t}",
                         rel=5e-3, mx=2e-2)
            assert_weights_follow_logits(logits, weights, indices, norm, f"c2 moe_block T={t}")
            ref, *_ = om.qwen_block(x, lay, reader, L, routes=(weights.cpu(), indices.cpu()))
            assert_close(out, ref, f"c2 moe_block T={t}")
        assert backend.cache_summary()["device_storage_bytes"] == _expected_cache(layer)
        assert backend.cache_summary()["dequantized_weight_bytes"] == 0
        backend.status()  # no fused launch hit its wait budget
    finally:
        unregister_expert_pack(handle)
        reader.close()
    assert backend.cache_summary()["tensor_count"] == 0


def test_correctness_mode_on_the_device(tmp_path):
    """performance_mode=False on device tensors runs the library's correctness
    path (experts dequantised transiently to BF16, then the BF16 expert
    kernels): within the north-star tolerance of the oracle and of performance
    mode, an invalid expert id refused as the reference refuses it, nothing
    cached. An implementation installed with register_reference_implementation
    runs instead (here the oracle), with the leased reader."""
    L = 3
    shape = syn.MoEShape("ops_small", 2048, 60, 4, 256, 512)
    layer = syn.build_experts(shape, device=DEV, seed=5)
    dense = syn.build_dense(shape, device=DEV, seed=5)
    reader = _qwen_q4_pack(tmp_path, layer, L)
    handle = register_target_pack(reader)
    backend = install_packed_q4_backend()
    try:
        for t in (1, 3, 40):
            note(f"ops correctness mode: qwen_moe_forward and moe_block T={t}")
            x = syn.hidden_states(shape, t, seed=3 + t)
            _l, w, idx = om.router(x, dense.router.cpu(), 4)
            slow = torch.ops.uma_qmoe.qwen_moe_forward(x.to(DEV), idx.to(DEV), w.to(DEV), L, handle, False)
            fast = torch.ops.uma_qmoe.qwen_moe_forward(x.to(DEV), idx.to(DEV), w.to(DEV), L, handle, True)
            ref = om.qwen_streaming_reference(x, idx, w, L, reader)
            assert_close(slow, ref, f"correctness mode vs oracle T={t}")
            assert_close(fast, slow, f"performance vs correctness mode T={t}")
            args = (dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate, 4,
                    False, L, handle)
            out, logits, weights, indices = torch.ops.uma_qmoe.moe_block(x.to(DEV), *args, False)
            assert_weights_follow_logits(logits, weights, indices, False, f"correctness-mode block T={t}")
            ref_b, *_ = om.qwen_block(x, {**_dense_cpu(dense), "top_k": 4, "num_experts": 60}, reader, L,
                                      routes=(weights.cpu(), indices.cpu()))
            assert_close(out, ref_b, f"correctness-mode moe_block vs oracle T={t}")
        bad = idx.clone()
        bad[0, 1] = 60
        with pytest.raises(RuntimeError, match="invalid expert"):
            torch.ops.uma_qmoe.qwen_moe_forward(x.to(DEV), bad.to(DEV), w.to(DEV), L, handle, False)
        assert backend.cache_summary()["dequantized_weight_bytes"] == 0
        seen = []

        def oracle_impl(hidden, indices, weights, layer_index, rd):
            seen.append(rd)
            return om.qwen_streaming_reference(hidden.cpu(), indices.cpu(), weights.cpu(), layer_index, rd).to(
                hidden.device)

        register_reference_implementation("qwen", oracle_impl)
        registered = torch.ops.uma_qmoe.qwen_moe_forward(x.to(DEV), idx.to(DEV), w.to(DEV), L, handle, False)
        assert seen == [reader]
        assert torch.equal(registered.cpu(), ref.to(registered.dtype))
    finally:
        unregister_expert_pack(handle)
        reader.close()


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128"])
def test_dequantize_bits_match_the_oracle_codec(hip_ext, encoding):
    """uqm_dequantize against the oracle's C codec then round-to-nearest-even
    to BF16, bit for bit: random payloads (every code the codec decodes:
    nibbles -7..7, bytes -128..127), scales of mixed magnitude, and a tensor
    whose 128-value groups cross its rows (3 x 136). Q4's reserved -8 code,
    which the codec refuses, decodes to -8 * scale as in every other kernel
    of the library."""
    import numpy as np

    from oracle import codec as oc

    rng = np.random.default_rng(11)
    for shape in ((3, 136), (2, 64, 256)):
        n = int(np.prod(shape))
        scales = (rng.uniform(0.5, 2.0, -(-n // 128)) * 10.0 ** rng.integers(-6, 3, -(-n // 128))).astype("<f4")
        if encoding == "q4_group128":
            nib = rng.choice(np.array([c for c in range(16) if c != 8], dtype=np.uint8), n)
            raw = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
            want = oc.q4_dequantize(raw.tobytes(), scales.tobytes(), shape)
        else:
            raw = rng.integers(-128, 128, n, dtype=np.int8)
            want = oc.q8_dequantize(raw.tobytes(), scales.tobytes(), shape)
        got = hip_ext.dequantize(torch.from_numpy(raw.copy()).to(DEV), torch.from_numpy(scales).to(DEV), encoding, 128)
        bits = got.cpu().view(torch.int16).numpy().view(np.uint16)
        assert np.array_equal(bits, oc.f32_to_bf16_bits(want)), f"{encoding} {shape}"
    if encoding == "q4_group128":  # the reserved code: 0x88 is (-8, -8)
        raw = np.full(64, 0x88, dtype=np.uint8)
        sc = np.array([0.25], dtype="<f4")
        got = hip_ext.dequantize(torch.from_numpy(raw).to(DEV), torch.from_numpy(sc).to(DEV), encoding, 128)
        assert bool((got.cpu().float() == -2.0).all())


# ------------------------------------------------------------------ c3 --
def test_c3_mixed_layers_from_memory_pack():
    note("ops c3: in-memory TargetPack, BF16 layer 0 + Q8 layer 16 -> install_mixed_target_backend")
    layers = {l: syn.build_experts(syn.c3_layer_shape(l), layer=l, device=DEV) for l in (0, 16)}
    denses = {l: syn.build_dense(syn.c3_layer_shape(l), layer=l, device=DEV) for l in (0, 16)}
    tensors = dict(syn.pack_tensors(layers))
    policy = {i: ("bf16_le" if i < 16 else "q8_group128") for i in range(24)}
    pack = memory_pack(tensors, policy, num_experts=60)
    handle = register_target_pack(pack)
    backend = install_mixed_target_backend()
    try:
        for l in (0, 16):
            d = denses[l]
            lay = {**_dense_cpu(d), "top_k": 4, "num_experts": 60}
            for t in (1, 4):
                x = syn.hidden_states(syn.c3_layer_shape(l), t, seed=40 + l + t)
                out, logits, weights, indices = torch.ops.uma_qmoe.moe_block(
                    x.to(DEV), d.router, d.shared_gate, d.shared_up, d.shared_down, d.shared_expert_gate, 4, False, l,
                    handle, True)
                assert_weights_follow_logits(logits, weights, indices, False, f"c3 layer {l} T={t}")
                ref, *_ = om.qwen_block(x, lay, pack, l, routes=(weights.cpu(), indices.cpu()))
                assert_close(out, ref, f"c3 layer {l} ({pack.layer_encoding(l)}) moe_block T={t}")
                routed = torch.ops.uma_qmoe.qwen_moe_forward(x.to(DEV), indices, weights, l, handle, True)
                assert_close(routed, om.qwen_streaming_reference(x, indices.cpu(), weights.cpu(), l, pack),
                             f"c3 layer {l} qwen_moe_forward T={t}")
        assert backend.cache_summary() == {"tensor_count": 2 * 180,
                                           "device_storage_bytes": sum(_expected_cache(v) for v in layers.values()),
                                           "dequantized_weight_bytes": 0}
    finally:
        unregister_expert_pack(handle)
    assert backend.cache_summary()["device_storage_bytes"] == 0


def test_q4_only_backend_refuses_mixed_layers():
    layers = {0: syn.build_experts(syn.MoEShape("ops_bf16", 2048, 4, 2, 256, encoding="bf16_le"), device=DEV)}
    pack = memory_pack(dict(syn.pack_tensors(layers)), {0: "bf16_le"}, num_experts=4)
    handle = register_target_pack(pack)
    install_packed_q4_backend()
    try:
        x = torch.zeros(1, 2048, dtype=torch.bfloat16, device=DEV)
        idx = torch.zeros(1, 2, dtype=torch.int64, device=DEV)
        with pytest.raises(RuntimeError, match="install the mixed backend"):
            torch.ops.uma_qmoe.qwen_moe_forward(x, idx, idx.to(torch.bfloat16), 0, handle, True)
    finally:
        unregister_expert_pack(handle)


def test_platform_gate_on_device():
    """The gate of custom_op.py:149-169 on this device: gfx950 is accepted."""
    from uma_qmoe_amd.custom_op import device_platform

    assert device_platform(torch, torch.zeros(1, device=DEV)) == "hip_gfx950"
