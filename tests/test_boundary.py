"""Operator boundary contract (CPU): mirrors the reference's
tests/unit/test_custom_operator_lifecycle.py and
tests/unit/test_native_backend_contracts.py for this build."""

from __future__ import annotations

import re
import threading
from types import SimpleNamespace

import pytest
import torch

from uma_qmoe_amd import custom_op
from uma_qmoe_amd.custom_op import (
    acquire_expert_pack,
    expert_pack_for_handle,
    register_expert_pack,
    register_moe_forward,
    register_performance_backend,
    register_reference_implementation,
    unregister_expert_pack,
)
from uma_qmoe_amd.native_backend import MixedTargetNativeBackend, PackedQ4NativeBackend
from uma_qmoe_amd.formats import ContractError


class _Reader:
    mapping_count = 1


def test_pack_access_requires_active_lease():
    reader = _Reader()
    handle = register_expert_pack(reader)
    try:
        with pytest.raises(RuntimeError, match="active operator lease"):
            expert_pack_for_handle(handle)
        with acquire_expert_pack(handle) as leased:
            assert leased is reader
            assert expert_pack_for_handle(handle) is reader
            with acquire_expert_pack(handle):  # re-entrant
                pass
            with pytest.raises(ContractError, match="active call"):
                unregister_expert_pack(handle)
    finally:
        unregister_expert_pack(handle)


def test_pack_requires_single_mapping():
    with pytest.raises(ContractError, match="exactly one"):
        register_expert_pack(SimpleNamespace(mapping_count=2))


def test_unregister_waits_for_active_call_and_rejects_new_calls():
    handle = register_expert_pack(_Reader())
    entered, release, done = threading.Event(), threading.Event(), threading.Event()

    def active():
        with acquire_expert_pack(handle):
            entered.set()
            assert release.wait(timeout=5)

    def close():
        unregister_expert_pack(handle)
        done.set()

    worker = threading.Thread(target=active)
    closer = threading.Thread(target=close)
    worker.start()
    assert entered.wait(timeout=5)
    closer.start()
    assert not done.wait(timeout=0.1)
    with pytest.raises(RuntimeError, match="unknown or closed"):
        with acquire_expert_pack(handle):
            pass
    release.set()
    worker.join(timeout=5)
    closer.join(timeout=5)
    assert done.is_set()


def test_platform_allowlist_and_callable_backend():
    with pytest.raises(ContractError, match="unsupported"):
        register_performance_backend("cuda_sm121", lambda *a: None)
    with pytest.raises(ContractError, match="callable"):
        register_performance_backend("hip_gfx950", object())


def _ops_inputs():
    x = torch.zeros(2, 2048, dtype=torch.bfloat16)
    idx = torch.zeros(2, 4, dtype=torch.int64)
    w = torch.zeros(2, 4, dtype=torch.bfloat16)
    return x, idx, w


def test_performance_mode_without_backend_fails_closed():
    register_moe_forward()
    handle = register_expert_pack(_Reader())
    try:
        x, idx, w = _ops_inputs()
        with pytest.raises(RuntimeError, match="silent reference fallback is forbidden"):
            torch.ops.uma_qmoe.qwen_moe_forward(x, idx, w, 0, handle, True)
        with pytest.raises(RuntimeError, match="silent reference fallback is forbidden"):
            torch.ops.uma_qmoe.moe_forward(x, idx, w, 0, handle, True)
    finally:
        unregister_expert_pack(handle)


def test_correctness_mode_runs_only_a_registered_implementation():
    register_moe_forward()
    handle = register_expert_pack(_Reader())
    custom_op.clear_reference_implementations()
    try:
        x, idx, w = _ops_inputs()
        with pytest.raises(RuntimeError, match="no registered qwen implementation"):
            torch.ops.uma_qmoe.qwen_moe_forward(x, idx, w, 0, handle, False)
        seen = {}

        def impl(hidden, indices, weights, layer, reader):
            seen["reader"] = reader
            return hidden + 1

        register_reference_implementation("qwen", impl)
        out = torch.ops.uma_qmoe.qwen_moe_forward(x, idx, w, 3, handle, False)
        assert isinstance(seen["reader"], _Reader)
        assert torch.equal(out, x + 1)
    finally:
        custom_op.clear_reference_implementations()
        unregister_expert_pack(handle)


def test_meta_dispatch_shapes():
    register_moe_forward()
    x = torch.empty(3, 2048, dtype=torch.bfloat16, device="meta")
    idx = torch.empty(3, 8, dtype=torch.int64, device="meta")
    w = torch.empty(3, 8, dtype=torch.bfloat16, device="meta")
    assert torch.ops.uma_qmoe.moe_forward(x, idx, w, 0, 1, True).shape == x.shape
    r = torch.empty(64, 2048, dtype=torch.bfloat16, device="meta")
    out, logits, weights, indices = torch.ops.uma_qmoe.moe_block(x, r, None, None, None, None, 8, False, 0, 1, True)
    assert out.shape == x.shape and logits.shape == (3, 64) and weights.shape == (3, 8)
    assert indices.dtype == torch.int64


def _fake_ext(**names):
    return SimpleNamespace(**{n: (lambda *a: None) for n in names})


Q4_EXT = dict(q4_linear=1, q4_moe_forward=1)


def test_backend_requires_entry_points_and_platform():
    with pytest.raises(ContractError, match="q4_moe_forward"):
        PackedQ4NativeBackend("hip_gfx950", _fake_ext(q4_linear=1))
    with pytest.raises(ContractError, match="q8_moe_forward"):
        MixedTargetNativeBackend("hip_gfx950", _fake_ext(**Q4_EXT, q8_linear=1, bf16_linear=1))
    with pytest.raises(ContractError, match="platform"):
        PackedQ4NativeBackend("hip_gfx1151", _fake_ext(**Q4_EXT))


def _cpu_layer(experts=4, hidden=256, inter=128):
    from uma_qmoe_amd import synthetic as syn

    shape = syn.MoEShape("boundary_cache", hidden, experts, 2, inter)
    return syn.build_experts(shape)


def test_backend_cache_summary_and_release_by_pack():
    backend = PackedQ4NativeBackend("hip_gfx950", _fake_ext(**Q4_EXT))
    first, second = _cpu_layer(), _cpu_layer(experts=6)
    single = ("q4_group128", torch.zeros(64, dtype=torch.uint8), torch.ones(1), (1, 128), 128)
    backend._layer_cache[(1, 0, "cuda:0")] = first
    backend._layer_cache[(2, 0, "cuda:0")] = second
    backend._cache[(1, "w", "cuda:0")] = single
    summary = backend.cache_summary()
    # compressed bytes: Q4 data (1/2 byte per weight) + FP32 scales (1/32 byte per weight), nothing expanded
    per_expert = 3 * 128 * 256 // 2 + 3 * 128 * 256 // 128 * 4
    assert summary == {"tensor_count": 1 + 3 * (4 + 6), "device_storage_bytes": 64 + 4 + (4 + 6) * per_expert,
                       "dequantized_weight_bytes": 0}
    backend.release_pack(1)
    assert set(backend._cache) == set() and set(backend._layer_cache) == {(2, 0, "cuda:0")}
    assert backend.cache_summary()["device_storage_bytes"] == 6 * per_expert
    backend.release_pack(2)
    assert backend.cache_summary() == {"tensor_count": 0, "device_storage_bytes": 0, "dequantized_weight_bytes": 0}


def test_unregister_releases_backend_caches():
    released = []

    class Backend:
        def __call__(self, *a):
            return None

        def release_pack(self, handle):
            released.append(handle)

    register_performance_backend("cpu", Backend())
    try:
        handle = register_expert_pack(_Reader())
        unregister_expert_pack(handle)
        assert handle in released
    finally:
        custom_op.REGISTRY.uninstall("cpu")


def test_mixed_backend_rejects_q4_only_backend_for_other_encodings():
    backend = PackedQ4NativeBackend("hip_gfx950", _fake_ext(**Q4_EXT))
    reader = SimpleNamespace(layer_encoding=lambda layer: "q8_group128")
    with pytest.raises(RuntimeError, match="install the mixed backend"):
        backend._device_layer(1, 0, "cuda:0", reader)


def test_source_identity_is_stable_sha256():
    from uma_qmoe_amd.native_backend import native_kernel_source_sha256

    digest = native_kernel_source_sha256()
    assert re.fullmatch(r"[0-9a-f]{64}", digest)
    assert native_kernel_source_sha256() == digest
