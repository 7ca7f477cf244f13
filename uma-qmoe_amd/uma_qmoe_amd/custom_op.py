"""PyTorch operator boundary for packed-expert MoE execution on MI355X.

Keeps the reference's operator contract (src/uma_qmoe/custom_op.py):
  * schemas ``uma_qmoe::moe_forward`` and ``uma_qmoe::qwen_moe_forward``
    (Tensor hidden_states, Tensor expert_indices, Tensor routing_weights,
    int layer_index, int pack_handle, bool performance_mode=False) -> Tensor,
    implemented for the CPU, CUDA (HIP builds of torch use this key) and Meta
    dispatch keys (custom_op.py:582-628);
  * pack handles with thread-local re-entrant leases; unregister drains active
    calls and refuses inside its own lease (custom_op.py:51-146);
  * explicit install-then-select performance backends; performance mode with
    no backend fails closed (custom_op.py:90-100, 509-579).

New in this build:
  * ``uma_qmoe::moe_block`` — the whole MoE block (router + routed experts +
    optional sigmoid-gated shared expert) as one op, so the router and shared
    expert run in the same HIP pipeline instead of separate torch modules.
  * The platform id of MI355X is ``hip_gfx950``.
  * The correctness mode (performance_mode=False) runs an explicitly
    registered correctness implementation (``register_reference_implementation``).
    None ships with the product; without one the call raises instead of
    computing anything on a fallback path.
"""

from __future__ import annotations

from contextlib import contextmanager
from dataclasses import dataclass
import itertools
import threading
from typing import Any, Callable, Iterator

from .q4 import ContractError

PLATFORMS = frozenset({"cpu", "hip_gfx950"})


@dataclass
class _PackState:
    reader: Any
    active_calls: int = 0
    closing: bool = False


_PACKS: dict[int, _PackState] = {}
_PACK_CONDITION = threading.Condition()
_PACK_IDS = itertools.count(1)
_PACK_LEASES = threading.local()
_LIBRARIES: list[Any] = []
_REGISTERED = False
_PERFORMANCE_BACKENDS: dict[str, Any] = {}
_REFERENCE_IMPLEMENTATIONS: dict[str, Callable[..., Any]] = {}


def register_expert_pack(reader: Any) -> int:
    """Register one pack reader (exactly one mapping) and return its handle."""
    if getattr(reader, "mapping_count", None) != 1:
        raise ContractError("custom operator requires exactly one ExpertPack mapping")
    with _PACK_CONDITION:
        handle = next(_PACK_IDS)
        _PACKS[handle] = _PackState(reader=reader)
    return handle


def register_target_pack(reader: Any) -> int:
    """Register one mixed TargetPack (same contract as register_expert_pack)."""
    return register_expert_pack(reader)


def _lease_counts() -> dict[int, int]:
    counts = getattr(_PACK_LEASES, "counts", None)
    if counts is None:
        counts = {}
        _PACK_LEASES.counts = counts
    return counts


def unregister_expert_pack(handle: int) -> None:
    """Close a handle: wait for active calls to drain, then release backends' caches."""
    if _lease_counts().get(handle, 0):
        raise ContractError("cannot unregister an ExpertPack from its active call")
    with _PACK_CONDITION:
        state = _PACKS.get(handle)
        if state is None:
            return
        if state.closing:
            while handle in _PACKS:
                _PACK_CONDITION.wait()
            return
        state.closing = True
        while state.active_calls:
            _PACK_CONDITION.wait()
        del _PACKS[handle]
        backends = list(_PERFORMANCE_BACKENDS.values())
        _PACK_CONDITION.notify_all()
    for backend in backends:
        release = getattr(backend, "release_pack", None)
        if callable(release):
            release(handle)


def register_performance_backend(platform: str, implementation: Any) -> None:
    """Install an explicit optimised backend; it is never an implicit fallback."""
    if platform not in PLATFORMS:
        raise ContractError(f"unsupported custom operator platform {platform!r}")
    if not callable(implementation):
        raise ContractError("custom operator backend must be callable")
    with _PACK_CONDITION:
        _PERFORMANCE_BACKENDS[platform] = implementation


def performance_backend(platform: str) -> Any:
    with _PACK_CONDITION:
        return _PERFORMANCE_BACKENDS.get(platform)


def register_reference_implementation(kind: str, implementation: Callable[..., Any]) -> None:
    """Install the correctness implementation used when performance_mode=False.

    ``kind`` is ``"olmoe"``, ``"qwen"`` or ``"block"``. The callable receives
    the op's tensors plus the leased pack reader.
    """
    if kind not in {"olmoe", "qwen", "block"}:
        raise ContractError(f"unknown reference implementation kind {kind!r}")
    if not callable(implementation):
        raise ContractError("reference implementation must be callable")
    with _PACK_CONDITION:
        _REFERENCE_IMPLEMENTATIONS[kind] = implementation


def clear_reference_implementations() -> None:
    with _PACK_CONDITION:
        _REFERENCE_IMPLEMENTATIONS.clear()


@contextmanager
def acquire_expert_pack(handle: int) -> Iterator[Any]:
    """Hold one pack open across staging and asynchronous kernel submission."""
    counts = _lease_counts()
    nested = counts.get(handle, 0) > 0
    with _PACK_CONDITION:
        state = _PACKS.get(handle)
        if state is None or (state.closing and not nested):
            raise RuntimeError(f"unknown or closed ExpertPack handle {handle}")
        if not nested:
            state.active_calls += 1
        counts[handle] = counts.get(handle, 0) + 1
    try:
        yield state.reader
    finally:
        with _PACK_CONDITION:
            left = counts[handle] - 1
            if left:
                counts[handle] = left
            else:
                del counts[handle]
                state.active_calls -= 1
                _PACK_CONDITION.notify_all()


def expert_pack_for_handle(handle: int) -> Any:
    """Resolve a registered pack; only valid inside an active lease."""
    if _lease_counts().get(handle, 0) == 0:
        raise RuntimeError("ExpertPack access requires an active operator lease")
    with _PACK_CONDITION:
        state = _PACKS.get(handle)
        if state is None:
            raise RuntimeError(f"unknown or closed ExpertPack handle {handle}")
        return state.reader


def device_platform(torch: Any, tensor: Any) -> str:
    """``cpu`` or ``hip_gfx950``; anything else is rejected (custom_op.py:149-169)."""
    if tensor.device.type == "cpu":
        return "cpu"
    if tensor.device.type != "cuda":
        raise RuntimeError(f"uma_qmoe operators do not support {tensor.device}")
    if not torch.version.hip:
        raise RuntimeError("uma_qmoe MI355X build requires a ROCm (HIP) PyTorch")
    arch = str(getattr(torch.cuda.get_device_properties(tensor.device), "gcnArchName", ""))
    if arch.split(":", 1)[0] != "gfx950":
        raise RuntimeError(f"HIP implementation requires gfx950, observed {arch!r}")
    return "hip_gfx950"


def _reference(kind: str) -> Callable[..., Any]:
    with _PACK_CONDITION:
        impl = _REFERENCE_IMPLEMENTATIONS.get(kind)
    if impl is None:
        raise RuntimeError(
            f"uma_qmoe correctness mode has no registered {kind} implementation; "
            "pass performance_mode=True to run the HIP backend"
        )
    return impl


def _dispatch(hidden_states, expert_indices, routing_weights, layer_index, pack_handle, performance_mode=False):
    import torch

    with acquire_expert_pack(pack_handle) as reader:
        platform = device_platform(torch, hidden_states)
        if performance_mode:
            backend = performance_backend(platform)
            if backend is None:
                raise RuntimeError(
                    f"performance mode has no registered {platform} backend; silent reference fallback is forbidden"
                )
            return backend(hidden_states, expert_indices, routing_weights, layer_index, pack_handle)
        return _reference("olmoe")(hidden_states, expert_indices, routing_weights, layer_index, reader)


def _qwen_dispatch(hidden_states, expert_indices, routing_weights, layer_index, pack_handle, performance_mode=False):
    import torch

    with acquire_expert_pack(pack_handle) as reader:
        platform = device_platform(torch, hidden_states)
        if performance_mode:
            qwen_forward = getattr(performance_backend(platform), "qwen_forward", None)
            if not callable(qwen_forward):
                raise RuntimeError(
                    f"performance mode has no Qwen-capable {platform} backend; silent reference fallback is forbidden"
                )
            return qwen_forward(hidden_states, expert_indices, routing_weights, layer_index, pack_handle)
        return _reference("qwen")(hidden_states, expert_indices, routing_weights, layer_index, reader)


def _block_dispatch(
    hidden_states,
    router_weight,
    shared_gate_proj,
    shared_up_proj,
    shared_down_proj,
    shared_expert_gate,
    top_k,
    norm_topk_prob,
    layer_index,
    pack_handle,
    performance_mode=False,
):
    import torch

    args = (
        hidden_states,
        router_weight,
        shared_gate_proj,
        shared_up_proj,
        shared_down_proj,
        shared_expert_gate,
        top_k,
        norm_topk_prob,
        layer_index,
        pack_handle,
    )
    with acquire_expert_pack(pack_handle) as reader:
        platform = device_platform(torch, hidden_states)
        if performance_mode:
            block = getattr(performance_backend(platform), "moe_block", None)
            if not callable(block):
                raise RuntimeError(
                    f"performance mode has no block-capable {platform} backend; silent reference fallback is forbidden"
                )
            return block(*args)
        return _reference("block")(*args[:-1], reader)


def _block_meta(hidden_states, router_weight, *_rest):
    top_k = _rest[4]
    flat = hidden_states.reshape(-1, hidden_states.shape[-1])
    t = flat.shape[0]
    e = router_weight.shape[0]
    return (
        hidden_states.new_empty(hidden_states.shape),
        hidden_states.new_empty((t, e)),
        hidden_states.new_empty((t, top_k)),
        hidden_states.new_empty((t, top_k), dtype=__import__("torch").int64),
    )


def register_moe_forward() -> None:
    """Register the uma_qmoe ops once (idempotent, under the registry lock)."""
    global _REGISTERED
    with _PACK_CONDITION:
        if _REGISTERED:
            return
        import torch

        definition = torch.library.Library("uma_qmoe", "DEF")
        definition.define(
            "moe_forward(Tensor hidden_states, Tensor expert_indices, Tensor routing_weights, "
            "int layer_index, int pack_handle, bool performance_mode=False) -> Tensor"
        )
        definition.define(
            "qwen_moe_forward(Tensor hidden_states, Tensor expert_indices, Tensor routing_weights, "
            "int layer_index, int pack_handle, bool performance_mode=False) -> Tensor"
        )
        definition.define(
            "moe_block(Tensor hidden_states, Tensor router_weight, Tensor? shared_gate_proj, "
            "Tensor? shared_up_proj, Tensor? shared_down_proj, Tensor? shared_expert_gate, int top_k, "
            "bool norm_topk_prob, int layer_index, int pack_handle, bool performance_mode=False) "
            "-> (Tensor, Tensor, Tensor, Tensor)"
        )
        for key in ("CPU", "CUDA"):
            impl = torch.library.Library("uma_qmoe", "IMPL", key)
            impl.impl("moe_forward", _dispatch)
            impl.impl("qwen_moe_forward", _qwen_dispatch)
            impl.impl("moe_block", _block_dispatch)
            _LIBRARIES.append(impl)
        meta = torch.library.Library("uma_qmoe", "IMPL", "Meta")
        meta.impl("moe_forward", lambda hidden_states, *_a: hidden_states.new_empty(hidden_states.shape))
        meta.impl("qwen_moe_forward", lambda hidden_states, *_a: hidden_states.new_empty(hidden_states.shape))
        meta.impl("moe_block", _block_meta)
        _LIBRARIES.extend((definition, meta))
        _REGISTERED = True


__all__ = [
    "acquire_expert_pack",
    "clear_reference_implementations",
    "device_platform",
    "expert_pack_for_handle",
    "performance_backend",
    "register_expert_pack",
    "register_moe_forward",
    "register_performance_backend",
    "register_reference_implementation",
    "register_target_pack",
    "unregister_expert_pack",
]
