"""PyTorch operator boundary for packed-expert MoE execution on MI355X.

The contract kept from the reference (src/uma_qmoe/custom_op.py):
  * op schemas ``uma_qmoe::moe_forward`` and ``uma_qmoe::qwen_moe_forward``
    (Tensor hidden_states, Tensor expert_indices, Tensor routing_weights,
    int layer_index, int pack_handle, bool performance_mode=False) -> Tensor,
    implemented for the CPU, CUDA (HIP builds of torch use this key) and Meta
    dispatch keys, registered once (custom_op.py:582-628);
  * integer pack handles from ``register_expert_pack`` /
    ``register_target_pack`` for readers with exactly one mapping; leases
    that are re-entrant per thread; ``unregister_expert_pack`` refuses inside
    the caller's own lease, waits for other active calls and then makes the
    installed backends release their device copies (custom_op.py:51-146);
  * explicit install-then-select performance backends per platform, and a
    performance-mode call without one fails closed with "silent reference
    fallback is forbidden" (custom_op.py:90-100, 509-579).

Different here:
  * ``uma_qmoe::moe_block`` runs the whole MoE block (router, routed experts,
    sigmoid-gated shared expert) as one op, so the router and the shared
    expert run in the same HIP pipeline;
  * the MI355X platform is ``hip_gfx950``;
  * performance_mode=False on HIP tensors runs the library's correctness
    path (``native_backend.CorrectnessPath``: the layer's experts dequantised
    transiently to BF16 by a HIP kernel, then the BF16 expert kernels), as the
    reference computes its streaming correctness path there
    (custom_op.py:509-579). An implementation installed with
    ``register_reference_implementation`` takes its place (tests install the
    CPU oracle this way); CPU tensors need one, since this build runs no
    expert arithmetic on the CPU.
"""

from __future__ import annotations

from collections import Counter
from contextlib import contextmanager
from dataclasses import dataclass
import itertools
import threading
from typing import Any, Callable, Iterator

from .formats import ContractError

PLATFORMS = frozenset({"cpu", "hip_gfx950"})
REFERENCE_KINDS = frozenset({"olmoe", "qwen", "block"})


@dataclass
class _Pack:
    reader: Any
    active: int = 0  # calls (threads) holding a lease
    closing: bool = False


class PackRegistry:
    """Registered pack readers, the per-thread leases on them, and the
    backends that hold device copies of their tensors.

    A lease counts once per thread however deeply it nests. Closing a handle
    refuses new leases from other calls, waits until the active ones end,
    forgets the handle and asks every installed backend to release it.
    """

    def __init__(self) -> None:
        self._cond = threading.Condition()
        self._ids = itertools.count(1)
        self._packs: dict[int, _Pack] = {}
        self._tls = threading.local()
        self.backends: dict[str, Any] = {}
        self.references: dict[str, Callable[..., Any]] = {}

    def held(self) -> Counter:
        """This thread's lease depth per handle."""
        depth = getattr(self._tls, "depth", None)
        if depth is None:
            depth = self._tls.depth = Counter()
        return depth

    def register(self, reader: Any) -> int:
        if getattr(reader, "mapping_count", None) != 1:
            raise ContractError("custom operator requires exactly one ExpertPack mapping")
        with self._cond:
            handle = next(self._ids)
            self._packs[handle] = _Pack(reader)
            return handle

    @contextmanager
    def lease(self, handle: int) -> Iterator[Any]:
        depth = self.held()
        outer = depth[handle] == 0
        with self._cond:
            pack = self._packs.get(handle)
            if pack is None or (pack.closing and outer):
                raise RuntimeError(f"unknown or closed ExpertPack handle {handle}")
            if outer:
                pack.active += 1
            depth[handle] += 1
        try:
            yield pack.reader
        finally:
            with self._cond:
                depth[handle] -= 1
                if depth[handle] == 0:
                    del depth[handle]
                    pack.active -= 1
                    self._cond.notify_all()

    def resolve(self, handle: int) -> Any:
        if self.held()[handle] == 0:
            raise RuntimeError("ExpertPack access requires an active operator lease")
        with self._cond:
            pack = self._packs.get(handle)
            if pack is None:
                raise RuntimeError(f"unknown or closed ExpertPack handle {handle}")
            return pack.reader

    def close(self, handle: int) -> None:
        if self.held()[handle]:
            raise ContractError("cannot unregister an ExpertPack from its active call")
        with self._cond:
            pack = self._packs.get(handle)
            if pack is None:
                return
            if pack.closing:  # another thread is closing it: wait for that
                self._cond.wait_for(lambda: handle not in self._packs)
                return
            pack.closing = True
            self._cond.wait_for(lambda: pack.active == 0)
            del self._packs[handle]
            backends = list(self.backends.values())
            self._cond.notify_all()
        for backend in backends:
            release = getattr(backend, "release_pack", None)
            if callable(release):
                release(handle)

    def install(self, platform: str, backend: Any) -> None:
        if platform not in PLATFORMS:
            raise ContractError(f"unsupported custom operator platform {platform!r}")
        if not callable(backend):
            raise ContractError("custom operator backend must be callable")
        with self._cond:
            self.backends[platform] = backend

    def backend(self, platform: str) -> Any:
        with self._cond:
            return self.backends.get(platform)

    def uninstall(self, platform: str) -> None:
        with self._cond:
            self.backends.pop(platform, None)

    def set_reference(self, kind: str, implementation: Callable[..., Any]) -> None:
        if kind not in REFERENCE_KINDS:
            raise ContractError(f"unknown reference implementation kind {kind!r}")
        if not callable(implementation):
            raise ContractError("reference implementation must be callable")
        with self._cond:
            self.references[kind] = implementation

    def reference(self, kind: str) -> Callable[..., Any] | None:
        with self._cond:
            return self.references.get(kind)


REGISTRY = PackRegistry()


# Reference-named entry points (src/uma_qmoe/custom_op.py:51-146).
def register_expert_pack(reader: Any) -> int:
    """Register one pack reader (exactly one mapping); returns its handle."""
    return REGISTRY.register(reader)


def register_target_pack(reader: Any) -> int:
    """Register one mixed TargetPack (same contract as register_expert_pack)."""
    return REGISTRY.register(reader)


def unregister_expert_pack(handle: int) -> None:
    """Close a handle once its active calls drain; backends drop its tensors."""
    REGISTRY.close(handle)


@contextmanager
def acquire_expert_pack(handle: int) -> Iterator[Any]:
    """Hold one pack open across staging and asynchronous kernel submission."""
    with REGISTRY.lease(handle) as reader:
        yield reader


def expert_pack_for_handle(handle: int) -> Any:
    """The registered reader of a handle; only inside an active lease."""
    return REGISTRY.resolve(handle)


def register_performance_backend(platform: str, implementation: Any) -> None:
    """Install an explicit optimised backend; it is never an implicit fallback."""
    REGISTRY.install(platform, implementation)


def performance_backend(platform: str) -> Any:
    return REGISTRY.backend(platform)


def register_reference_implementation(kind: str, implementation: Callable[..., Any]) -> None:
    """Install the correctness implementation of performance_mode=False, in
    place of the library's own (which runs on HIP tensors only).

    ``kind`` is ``"olmoe"`` (moe_forward), ``"qwen"`` (qwen_moe_forward) or
    ``"block"`` (moe_block). It is called with the op's arguments, the pack
    handle replaced by the leased reader.
    """
    REGISTRY.set_reference(kind, implementation)


def clear_reference_implementations() -> None:
    with REGISTRY._cond:
        REGISTRY.references.clear()


def device_platform(torch: Any, tensor: Any) -> str:
    """``cpu`` or ``hip_gfx950``; any other device is rejected (custom_op.py:149-169)."""
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


# What each op runs in performance mode: the backend attribute (None: the
# backend object itself) and the words of its fail-closed error.
_OPS = {
    "olmoe": (None, "registered"),
    "qwen": ("qwen_forward", "Qwen-capable"),
    "block": ("moe_block", "block-capable"),
}


def _run(kind: str, hidden_states: Any, args: tuple, pack_handle: int, performance_mode: bool) -> Any:
    import torch

    with REGISTRY.lease(pack_handle) as reader:
        platform = device_platform(torch, hidden_states)
        if not performance_mode:
            impl = REGISTRY.reference(kind)
            if impl is not None:
                return impl(hidden_states, *args, reader)
            if platform != "hip_gfx950":
                raise RuntimeError(f"uma_qmoe correctness mode on {platform} tensors has no registered {kind} "
                                   "implementation; the built-in correctness path runs on hip_gfx950 devices")
            from .native_backend import correctness_forward

            return correctness_forward(kind, hidden_states, args, reader)
        attr, words = _OPS[kind]
        backend = REGISTRY.backend(platform)
        fn = backend if attr is None else getattr(backend, attr, None)
        if fn is None or not callable(fn):
            raise RuntimeError(f"performance mode has no {words} {platform} backend; "
                               "silent reference fallback is forbidden")
        return fn(hidden_states, *args, pack_handle)


def _dispatch(hidden_states, expert_indices, routing_weights, layer_index, pack_handle, performance_mode=False):
    return _run("olmoe", hidden_states, (expert_indices, routing_weights, layer_index), pack_handle, performance_mode)


def _qwen_dispatch(hidden_states, expert_indices, routing_weights, layer_index, pack_handle, performance_mode=False):
    return _run("qwen", hidden_states, (expert_indices, routing_weights, layer_index), pack_handle, performance_mode)


def _block_dispatch(hidden_states, router_weight, shared_gate_proj, shared_up_proj, shared_down_proj,
                    shared_expert_gate, top_k, norm_topk_prob, layer_index, pack_handle, performance_mode=False):
    args = (router_weight, shared_gate_proj, shared_up_proj, shared_down_proj, shared_expert_gate, top_k,
            norm_topk_prob, layer_index)
    return _run("block", hidden_states, args, pack_handle, performance_mode)


def _same_shape(hidden_states, *_rest):
    return hidden_states.new_empty(hidden_states.shape)


def _block_meta(hidden_states, router_weight, *rest):
    import torch

    top_k = rest[4]
    t = hidden_states.reshape(-1, hidden_states.shape[-1]).shape[0]
    return (hidden_states.new_empty(hidden_states.shape), hidden_states.new_empty((t, router_weight.shape[0])),
            hidden_states.new_empty((t, top_k)), hidden_states.new_empty((t, top_k), dtype=torch.int64))


_SCHEMAS = {
    "moe_forward": ("(Tensor hidden_states, Tensor expert_indices, Tensor routing_weights, int layer_index, "
                    "int pack_handle, bool performance_mode=False) -> Tensor", _dispatch, _same_shape),
    "qwen_moe_forward": ("(Tensor hidden_states, Tensor expert_indices, Tensor routing_weights, int layer_index, "
                         "int pack_handle, bool performance_mode=False) -> Tensor", _qwen_dispatch, _same_shape),
    "moe_block": ("(Tensor hidden_states, Tensor router_weight, Tensor? shared_gate_proj, Tensor? shared_up_proj, "
                  "Tensor? shared_down_proj, Tensor? shared_expert_gate, int top_k, bool norm_topk_prob, "
                  "int layer_index, int pack_handle, bool performance_mode=False) -> (Tensor, Tensor, Tensor, Tensor)",
                  _block_dispatch, _block_meta),
}
_LIBRARIES: list[Any] = []


def register_moe_forward() -> None:
    """Define and implement the uma_qmoe ops once (idempotent, under a lock)."""
    with REGISTRY._cond:
        if _LIBRARIES:
            return
        import torch

        libs = {key: torch.library.Library("uma_qmoe", kind, *(() if key == "DEF" else (key,)))
                for key, kind in (("DEF", "DEF"), ("CPU", "IMPL"), ("CUDA", "IMPL"), ("Meta", "IMPL"))}
        for name, (schema, impl, meta) in _SCHEMAS.items():
            libs["DEF"].define(name + schema)
            libs["CPU"].impl(name, impl)
            libs["CUDA"].impl(name, impl)
            libs["Meta"].impl(name, meta)
        _LIBRARIES.extend(libs.values())


__all__ = [
    "REGISTRY",
    "PackRegistry",
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
