"""Explicit MI355X (gfx950) performance backends for packed MoE experts.

Same install-then-select flow and backend protocol as the reference's
src/uma_qmoe/native_backend.py:
  * ``install_packed_q4_backend()`` / ``install_mixed_target_backend()`` load
    the prebuilt HIP library and register a backend for platform
    ``hip_gfx950``; nothing is selected until a call passes
    ``performance_mode=True`` (native_backend.py:1141-1154);
  * a backend is callable as ``backend(hidden, indices, weights, layer, handle)``
    (OLMoE op) and exposes ``qwen_forward`` (Qwen op), ``release_pack``,
    ``cache_summary`` (native_backend.py:457-552) and, new here, ``moe_block``;
  * expert tensors are staged once per (pack, layer, device) in their
    compressed form, expert-major (native_backend.py:374-455); the
    dequantized-weight cache is always zero bytes.

What changes is everything below the Python surface: the reference runs a
Python loop over hit experts with one host sync and three GEMV launches per
expert for Qwen (native_backend.py:319-372, 722-753) and compile-time OLMoE
shapes elsewhere; here every call is one C-ABI call into libuma_qmoe_hip.so
(include/uma_qmoe_hip.h) that keeps the routing on the device, for any E, k,
H and I.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
import hashlib
from pathlib import Path
import threading
from typing import Any

from . import _native
from .build import CSRC
from .custom_op import acquire_expert_pack, register_performance_backend
from .formats import ENCODINGS, ContractError

EXPERT_NAME = "model.layers.{layer}.mlp.experts.{expert}.{proj}.weight"
PROJECTIONS = ("gate_proj", "up_proj", "down_proj")
PLATFORM = "hip_gfx950"

_EXTENSIONS: dict[str, Any] = {}
_BUILD_LOCK = threading.Lock()


def native_kernel_source_sha256() -> str:
    """SHA-256 over the HIP sources (name, NUL, bytes), as native_backend.py:32-38."""
    digest = hashlib.sha256()
    for path in sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.h")):
        digest.update(path.name.encode("utf-8"))
        digest.update(b"\0")
        digest.update(path.read_bytes())
    return digest.hexdigest()


def observed_native_platform(torch: Any, device: Any = 0) -> str:
    if not torch.cuda.is_available():
        raise ContractError("packed MoE native backend requires a HIP device")
    if not torch.version.hip:
        raise ContractError("packed MoE native backend requires a ROCm build of PyTorch")
    arch = str(getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")).split(":", 1)[0]
    if arch != "gfx950":
        raise ContractError(f"packed MoE HIP backend requires gfx950, got {arch!r}")
    return PLATFORM


def _stream_handle(torch: Any, device: Any) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def _ptr(t: Any) -> int | None:
    return None if t is None else int(t.data_ptr())


@dataclass(frozen=True)
class DeviceExperts:
    """One layer's routed experts, compressed, expert-major on one device.

    gate/up: [E, I, row_bytes(H)], down: [E, H, row_bytes(I)] (uint8 for Q4,
    int8 for Q8, bfloat16 for BF16); scales float32 [E, rows*cols/group].
    """

    encoding: str
    group_size: int
    num_experts: int
    hidden_size: int
    intermediate_size: int
    gate: Any
    gate_scales: Any
    up: Any
    up_scales: Any
    down: Any
    down_scales: Any

    @property
    def tensors(self) -> tuple[Any, ...]:
        return tuple(t for t in (self.gate, self.gate_scales, self.up, self.up_scales, self.down, self.down_scales) if t is not None)

    @property
    def device_storage_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.tensors)

    def bytes_per_expert(self) -> int:
        return self.device_storage_bytes // self.num_experts

    def descriptor(self) -> _native.ExpertWeights:
        return _native.ExpertWeights(
            _native.ENCODING_IDS[self.encoding],
            self.group_size if self.encoding != "bf16_le" else 0,
            self.num_experts,
            self.hidden_size,
            self.intermediate_size,
            _ptr(self.gate),
            _ptr(self.gate_scales),
            _ptr(self.up),
            _ptr(self.up_scales),
            _ptr(self.down),
            _ptr(self.down_scales),
        )


@dataclass(frozen=True)
class DenseBlock:
    """BF16 dense tensors of one MoE block (router and optional shared expert)."""

    router: Any  # [E, H]
    shared_gate: Any = None  # [Is, H]
    shared_up: Any = None  # [Is, H]
    shared_down: Any = None  # [H, Is]
    shared_expert_gate: Any = None  # [1, H]

    @property
    def has_shared(self) -> bool:
        return self.shared_gate is not None


class HipExtension:
    """torch-facing wrappers over the C ABI, named like the reference binding's
    entry points (src/uma_qmoe/native/packed_q4_binding.cpp:490-515)."""

    def __init__(self) -> None:
        import torch

        self.torch = torch
        self.lib = _native.library()
        self._ws_lock = threading.Lock()
        self._ws_cache: dict[tuple[int, int], Any] = {}

    # ------------------------------------------------------------ helpers --
    def _workspace(self, device, tokens, hidden, inter, shared_inter, experts, top_k):
        """A zero-filled workspace of the size the library asks for, reused by
        later calls on the same device and stream (stream order keeps them
        from overlapping; the fused single-token kernel leaves its sync words
        ready for the next call). It grows when a call needs more."""
        n = self.lib.uqm_moe_workspace_bytes(tokens, hidden, inter, shared_inter, experts, top_k)
        if n == 0:
            raise RuntimeError("invalid workspace shape")
        torch = self.torch
        dev = torch.device(device)
        key = (dev.index if dev.index is not None else torch.cuda.current_device(), _stream_handle(torch, dev))
        with self._ws_lock:
            ws = self._ws_cache.get(key)
            if ws is None or ws.numel() < n:
                # Zero-filling inside a HIP-graph capture would record the
                # fill, and every replay would reset the fused kernel's launch
                # epochs (stale hand-offs would then look current).
                if torch.cuda.is_current_stream_capturing():
                    raise RuntimeError("uma_qmoe workspace would be allocated inside a HIP-graph capture: run one "
                                       "call of this shape on the capture stream before capturing")
                ws = torch.zeros(n, dtype=torch.uint8, device=dev)
                self._ws_cache[key] = ws
            return ws

    def new_workspace(self, device, tokens, hidden, inter, shared_inter, experts, top_k):
        """A fresh zero-filled workspace owned by the caller (not the shared cache)."""
        n = self.lib.uqm_moe_workspace_bytes(tokens, hidden, inter, shared_inter, experts, top_k)
        if n == 0:
            raise RuntimeError("invalid workspace shape")
        return self.torch.zeros(n, dtype=self.torch.uint8, device=device)

    def _check_hidden(self, hidden):
        torch = self.torch
        if hidden.dtype != torch.bfloat16:
            raise RuntimeError("uma_qmoe HIP kernels require BF16 hidden states")
        if not hidden.is_cuda:
            raise RuntimeError("uma_qmoe HIP kernels require device tensors")

    # ------------------------------------------------------------ linears --
    def _linear(self, fn, input_tensor, w, s, out_features, in_features, group_size):
        torch = self.torch
        self._check_hidden(input_tensor)
        x = input_tensor.reshape(-1, in_features).contiguous()
        out = torch.empty((x.shape[0], out_features), dtype=torch.bfloat16, device=x.device)
        rc = fn(_ptr(x), x.shape[0], _ptr(w), _ptr(s), out_features, in_features, group_size, _ptr(out),
                _stream_handle(torch, x.device))
        _native.check(rc, fn.__name__)
        return out.reshape(*input_tensor.shape[:-1], out_features)

    def q4_linear(self, input_tensor, packed, scales, output_features, input_features, group_size):
        return self._linear(self.lib.uqm_q4_linear, input_tensor, packed, scales, output_features, input_features, group_size)

    def q8_linear(self, input_tensor, quantized, scales, output_features, input_features, group_size):
        return self._linear(self.lib.uqm_q8_linear, input_tensor, quantized, scales, output_features, input_features, group_size)

    def bf16_linear(self, input_tensor, weight):
        torch = self.torch
        self._check_hidden(input_tensor)
        out_features, in_features = weight.shape
        x = input_tensor.reshape(-1, in_features).contiguous()
        out = torch.empty((x.shape[0], out_features), dtype=torch.bfloat16, device=x.device)
        rc = self.lib.uqm_bf16_linear(_ptr(x), x.shape[0], _ptr(weight.contiguous()), out_features, in_features,
                                      _ptr(out), _stream_handle(torch, x.device))
        _native.check(rc, "uqm_bf16_linear")
        return out.reshape(*input_tensor.shape[:-1], out_features)

    # ------------------------------------------------------ dequantisation --
    def dequantize(self, data, scales, encoding: str, group_size: int):
        """bf16(q * scale) of every value of an encoded Q4 or Q8 tensor, flat
        (the library's HIP kernel; the reference's correctness path
        dequantises the same way, q4.py:168-179 then .to(bfloat16))."""
        torch = self.torch
        if encoding not in ("q4_group128", "q8_group128"):
            raise RuntimeError(f"cannot dequantize a {encoding} tensor")
        data = data.contiguous()
        n = data.numel() * (2 if encoding == "q4_group128" else 1)
        out = torch.empty(n, dtype=torch.bfloat16, device=data.device)
        rc = self.lib.uqm_dequantize(_native.ENCODING_IDS[encoding], _ptr(data), _ptr(scales.contiguous()), n,
                                     int(group_size), _ptr(out), _stream_handle(torch, data.device))
        _native.check(rc, "uqm_dequantize")
        return out

    def bf16_experts(self, layer: DeviceExperts) -> DeviceExperts:
        """The layer with every expert dequantised to BF16 (a transient copy:
        nothing keeps it after the caller drops it); a BF16 layer as is."""
        if layer.encoding == "bf16_le":
            return layer
        E, H, I = layer.num_experts, layer.hidden_size, layer.intermediate_size

        def deq(data, scales, rows, cols):
            return self.dequantize(data, scales, layer.encoding, layer.group_size).view(E, rows, cols)

        return DeviceExperts("bf16_le", layer.group_size, E, H, I, deq(layer.gate, layer.gate_scales, I, H), None,
                             deq(layer.up, layer.up_scales, I, H), None, deq(layer.down, layer.down_scales, H, I),
                             None)

    # ------------------------------------------------------------ routing --
    def route_permute(self, expert_indices, num_experts):
        """(route_order int64 [T*k], expert_offsets int64 [E+1]) on the device."""
        torch = self.torch
        idx = expert_indices.to(torch.int64).contiguous()
        t, k = idx.shape
        order = torch.empty(t * k, dtype=torch.int64, device=idx.device)
        offsets = torch.empty(num_experts + 1, dtype=torch.int64, device=idx.device)
        ws = self._workspace(idx.device, t, 8, 8, 0, num_experts, k)
        rc = self.lib.uqm_route_permute(_ptr(idx), t, k, num_experts, _ptr(order), _ptr(offsets), _ptr(ws), ws.numel(),
                                        _stream_handle(torch, idx.device))
        _native.check(rc, "uqm_route_permute")
        return order, offsets

    def router_topk(self, hidden, router_weight, top_k, norm_topk_prob=False):
        torch = self.torch
        self._check_hidden(hidden)
        e, h = router_weight.shape
        x = hidden.reshape(-1, h).contiguous()
        t = x.shape[0]
        logits = torch.empty((t, e), dtype=torch.bfloat16, device=x.device)
        weights = torch.empty((t, top_k), dtype=torch.bfloat16, device=x.device)
        indices = torch.empty((t, top_k), dtype=torch.int64, device=x.device)
        ws = self._workspace(x.device, t, h, 8, 0, e, top_k)
        rc = self.lib.uqm_router_topk(_ptr(x), t, h, _ptr(router_weight.contiguous()), e, top_k, int(bool(norm_topk_prob)),
                                      _ptr(logits), _ptr(weights), _ptr(indices), _ptr(ws), ws.numel(),
                                      _stream_handle(torch, x.device))
        _native.check(rc, "uqm_router_topk")
        return logits, weights, indices

    # ------------------------------------------------------------ experts --
    def moe_forward(self, layer: DeviceExperts, hidden, expert_indices, routing_weights, *, out=None, workspace=None):
        torch = self.torch
        self._check_hidden(hidden)
        x = hidden.reshape(-1, layer.hidden_size).contiguous()
        t = x.shape[0]
        if expert_indices.ndim != 2 or expert_indices.shape[0] != t or tuple(routing_weights.shape) != tuple(expert_indices.shape):
            raise RuntimeError("expert_indices and routing_weights must both be [tokens, top_k]")
        if expert_indices.dtype not in (torch.int32, torch.int64):
            raise RuntimeError("expert_indices must use int32 or int64")
        k = expert_indices.shape[1]
        idx = expert_indices.to(torch.int64).contiguous()
        w = routing_weights.to(torch.bfloat16).contiguous()
        out = torch.empty_like(x) if out is None else out
        ws = workspace
        if ws is None:
            ws = self._workspace(x.device, t, layer.hidden_size, layer.intermediate_size, 0, layer.num_experts, k)
        desc = layer.descriptor()
        rc = self.lib.uqm_moe_forward(ctypes.byref(desc), _ptr(x), t, _ptr(idx), _ptr(w), k, _ptr(out), _ptr(ws),
                                      ws.numel(), _stream_handle(torch, x.device))
        _native.check(rc, "uqm_moe_forward")
        return out.reshape(hidden.shape)

    def moe_layer(self, layer: DeviceExperts, dense: DenseBlock, hidden, top_k, norm_topk_prob=False, *,
                  out=None, workspace=None):
        """Router + routed experts (+ shared expert). Returns (out, logits, weights, indices)."""
        torch = self.torch
        self._check_hidden(hidden)
        x = hidden.reshape(-1, layer.hidden_size).contiguous()
        t = x.shape[0]
        e = layer.num_experts
        shared_i = int(dense.shared_gate.shape[0]) if dense.has_shared else 0
        result = torch.empty_like(x) if out is None else out
        logits = torch.empty((t, e), dtype=torch.bfloat16, device=x.device)
        weights = torch.empty((t, top_k), dtype=torch.bfloat16, device=x.device)
        indices = torch.empty((t, top_k), dtype=torch.int64, device=x.device)
        ws = workspace
        if ws is None:
            ws = self._workspace(x.device, t, layer.hidden_size, layer.intermediate_size, shared_i, e, top_k)
        desc = self.layer_descriptor(layer, dense, top_k, norm_topk_prob)
        rc = self.lib.uqm_moe_layer(ctypes.byref(desc), _ptr(x), t, _ptr(result), _ptr(logits), _ptr(weights),
                                    _ptr(indices), _ptr(ws), ws.numel(), _stream_handle(torch, x.device))
        _native.check(rc, "uqm_moe_layer")
        return result.reshape(hidden.shape), logits, weights, indices

    def moe_layer_noalloc(self, layer: DeviceExperts, dense: DenseBlock, hidden, top_k, norm_topk_prob=False, *,
                          out=None, logits=None, weights=None, indices=None):
        """``moe_layer`` through uqm_moe_layer_noalloc: the library's static
        scratch array instead of a workspace. Outputs may be passed in, so a
        caller that cannot allocate passes every tensor."""
        torch = self.torch
        self._check_hidden(hidden)
        x = hidden.reshape(-1, layer.hidden_size).contiguous()
        t, e = x.shape[0], layer.num_experts
        out = torch.empty_like(x) if out is None else out
        logits = torch.empty((t, e), dtype=torch.bfloat16, device=x.device) if logits is None else logits
        weights = torch.empty((t, top_k), dtype=torch.bfloat16, device=x.device) if weights is None else weights
        indices = torch.empty((t, top_k), dtype=torch.int64, device=x.device) if indices is None else indices
        desc = self.layer_descriptor(layer, dense, top_k, norm_topk_prob)
        rc = self.lib.uqm_moe_layer_noalloc(ctypes.byref(desc), _ptr(x), t, _ptr(out), _ptr(logits), _ptr(weights),
                                            _ptr(indices), _stream_handle(torch, x.device))
        _native.check(rc, "uqm_moe_layer_noalloc")
        return out.reshape(hidden.shape), logits, weights, indices

    def norm_moe_layer(self, layer: DeviceExperts, dense: DenseBlock, hidden, top_k, eps=1e-6, norm_weight=None,
                       norm_topk_prob=False, *, out=None, workspace=None):
        """MoE block on RMSNorm(hidden) (eps, bf16 weight [H] or None for ones).
        Returns (out, logits, weights, indices) like ``moe_layer``."""
        torch = self.torch
        self._check_hidden(hidden)
        x = hidden.reshape(-1, layer.hidden_size).contiguous()
        t = x.shape[0]
        e = layer.num_experts
        shared_i = int(dense.shared_gate.shape[0]) if dense.has_shared else 0
        result = torch.empty_like(x) if out is None else out
        logits = torch.empty((t, e), dtype=torch.bfloat16, device=x.device)
        weights = torch.empty((t, top_k), dtype=torch.bfloat16, device=x.device)
        indices = torch.empty((t, top_k), dtype=torch.int64, device=x.device)
        ws = workspace
        if ws is None:
            ws = self._workspace(x.device, t, layer.hidden_size, layer.intermediate_size, shared_i, e, top_k)
        if norm_weight is not None:
            if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != layer.hidden_size:
                raise RuntimeError("norm_weight must be bf16 [hidden_size]")
            norm_weight = norm_weight.contiguous()
        desc = self.layer_descriptor(layer, dense, top_k, norm_topk_prob)
        rc = self.lib.uqm_norm_moe_layer(ctypes.byref(desc), _ptr(x), t, _ptr(norm_weight), float(eps), _ptr(result),
                                         _ptr(logits), _ptr(weights), _ptr(indices), _ptr(ws), ws.numel(),
                                         _stream_handle(torch, x.device))
        _native.check(rc, "uqm_norm_moe_layer")
        return result.reshape(hidden.shape), logits, weights, indices

    @staticmethod
    def layer_descriptor(layer: DeviceExperts, dense: DenseBlock, top_k: int, norm_topk_prob=False) -> _native.LayerWeights:
        shared_i = int(dense.shared_gate.shape[0]) if dense.has_shared else 0
        return _native.LayerWeights(
            layer.descriptor(),
            _ptr(dense.router),
            int(top_k),
            int(bool(norm_topk_prob)),
            int(dense.has_shared),
            shared_i,
            _ptr(dense.shared_gate),
            _ptr(dense.shared_up),
            _ptr(dense.shared_down),
            _ptr(dense.shared_expert_gate),
        )

    def set_option(self, option: int, value: int) -> None:
        _native.check(self.lib.uqm_set_option(int(option), int(value)), "uqm_set_option")

    def workspace_status(self, workspace) -> None:
        """Raises if a fused launch on ``workspace`` hit its wait bound."""
        torch = self.torch
        rc = self.lib.uqm_workspace_status(_ptr(workspace), workspace.numel(), _stream_handle(torch, workspace.device))
        _native.check(rc, "uqm_workspace_status")

    def noalloc_status(self, device=None) -> None:
        """Raises if a fused launch through ``moe_layer_noalloc`` on ``device``
        (default: the current one) hit its wait bound; clears the report."""
        torch = self.torch
        dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
        with torch.cuda.device(dev):
            _native.check(self.lib.uqm_noalloc_status(_stream_handle(torch, dev)), "uqm_noalloc_status")

    def rmsnorm(self, hidden, eps=1e-6, weight=None):
        torch = self.torch
        self._check_hidden(hidden)
        h = hidden.shape[-1]
        x = hidden.reshape(-1, h).contiguous()
        out = torch.empty_like(x)
        rc = self.lib.uqm_rmsnorm(_ptr(x), x.shape[0], h, _ptr(weight), float(eps), _ptr(out),
                                  _stream_handle(torch, x.device))
        _native.check(rc, "uqm_rmsnorm")
        return out.reshape(hidden.shape)

    # ------------------------------------- reference binding signatures --
    def _fixed(self, encoding, hidden, indices, weights, gate, gate_scales, up, up_scales, down, down_scales,
               group_size, num_experts):
        h = hidden.shape[-1]
        if num_experts is None:
            if gate.ndim < 2:
                raise RuntimeError("pass num_experts for flat expert tensors")
            num_experts = int(gate.shape[0])
        per_expert = gate.numel() // num_experts
        bytes_per_weight = {"q4_group128": 0.5, "q8_group128": 1, "bf16_le": 1}[encoding]
        inter = int(per_expert / bytes_per_weight) // h
        layer = DeviceExperts(encoding, int(group_size), int(num_experts), int(h), inter, gate, gate_scales, up, up_scales,
                              down, down_scales)
        return self.moe_forward(layer, hidden, indices, weights)

    def q4_moe_forward(self, hidden, indices, weights, gate_packed, gate_scales, up_packed, up_scales, down_packed,
                       down_scales, group_size, *, num_experts=None):
        """Routed experts of any token count (the route permutation is built
        on the device; packed_q4_binding.cpp:197-347 took host-built tables
        for prefill)."""
        return self._fixed("q4_group128", hidden, indices, weights, gate_packed, gate_scales, up_packed, up_scales,
                           down_packed, down_scales, group_size, num_experts)

    def q8_moe_forward(self, hidden, indices, weights, gate_q, gate_scales, up_q, up_scales, down_q, down_scales,
                       group_size, *, num_experts=None):
        return self._fixed("q8_group128", hidden, indices, weights, gate_q, gate_scales, up_q, up_scales, down_q,
                           down_scales, group_size, num_experts)

    def status(self) -> None:
        """Raises if a fused launch on any workspace this extension holds hit
        its wait budget (synchronises each workspace's stream)."""
        with self._ws_lock:
            spaces = list(self._ws_cache.values())
        for ws in spaces:
            self.workspace_status(ws)


def load_native_extension(*, build_directory: str | Path | None = None, verbose: bool = False) -> tuple[str, HipExtension]:
    """Load the prebuilt library for the current device; returns (platform, extension).

    Unlike the reference (JIT build through torch.utils.cpp_extension), the
    library is built ahead of time in-tree; ``build_directory`` is accepted for
    signature compatibility and ignored.
    """
    import torch

    platform = observed_native_platform(torch)
    with _BUILD_LOCK:
        cached = _EXTENSIONS.get(platform)
        if cached is None:
            cached = HipExtension()
            buf = ctypes.create_string_buffer(64)
            _native.check(cached.lib.uqm_device_arch(torch.cuda.current_device(), buf, 64), "uqm_device_arch")
            if not buf.value.decode().startswith("gfx950"):
                raise ContractError(f"libuma_qmoe_hip sees {buf.value!r}, not gfx950")
            if verbose:
                print(f"loaded {_native.library_path()} for {platform}")
            _EXTENSIONS[platform] = cached
        return platform, cached


# --------------------------------------------------------------- staging --
_NP_DTYPE = {"q4_group128": "u1", "q8_group128": "i1", "bf16_le": "<u2"}


def _release(*views: Any) -> None:
    for v in views:
        release = getattr(v, "release", None)
        if callable(release):
            release()


def layer_expert_count(reader: Any, layer_index: int) -> int:
    """E of one layer: the fixed model's expert count when the pack names its
    model, else the experts 0..E-1 whose gate projection the pack holds."""
    header = getattr(reader, "header", None)
    model = header.get("model", {}) if isinstance(header, dict) else {}
    if "num_experts" in model:
        return int(model["num_experts"])
    names = getattr(reader, "names", None)
    if callable(names):
        prefix = f"model.layers.{layer_index}.mlp.experts."
        ids = {int(n[len(prefix):].split(".", 1)[0]) for n in names()
               if n.startswith(prefix) and n.endswith(".gate_proj.weight")}
        if ids and ids == set(range(len(ids))):
            return len(ids)
        if ids:
            raise RuntimeError(f"layer {layer_index} experts are not numbered 0..E-1")
    raise RuntimeError(f"pack has no experts for layer {layer_index}")


def _layer_encoding(reader: Any, layer_index: int) -> str:
    getter = getattr(reader, "layer_encoding", None)
    return getter(layer_index) if callable(getter) else "q4_group128"


class PinnedStaging:
    """A grow-only pinned host buffer: expert tensors are gathered into it
    from the pack's (memory-mapped) views and reach the device in one DMA per
    projection."""

    def __init__(self) -> None:
        self._buf = None
        self.lock = threading.Lock()

    def take(self, nbytes: int, pinned: bool = True):
        import torch

        if not pinned:  # staging for a host-memory destination
            return torch.empty(nbytes, dtype=torch.uint8)
        if self._buf is None or self._buf.numel() < nbytes:
            self._buf = torch.empty(max(nbytes, 1 << 20), dtype=torch.uint8, pin_memory=True)
        return self._buf[:nbytes]


_STAGING = PinnedStaging()


def stage_experts(reader: Any, layer_index: int, device: Any, num_experts: int | None = None,
                  staging: PinnedStaging | None = None) -> DeviceExperts:
    """Copy one layer's compressed experts to the device, expert-major.

    The staged layout is the reference's (_host_projection / _device_layer,
    src/uma_qmoe/native_backend.py:374-455, 769-842): projection by
    projection, experts 0..E-1 concatenated, every expert of one shape,
    nothing expanded. A pack file opened by the library's reader is staged by
    the library itself (``uqm_pack_stage_projection``: straight from the
    mapping through pinned buffers to the device); other readers' views are
    gathered here into one pinned buffer and copied once per tensor kind.
    """
    import numpy as np
    import torch

    encoding = _layer_encoding(reader, layer_index)
    if encoding not in ENCODINGS:
        raise RuntimeError(f"layer {layer_index} has unsupported encoding {encoding!r}")
    E = layer_expert_count(reader, layer_index) if num_experts is None else int(num_experts)
    stg = staging or _STAGING
    dev = torch.device(device)
    out: dict[str, tuple[Any, Any]] = {}
    shapes: dict[str, tuple[int, int]] = {}
    # an ExpertPack names its group size in the header, a TargetPack per tensor
    header = getattr(reader, "header", None)
    quant = header.get("quantization") if isinstance(header, dict) else None
    group = int(quant.get("group_size", 128)) if isinstance(quant, dict) else 128
    native = dev.type == "cuda" and callable(getattr(reader, "stage_projection", None))
    with stg.lock:
        for proj in PROJECTIONS:
            if native:
                name = EXPERT_NAME.format(layer=layer_index, expert=0, proj=proj)
                data, scales, meta = reader.tensor_views(name)
                db, sb = len(data), len(scales)
                _release(data, scales)
                if meta.get("encoding", encoding) != encoding:
                    raise RuntimeError(f"tensor {name!r} is {meta.get('encoding')}, layer {layer_index} is {encoding}")
                shape = tuple(int(v) for v in meta["shape"])
                if len(shape) != 2:
                    raise RuntimeError(f"expert tensor {name!r} is not a matrix")
                shapes[proj] = shape
                if meta.get("group_size"):
                    group = int(meta["group_size"])
                s0 = -(-E * db // 256) * 256  # scales start 256-byte aligned
                staged = torch.empty(s0 + E * sb, dtype=torch.uint8, device=dev)
                reader.stage_projection(layer_index, proj, E, staged.data_ptr(),
                                        staged.data_ptr() + s0 if sb else 0,
                                        torch.cuda.current_stream(dev).cuda_stream)
                rows, cols = shape
                data = staged[:E * db].view({"u1": torch.uint8, "i1": torch.int8,
                                             "<u2": torch.bfloat16}[_NP_DTYPE[encoding]]).view(E, rows, -1)
                out[proj] = (data, staged[s0:].view(torch.float32).view(E, -1) if sb else None)
                continue
            views = []
            try:
                for e in range(E):
                    name = EXPERT_NAME.format(layer=layer_index, expert=e, proj=proj)
                    data, scales, meta = reader.tensor_views(name)
                    views.append((data, scales))
                    if meta.get("encoding", encoding) != encoding:
                        raise RuntimeError(f"tensor {name!r} is {meta.get('encoding')}, layer {layer_index} is {encoding}")
                    shape = tuple(int(v) for v in meta["shape"])
                    if len(shape) != 2:
                        raise RuntimeError(f"expert tensor {name!r} is not a matrix")
                    if shapes.setdefault(proj, shape) != shape:
                        raise RuntimeError(f"expert tensor {name!r} has unexpected shape {shape!r}")
                    if meta.get("group_size"):
                        group = int(meta["group_size"])
                db, sb = len(views[0][0]), len(views[0][1])
                if any(len(d) != db or len(sc) != sb for d, sc in views):
                    raise RuntimeError(f"layer {layer_index} {proj} tensors differ in size")
                s0 = -(-E * db // 256) * 256  # scales start 256-byte aligned
                host = stg.take(s0 + E * sb, pinned=dev.type == "cuda")
                flat = host.numpy()
                for e, (d, sc) in enumerate(views):
                    flat[e * db:(e + 1) * db] = np.frombuffer(d, dtype=np.uint8)
                    if sb:
                        flat[s0 + e * sb:s0 + (e + 1) * sb] = np.frombuffer(sc, dtype=np.uint8)
                if dev.type == "cuda":
                    staged = torch.empty(s0 + E * sb, dtype=torch.uint8, device=dev)
                    staged.copy_(host, non_blocking=True)
                    torch.cuda.current_stream(dev).synchronize()  # the buffer is reused for the next projection
                else:
                    staged = host
            finally:
                for d, sc in views:
                    _release(d, sc)
            rows, cols = shapes[proj]
            data = staged[:E * db].view({"u1": torch.uint8, "i1": torch.int8, "<u2": torch.bfloat16}[_NP_DTYPE[encoding]])
            data = data.view(E, rows, -1)
            sc_t = staged[s0:].view(torch.float32).view(E, -1) if sb else None
            out[proj] = (data, sc_t)
    inter, hidden = shapes["gate_proj"]
    if shapes["up_proj"] != (inter, hidden) or shapes["down_proj"] != (hidden, inter):
        raise RuntimeError(f"layer {layer_index} projection shapes are inconsistent: {shapes}")
    return DeviceExperts(encoding, group, E, hidden, inter, out["gate_proj"][0], out["gate_proj"][1], out["up_proj"][0],
                         out["up_proj"][1], out["down_proj"][0], out["down_proj"][1])


class CorrectnessPath:
    """``performance_mode=False`` on HIP tensors: the reference's correctness
    path (custom_op.py:172-340 and :343-506: every expert of the layer
    dequantised transiently to BF16, then BF16 expert GEMMs with FP32
    accumulation) in this library's kernels. Each call stages the layer's
    compressed experts from the leased reader, dequantises them with
    ``uqm_dequantize`` and runs the BF16 expert kernels on them; nothing is
    cached between calls. The routes are checked on the host first (one
    synchronisation), as the reference does, so an id outside [0, E) is an
    error here rather than a route that contributes nothing.

    It shares no state with the performance backends and needs none of them
    installed; it is not a fallback: a performance-mode call never reaches it.
    """

    @staticmethod
    def extension() -> HipExtension:
        return load_native_extension()[1]

    @classmethod
    def _experts(cls, reader: Any, layer_index: int, hidden_states: Any) -> DeviceExperts:
        import torch

        if hidden_states.dtype != torch.bfloat16:
            raise RuntimeError("uma_qmoe correctness mode requires BF16 hidden states")
        layer = stage_experts(reader, layer_index, hidden_states.device)
        if hidden_states.shape[-1] != layer.hidden_size:
            raise RuntimeError(f"hidden size {hidden_states.shape[-1]} does not match the layer's {layer.hidden_size}")
        return cls.extension().bf16_experts(layer)

    @classmethod
    def routed(cls, hidden_states, expert_indices, routing_weights, layer_index, reader):
        """moe_forward / qwen_moe_forward: out [*, H]."""
        import torch

        if expert_indices.dtype not in (torch.int32, torch.int64):
            raise RuntimeError("expert_indices must use int32 or int64")
        if tuple(expert_indices.shape) != tuple(routing_weights.shape):
            raise RuntimeError("expert_indices and routing_weights shapes must match")
        layer = cls._experts(reader, layer_index, hidden_states)
        flat = hidden_states.reshape(-1, layer.hidden_size)
        if expert_indices.ndim != 2 or expert_indices.shape[0] != flat.shape[0]:
            raise RuntimeError("expert_indices must have shape [tokens, top_k]")
        if expert_indices.numel() and bool(((expert_indices < 0) | (expert_indices >= layer.num_experts)).any()):
            raise RuntimeError("expert_indices contains an invalid expert")
        out = cls.extension().moe_forward(layer, flat, expert_indices, routing_weights)
        return out.reshape(hidden_states.shape)

    @classmethod
    def block(cls, hidden_states, router_weight, shared_gate_proj, shared_up_proj, shared_down_proj,
              shared_expert_gate, top_k, norm_topk_prob, layer_index, reader):
        """moe_block: (out, router logits, routing weights, expert indices)."""
        import torch

        layer = cls._experts(reader, layer_index, hidden_states)
        shared = (shared_gate_proj, shared_up_proj, shared_down_proj, shared_expert_gate)
        if any(t is None for t in shared) and not all(t is None for t in shared):
            raise RuntimeError("shared expert tensors must be given together")
        dense = DenseBlock(router_weight.to(torch.bfloat16).contiguous(),
                           *(None if t is None else t.to(torch.bfloat16).contiguous() for t in shared))
        if tuple(dense.router.shape) != (layer.num_experts, layer.hidden_size):
            raise RuntimeError(f"router weight must be [{layer.num_experts}, {layer.hidden_size}]")
        return cls.extension().moe_layer(layer, dense, hidden_states, int(top_k), bool(norm_topk_prob))


def correctness_forward(kind: str, hidden_states: Any, args: tuple, reader: Any) -> Any:
    """Runs op ``kind`` ("olmoe", "qwen" or "block") in correctness mode on HIP tensors."""
    if kind == "block":
        return CorrectnessPath.block(hidden_states, *args, reader)
    return CorrectnessPath.routed(hidden_states, *args, reader)


class _NativeMoEBackend:
    """Shared machinery: per-(pack, layer, device) compressed caches."""

    REQUIRED: tuple[str, ...] = ()
    ENCODINGS: frozenset[str] = frozenset()

    def __init__(self, platform: str, extension: Any) -> None:
        if platform != PLATFORM:
            raise ContractError(f"unsupported packed MoE platform {platform!r}")
        missing = [name for name in self.REQUIRED if not hasattr(extension, name)]
        if missing:
            raise ContractError(f"native extension does not expose {', '.join(missing)}")
        self.platform = platform
        self.extension = extension
        self._cache: dict[tuple[int, str, str], Any] = {}
        self._layer_cache: dict[tuple[int, int, str], DeviceExperts] = {}
        self._lock = threading.Lock()
        # Raise after every call whose fused launch hit its wait budget (one
        # host synchronisation per call; off by default: such a launch writes
        # NaN outputs, and status() checks on demand).
        self.check_each_call = False

    @classmethod
    def build_and_register(cls, *, build_directory: str | Path | None = None, verbose: bool = False):
        platform, extension = load_native_extension(build_directory=build_directory, verbose=verbose)
        backend = cls(platform, extension)
        register_performance_backend(platform, backend)
        return backend

    # staging ---------------------------------------------------------------
    def _device_layer(self, pack_handle: int, layer_index: int, device: Any, reader: Any) -> DeviceExperts:
        key = (pack_handle, layer_index, str(device))
        with self._lock:
            cached = self._layer_cache.get(key)
        if cached is not None:
            return cached
        encoding = _layer_encoding(reader, layer_index)
        if encoding not in self.ENCODINGS:
            raise RuntimeError(
                f"{type(self).__name__} cannot execute layer {layer_index} encoded as {encoding}; "
                "install the mixed backend"
            )
        value = stage_experts(reader, layer_index, device)
        with self._lock:
            return self._layer_cache.setdefault(key, value)

    def _device_tensor(self, pack_handle: int, name: str, device: Any, reader: Any):
        import numpy as np
        import torch

        key = (pack_handle, name, str(device))
        with self._lock:
            cached = self._cache.get(key)
        if cached is not None:
            return cached
        data_view, scale_view, meta = reader.tensor_views(name)
        try:
            encoding = meta.get("encoding", "q4_group128")
            shape = tuple(int(v) for v in meta["shape"])
            data = torch.from_numpy(np.frombuffer(data_view, dtype=_NP_DTYPE[encoding]).copy())
            if encoding == "bf16_le":
                data = data.view(torch.bfloat16)
            scales = (torch.from_numpy(np.frombuffer(scale_view, dtype="<f4").copy()).to(device)
                      if ENCODINGS[encoding].grouped else None)
        finally:
            _release(data_view, scale_view)
        if len(shape) != 2:
            raise RuntimeError(f"tensor {name!r} is not a matrix")
        value = (encoding, data.to(device), scales, shape, int(meta.get("group_size") or 128))
        with self._lock:
            return self._cache.setdefault(key, value)

    def _linear(self, input_tensor: Any, pack_handle: int, name: str, expected: str):
        import torch

        with acquire_expert_pack(pack_handle) as reader:
            encoding, data, scales, shape, group = self._device_tensor(pack_handle, name, input_tensor.device, reader)
        if encoding != expected:
            raise RuntimeError(f"tensor {name!r} is {encoding}, not {expected}")
        stream = torch.cuda.current_stream(input_tensor.device)
        for t in (data, scales):
            if t is not None:
                t.record_stream(stream)
        if encoding == "q4_group128":
            return self.extension.q4_linear(input_tensor, data, scales, shape[0], shape[1], group)
        if encoding == "q8_group128":
            return self.extension.q8_linear(input_tensor, data, scales, shape[0], shape[1], group)
        return self.extension.bf16_linear(input_tensor, data.reshape(shape))

    def q4_linear(self, input_tensor: Any, pack_handle: int, name: str):
        return self._linear(input_tensor, pack_handle, name, "q4_group128")

    # execution -------------------------------------------------------------
    def _layer_for_call(self, hidden_states, layer_index, pack_handle):
        import torch

        if hidden_states.dtype != torch.bfloat16:
            raise RuntimeError("packed MoE performance backend requires BF16 hidden states")
        with acquire_expert_pack(pack_handle) as reader:
            layer = self._device_layer(pack_handle, layer_index, hidden_states.device, reader)
        if hidden_states.shape[-1] != layer.hidden_size:
            raise RuntimeError(f"hidden size {hidden_states.shape[-1]} does not match the layer's {layer.hidden_size}")
        stream = torch.cuda.current_stream(hidden_states.device)
        for t in layer.tensors:
            t.record_stream(stream)
        return layer

    def _routed(self, hidden_states, expert_indices, routing_weights, layer_index, pack_handle):
        import torch

        if expert_indices.dtype not in (torch.int32, torch.int64):
            raise RuntimeError("expert_indices must use int32 or int64")
        layer = self._layer_for_call(hidden_states, layer_index, pack_handle)
        flat = hidden_states.reshape(-1, layer.hidden_size)
        if expert_indices.ndim != 2 or expert_indices.shape[0] != flat.shape[0]:
            raise RuntimeError("expert_indices must have shape [tokens, top_k]")
        out = self.extension.moe_forward(layer, flat, expert_indices, routing_weights)
        return out.reshape(hidden_states.shape)

    def __call__(self, hidden_states, expert_indices, routing_weights, layer_index, pack_handle):
        return self._routed(hidden_states, expert_indices, routing_weights, layer_index, pack_handle)

    def qwen_forward(self, hidden_states, expert_indices, routing_weights, layer_index, pack_handle):
        return self._routed(hidden_states, expert_indices, routing_weights, layer_index, pack_handle)

    def moe_block(self, hidden_states, router_weight, shared_gate_proj, shared_up_proj, shared_down_proj,
                  shared_expert_gate, top_k, norm_topk_prob, layer_index, pack_handle):
        """Router + routed experts (+ gated shared expert) of one block;
        returns (out, router logits, routing weights, expert indices)."""
        import torch

        layer = self._layer_for_call(hidden_states, layer_index, pack_handle)
        shared = (shared_gate_proj, shared_up_proj, shared_down_proj, shared_expert_gate)
        if any(t is None for t in shared) and not all(t is None for t in shared):
            raise RuntimeError("shared expert tensors must be given together")
        dense = DenseBlock(
            router_weight.to(torch.bfloat16).contiguous(),
            *(None if t is None else t.to(torch.bfloat16).contiguous() for t in shared),
        )
        if tuple(dense.router.shape) != (layer.num_experts, layer.hidden_size):
            raise RuntimeError(f"router weight must be [{layer.num_experts}, {layer.hidden_size}]")
        result = self.extension.moe_layer(layer, dense, hidden_states, int(top_k), bool(norm_topk_prob))
        if self.check_each_call:
            self.extension.status()
        return result

    # bookkeeping -----------------------------------------------------------
    def status(self) -> None:
        """Raises if any fused launch since the last check hit its wait
        budget (its outputs are NaN); synchronises the workspaces' streams."""
        self.extension.status()

    def cache_summary(self) -> dict[str, int]:
        with self._lock:
            tensors = list(self._cache.values())
            layers = list(self._layer_cache.values())
        tensor_bytes = sum(sum(t.numel() * t.element_size() for t in v[1:3] if t is not None) for v in tensors)
        return {
            "tensor_count": len(tensors) + sum(3 * layer.num_experts for layer in layers),
            "device_storage_bytes": tensor_bytes + sum(layer.device_storage_bytes for layer in layers),
            "dequantized_weight_bytes": 0,
        }

    def release_pack(self, pack_handle: int) -> None:
        """Drop every compressed device tensor owned by a closed pack handle."""
        with self._lock:
            for cache in (self._cache, self._layer_cache):
                for key in [k for k in cache if k[0] == pack_handle]:
                    del cache[key]


class PackedQ4NativeBackend(_NativeMoEBackend):
    """All-Q4 backend (ExpertPack or all-Q4 TargetPack layers)."""

    REQUIRED = ("q4_linear", "q4_moe_forward")
    ENCODINGS = frozenset({"q4_group128"})


class MixedTargetNativeBackend(_NativeMoEBackend):
    """Mixed Q4 / Q8 / BF16 TargetPack backend; every encoding runs from its
    stored bytes through the same HIP pipeline (no BF16/F32 expansion)."""

    REQUIRED = ("q4_linear", "q4_moe_forward", "q8_linear", "q8_moe_forward", "bf16_linear")
    ENCODINGS = frozenset({"q4_group128", "q8_group128", "bf16_le"})

    def q8_linear(self, input_tensor: Any, pack_handle: int, name: str):
        return self._linear(input_tensor, pack_handle, name, "q8_group128")

    def bf16_linear(self, input_tensor: Any, pack_handle: int, name: str):
        return self._linear(input_tensor, pack_handle, name, "bf16_le")


def install_packed_q4_backend(*, build_directory: str | Path | None = None, verbose: bool = False) -> PackedQ4NativeBackend:
    return PackedQ4NativeBackend.build_and_register(build_directory=build_directory, verbose=verbose)


def install_mixed_target_backend(*, build_directory: str | Path | None = None, verbose: bool = False) -> MixedTargetNativeBackend:
    return MixedTargetNativeBackend.build_and_register(build_directory=build_directory, verbose=verbose)


__all__ = [
    "DenseBlock",
    "DeviceExperts",
    "HipExtension",
    "MixedTargetNativeBackend",
    "PackedQ4NativeBackend",
    "PinnedStaging",
    "install_mixed_target_backend",
    "install_packed_q4_backend",
    "layer_expert_count",
    "load_native_extension",
    "native_kernel_source_sha256",
    "observed_native_platform",
    "stage_experts",
]
