"""TEST INFRASTRUCTURE ONLY: torch-CPU restatement of the MoE operator path.

Reference files restated (zihaomu/UMA-QMoE; ``tf:`` = Transformers source,
models/qwen2_moe/modeling_qwen2_moe.py):

  streaming_reference   src/uma_qmoe/custom_op.py:465-506 (Qwen CPU branch) and
                        :301-340 (OLMoE CPU branch): ascending expert id, FP32
                        dequantized [gate; up] fused linear, chunk(2),
                        silu(gate)*up, FP32 down, times the route weight, cast
                        to BF16, index_add_ into a BF16 accumulator.
  router                tf:330-336 (F.linear in BF16, softmax in FP32, top-k,
                        optional renormalisation, cast to BF16). Top-k order
                        is made explicit: larger logit first, then lower id.
  shared_expert         tf:130-142 (Qwen2MoeMLP, BF16) and
                        src/uma_qmoe/qwen_compressed_loader.py:72,82-85
                        (sigmoid(shared_expert_gate(x)) * shared_expert(x)).
  qwen_block            src/uma_qmoe/qwen_compressed_loader.py:67-86.
  olmoe_block           src/uma_qmoe/compressed_loader.py:58-67.
  rmsnorm               tf:56-70 (Qwen2MoeRMSNorm, weight ones).
  route_permutation     src/uma_qmoe/native_backend.py:530-543 (stable argsort,
                        bincount, cumsum -> route_order, expert_offsets[E+1]);
                        ids outside [0, E) are dropped instead of raising.

The product never imports this module.
"""

from __future__ import annotations

from typing import Any

import numpy as np
import torch
import torch.nn.functional as F

from . import codec

EXPERT_NAME = "model.layers.{layer}.mlp.experts.{expert}.{proj}.weight"


def expert_name(layer: int, expert: int, proj: str) -> str:
    return EXPERT_NAME.format(layer=layer, expert=expert, proj=proj)


def read_tensor(reader: Any, name: str) -> np.ndarray:
    """Decode one tensor through the reference reader interface.

    ``reader.tensor_views(name) -> (data_view, scale_view, metadata)`` is the
    interface of src/uma_qmoe/target_pack.py:695-740 / expert_pack.py:515-540.
    """
    data, scales, metadata = reader.tensor_views(name)
    try:
        return codec.decode_tensor(bytes(data), bytes(scales), metadata)
    finally:
        for view in (data, scales):
            release = getattr(view, "release", None)
            if callable(release):
                release()


def _fused_gate_up(selected: torch.Tensor, gate_up: torch.Tensor) -> torch.Tensor:
    # src/uma_qmoe/custom_op.py:44-48
    gate, up = F.linear(selected, gate_up).chunk(2, dim=-1)
    intermediate = F.silu(gate)
    intermediate.mul_(up)
    return intermediate


def decoded_expert(reader: Any, layer_index: int, e: int) -> tuple[torch.Tensor, torch.Tensor]:
    """FP32 ([gate; up], down) of one expert, dequantized from the reader
    (src/uma_qmoe/custom_op.py:475-490, _combine_gate_up_arrays :35-40)."""
    gate = read_tensor(reader, expert_name(layer_index, e, "gate_proj"))
    up = read_tensor(reader, expert_name(layer_index, e, "up_proj"))
    down = read_tensor(reader, expert_name(layer_index, e, "down_proj"))
    if gate.shape != up.shape:
        raise RuntimeError("Gate and Up projection shapes must match")
    return torch.from_numpy(np.concatenate((gate, up), axis=0)), torch.from_numpy(np.ascontiguousarray(down))


def predequantized(reader: Any, layer_index: int, num_experts: int):
    """All experts of a layer dequantized once; a ``weights_of`` for
    streaming_reference that then does only the FP32 arithmetic (the
    compute-only CPU bound: the reference dequantizes on every call)."""
    table = {e: decoded_expert(reader, layer_index, e) for e in range(num_experts)}
    return table.__getitem__


def streaming_reference(
    hidden_states: torch.Tensor,
    expert_indices: torch.Tensor,
    routing_weights: torch.Tensor,
    layer_index: int,
    reader: Any,
    *,
    num_experts: int,
    weights_of=None,
) -> torch.Tensor:
    """CPU correctness branch of the operator, generic in E and k.

    src/uma_qmoe/custom_op.py:465-506 (Qwen) / :307-340 (OLMoE). Experts are
    dequantized per call from ``reader`` unless ``weights_of(e)`` supplies
    them.
    """
    if weights_of is None:
        weights_of = lambda e: decoded_expert(reader, layer_index, e)  # noqa: E731
    flattened = hidden_states.reshape(-1, hidden_states.shape[-1])
    final = torch.zeros_like(flattened)
    if flattened.shape[0] == 0:
        return final.reshape(hidden_states.shape)
    with torch.no_grad():
        mask = F.one_hot(expert_indices.long(), num_classes=num_experts).permute(2, 1, 0)
        hit = torch.greater(mask.sum(dim=(-1, -2)), 0).nonzero()
    for entry in hit:
        e = int(entry[0].item())
        slots, rows = torch.where(mask[e])
        gate_up, down_t = weights_of(e)
        selected = flattened.index_select(0, rows).to(torch.float32)
        intermediate = _fused_gate_up(selected, gate_up)
        expert_output = F.linear(intermediate, down_t)
        weights = routing_weights[rows, slots].to(torch.float32).unsqueeze(-1)
        expert_output = expert_output * weights
        final.index_add_(0, rows, expert_output.to(final.dtype))
    return final.reshape(hidden_states.shape)


def qwen_streaming_reference(hidden_states, expert_indices, routing_weights, layer_index, reader):
    """Validation of src/uma_qmoe/custom_op.py:355-367, then the CPU branch."""
    if not 0 <= layer_index < 24:
        raise RuntimeError("Qwen layer_index must be in [0, 23]")
    if hidden_states.shape[-1] != 2048:
        raise RuntimeError("Qwen hidden size must be 2048")
    flattened = hidden_states.reshape(-1, hidden_states.shape[-1])
    if expert_indices.shape != routing_weights.shape:
        raise RuntimeError("expert_indices and routing_weights shapes must match")
    if expert_indices.ndim != 2 or tuple(expert_indices.shape) != (flattened.shape[0], 4):
        raise RuntimeError("Qwen routes must have shape [tokens, 4]")
    if expert_indices.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("expert_indices must use int32 or int64")
    if bool(torch.any(expert_indices < 0)) or bool(torch.any(expert_indices >= 60)):
        raise RuntimeError("expert_indices contains an invalid Qwen expert")
    return streaming_reference(
        hidden_states, expert_indices, routing_weights, layer_index, reader, num_experts=60
    )


def olmoe_streaming_reference(hidden_states, expert_indices, routing_weights, layer_index, reader):
    """Validation of src/uma_qmoe/custom_op.py:188-200, then the CPU branch."""
    if not 0 <= layer_index < 16:
        raise RuntimeError("OLMoE layer_index must be in [0, 15]")
    if hidden_states.shape[-1] != 2048:
        raise RuntimeError("OLMoE hidden size must be 2048")
    flattened = hidden_states.reshape(-1, hidden_states.shape[-1])
    if expert_indices.shape != routing_weights.shape:
        raise RuntimeError("expert_indices and routing_weights shapes must match")
    if expert_indices.ndim != 2 or tuple(expert_indices.shape) != (flattened.shape[0], 8):
        raise RuntimeError("OLMoE routes must have shape [tokens, 8]")
    if expert_indices.dtype not in (torch.int32, torch.int64):
        raise RuntimeError("expert_indices must use int32 or int64")
    if bool(torch.any(expert_indices < 0)) or bool(torch.any(expert_indices >= 64)):
        raise RuntimeError("expert_indices contains an invalid expert")
    out = streaming_reference(
        hidden_states, expert_indices, routing_weights, layer_index, reader, num_experts=64
    )
    return out.to(hidden_states.dtype)


def route_permutation(expert_indices, num_experts: int) -> tuple[list[int], list[int]]:
    """Stable grouping of the routes t*k+slot by expert id, as a counting sort
    written out in plain Python (src/uma_qmoe/native_backend.py:530-543 does
    the same with torch.argsort(stable=True), bincount and cumsum). Routes whose
    id is outside [0, num_experts) are left out. Returns (route_order,
    expert_offsets) with len(expert_offsets) == num_experts + 1.
    """
    flat = [int(v) for v in torch.as_tensor(expert_indices).reshape(-1).tolist()]
    buckets: list[list[int]] = [[] for _ in range(num_experts)]
    for route, e in enumerate(flat):
        if 0 <= e < num_experts:
            buckets[e].append(route)
    order: list[int] = []
    offsets = [0]
    for b in buckets:
        order.extend(b)
        offsets.append(len(order))
    return order, offsets


def topk_ordered(logits: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest logits per row; equal logits go to the lower id.

    A stable descending sort keeps equal keys in ascending index order.
    """
    return torch.sort(logits.float(), dim=-1, descending=True, stable=True).indices[..., :k]


def router(hidden: torch.Tensor, weight: torch.Tensor, top_k: int, norm_topk_prob: bool = False):
    """Qwen2MoeTopKRouter.forward (tf:330-336) with the explicit tie rule.

    Returns (logits bf16 [T,E], weights bf16 [T,k], indices int64 [T,k]).
    """
    x = hidden.reshape(-1, weight.shape[1])
    logits = F.linear(x, weight)
    probs = F.softmax(logits, dim=-1, dtype=torch.float32)
    indices = topk_ordered(logits, top_k)
    top = probs.gather(-1, indices)
    if norm_topk_prob:
        top = top / top.sum(dim=-1, keepdim=True)
    return logits, top.to(logits.dtype), indices


def shared_expert(hidden, gate_w, up_w, down_w, shared_gate_w):
    """sigmoid(x . w_g) * down(silu(gate x) * up x), all BF16 (tf:130-142;
    src/uma_qmoe/qwen_compressed_loader.py:72,82-84)."""
    y = F.linear(F.silu(F.linear(hidden, gate_w)) * F.linear(hidden, up_w), down_w)
    return torch.sigmoid(F.linear(hidden, shared_gate_w)) * y


def qwen_block(hidden, layer, reader, layer_index: int, *, routes=None, weights_of=None):
    """QuantizedQwenMoEBlock.forward, src/uma_qmoe/qwen_compressed_loader.py:67-86.

    ``layer`` holds the dense BF16 tensors: router [E,H], shared_gate/up [Is,H],
    shared_down [H,Is], shared_expert_gate [1,H]; and ``num_experts``/``top_k``.
    ``routes`` optionally forces (weights, indices) instead of the router's.
    Returns (output bf16, logits, weights, indices).
    """
    flat = hidden.reshape(-1, hidden.shape[-1])
    logits, weights, indices = router(flat, layer["router"], layer["top_k"], layer.get("norm_topk_prob", False))
    if routes is not None:
        weights, indices = routes
    out = streaming_reference(flat, indices, weights, layer_index, reader, num_experts=layer["num_experts"],
                              weights_of=weights_of)
    if layer.get("shared_gate") is not None:
        sh = shared_expert(flat, layer["shared_gate"], layer["shared_up"], layer["shared_down"], layer["shared_expert_gate"])
        out = out.add_(sh)
    return out.reshape(hidden.shape), logits, weights, indices


def olmoe_block(hidden, layer, reader, layer_index: int, *, routes=None):
    """QuantizedMoEBlock.forward, src/uma_qmoe/compressed_loader.py:58-67."""
    flat = hidden.reshape(-1, hidden.shape[-1])
    logits, weights, indices = router(flat, layer["router"], layer["top_k"], layer.get("norm_topk_prob", False))
    if routes is not None:
        weights, indices = routes
    out = streaming_reference(flat, indices, weights, layer_index, reader, num_experts=layer["num_experts"])
    return out.to(hidden.dtype).reshape(hidden.shape), logits, weights, indices


def rmsnorm(hidden: torch.Tensor, eps: float = 1e-6, weight: torch.Tensor | None = None) -> torch.Tensor:
    """Qwen2MoeRMSNorm.forward, tf:65-70."""
    dtype = hidden.dtype
    h = hidden.to(torch.float32)
    variance = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(variance + eps)
    w = torch.ones(hidden.shape[-1], dtype=dtype) if weight is None else weight
    return w * h.to(dtype)


def rel_l2(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.double()
    b = b.double()
    return float(torch.linalg.vector_norm(a - b) / torch.linalg.vector_norm(b).clamp_min(1e-30))


def max_abs(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.double() - b.double()).abs().max()) if a.numel() else 0.0
