"""RouteTrace documents: validation and replay of measured routing.

A RouteTrace (the format of src/uma_qmoe/route_trace.py) records the router
decisions of one greedy generation run of a fixed model: one prefill event of
batch x prompt tokens followed by single-token decode events, and for every
(layer, event) the top-k expert ids and routing weights of each token,
token-major. The document also carries derived fields that a reader must be
able to recompute:

  per layer    tokens per expert, the k hottest experts (most tokens, then
               lower id), the k coldest non-empty ones, the empty ones, min /
               max / mean and the nearest-rank p95 of the counts;
  summary      event and layer counts, tokens per layer, routed decisions
               (x layers), expert assignments (x k), the two batch shapes;
  payload      SHA-256 over "UMA-QMoE.RouteTrace.v<schema>" NUL, then per
               layer its index (u16), per event its index and token count
               (u32, u32), its expert ids (u8 each) and weights (f64 each),
               all little endian.

The two fixed models (src/uma_qmoe/fixed_models.py:34-55): OLMoE-1B-7B-0125
(16 layers, 64 experts, top-8, trace schema 1) and Qwen1.5-MoE-A2.7B (24, 60,
top-4, schema 2).

``trace_arrays`` turns a validated document into dense arrays (expert ids
[layers, tokens, k], weights, per-event token counts), which is all a replay
needs; ``replay`` walks them event-major, layer-major as the reference's
iter_replay_events does (route_trace.py:382-405), and ``payload_sha256``
recomputes the document's route hash from the arrays alone, so a stored copy
of the arrays is checked against the document it came from.
"""

from __future__ import annotations

from dataclasses import dataclass
import hashlib
import json
import math
from pathlib import Path
import struct
from typing import Any, Iterator, Mapping

import numpy as np

from .formats import ContractError


@dataclass(frozen=True)
class TraceModel:
    model_id: str
    model_revision: str
    num_layers: int
    num_experts: int
    top_k: int
    schema_version: int


MODELS = {
    "allenai/OLMoE-1B-7B-0125": TraceModel("allenai/OLMoE-1B-7B-0125", "9b0c1aa87e34a20052389dce1f0cf01da783f654",
                                           16, 64, 8, 1),
    "Qwen/Qwen1.5-MoE-A2.7B": TraceModel("Qwen/Qwen1.5-MoE-A2.7B", "1a758c50ecb6350748b9ce0a99d2352fd9fc11c9",
                                         24, 60, 4, 2),
}


def trace_model(model: Mapping[str, Any]) -> TraceModel:
    spec = MODELS.get(model.get("model_id"))
    if spec is None or model.get("model_revision") != spec.model_revision:
        raise ContractError(f"unsupported fixed model identity: {model.get('model_id')!r} at revision "
                            f"{model.get('model_revision')!r}")
    return spec


def load_route_trace(path: str | Path) -> dict[str, Any]:
    try:
        doc = json.loads(Path(path).read_text(encoding="utf-8"))
    except (OSError, json.JSONDecodeError) as exc:
        raise ContractError(f"cannot read RouteTrace {path}: {exc}") from exc
    if not isinstance(doc, dict):
        raise ContractError("RouteTrace root must be an object")
    return doc


def _uint(v: Any, what: str, least: int = 0) -> int:
    if isinstance(v, bool) or not isinstance(v, int) or v < least:
        raise ContractError(f"{what} must be an integer of at least {least}")
    return v


def _events(raw: Any) -> list[dict[str, Any]]:
    """Event records, checked: prefill first, then contiguous decode steps."""
    if not isinstance(raw, list) or len(raw) < 2:
        raise ContractError("RouteTrace requires prefill and decode events")
    out = []
    for i, e in enumerate(raw):
        if not isinstance(e, dict) or _uint(e.get("event_index"), "event_index") != i:
            raise ContractError("RouteTrace event indices must be contiguous from zero")
        phase, step = e.get("phase"), e.get("decode_step")
        if (i == 0) != (phase == "prefill") or phase not in {"prefill", "decode"}:
            raise ContractError("RouteTrace must contain one prefill followed by decode events")
        if (phase == "prefill" and step is not None) or (phase == "decode" and _uint(step, "decode_step") != i - 1):
            raise ContractError("decode steps must be contiguous after prefill")
        b = _uint(e.get("batch_size"), "batch_size", 1)
        s = _uint(e.get("tokens_per_sequence"), "tokens_per_sequence", 1)
        out.append({"event_index": i, "phase": phase, "decode_step": step, "batch_size": b,
                    "tokens_per_sequence": s, "token_count": b * s})
    return out


def expert_statistics(counts: np.ndarray, top_k: int) -> dict[str, Any]:
    """The per-layer statistics of route_trace.py:100-116 from token counts per expert."""
    c = [int(v) for v in counts]
    ids = range(len(c))
    hot = sorted(ids, key=lambda e: (-c[e], e))[:top_k]
    tail = sorted((e for e in ids if c[e] > 0), key=lambda e: (c[e], e))[:top_k]
    ordered = sorted(c)
    return {"tokens_per_expert": c, "hot_experts": hot, "long_tail_experts": tail,
            "empty_experts": [e for e in ids if c[e] == 0], "minimum_tokens": min(c), "maximum_tokens": max(c),
            "mean_tokens": sum(c) / len(c), "p95_tokens": ordered[max(0, math.ceil(0.95 * len(c)) - 1)]}


def payload_sha256(indices: np.ndarray, weights: np.ndarray, token_counts: np.ndarray, schema_version: int) -> str:
    """SHA-256 of the binary route payload from dense arrays: indices and
    weights [layers, tokens, k] (events concatenated in order), token_counts
    [events]."""
    h = hashlib.sha256(f"UMA-QMoE.RouteTrace.v{schema_version}\0".encode())
    bounds = np.concatenate(([0], np.cumsum(token_counts)))
    for layer in range(indices.shape[0]):
        h.update(struct.pack("<H", layer))
        for ev, t in enumerate(token_counts):
            lo, hi = int(bounds[ev]), int(bounds[ev + 1])
            h.update(struct.pack("<II", ev, int(t)))
            h.update(np.ascontiguousarray(indices[layer, lo:hi], dtype=np.uint8).tobytes())
            h.update(np.ascontiguousarray(weights[layer, lo:hi], dtype="<f8").tobytes())
    return h.hexdigest()


def trace_arrays(document: Mapping[str, Any]) -> dict[str, Any]:
    """Validates a RouteTrace document completely (every derived field and the
    payload hash are recomputed) and returns its routes as dense arrays."""
    spec = trace_model(document.get("model", {}))
    if document.get("schema_version") != spec.schema_version:
        raise ContractError("RouteTrace schema version does not match fixed model")
    if document.get("model") != {"model_id": spec.model_id, "model_revision": spec.model_revision,
                                 "num_layers": spec.num_layers, "num_experts": spec.num_experts, "top_k": spec.top_k}:
        raise ContractError("RouteTrace model architecture is inconsistent")
    events = _events(document.get("events"))
    if events != document["events"]:
        raise ContractError("RouteTrace event records are inconsistent")
    layers = document.get("layers")
    if not isinstance(layers, list) or len(layers) != spec.num_layers:
        raise ContractError(f"RouteTrace must contain exactly {spec.num_layers} layers")
    counts = np.array([e["token_count"] for e in events], dtype=np.int64)
    total, k = int(counts.sum()), spec.top_k
    indices = np.zeros((spec.num_layers, total, k), dtype=np.int64)
    weights = np.zeros((spec.num_layers, total, k), dtype=np.float64)
    for li, layer in enumerate(layers):
        if not isinstance(layer, dict) or layer.get("layer_index") != li:
            raise ContractError("RouteTrace layers must be ordered contiguously")
        evs = layer.get("events")
        if not isinstance(evs, list) or len(evs) != len(events):
            raise ContractError("each RouteTrace layer must cover every event")
        row = 0
        for e, le in zip(events, evs):
            if not isinstance(le, dict) or le.get("event_index") != e["event_index"] \
                    or le.get("token_count") != e["token_count"]:
                raise ContractError("RouteTrace layer event index mismatch")
            ids, ws = le.get("expert_indices"), le.get("routing_weights")
            n = e["token_count"] * k
            if not isinstance(ids, list) or not isinstance(ws, list) or len(ids) != n or len(ws) != n:
                raise ContractError("RouteTrace route arrays do not match token_count × Top-K")
            if any(isinstance(v, bool) or not isinstance(v, int) for v in ids):
                raise ContractError("expert index must be an integer of at least 0")
            if any(isinstance(v, bool) or not isinstance(v, (int, float)) for v in ws):
                raise ContractError("routing weight must be finite and in [0, 1]")
            a = np.asarray(ids, dtype=np.int64).reshape(-1, k)
            w = np.asarray(ws, dtype=np.float64).reshape(-1, k)
            if (a < 0).any() or (a >= spec.num_experts).any():
                raise ContractError("RouteTrace expert index exceeds model expert count")
            if not (np.isfinite(w).all() and (w >= 0).all() and (w <= 1).all()):
                raise ContractError("routing weight must be finite and in [0, 1]")
            srt = np.sort(a, axis=1)
            if (srt[:, 1:] == srt[:, :-1]).any():
                raise ContractError("RouteTrace Top-K row contains duplicate experts")
            indices[li, row:row + a.shape[0]] = a
            weights[li, row:row + a.shape[0]] = w
            row += a.shape[0]
        per_expert = np.bincount(indices[li].reshape(-1), minlength=spec.num_experts)
        if layer.get("top_k") != k or layer.get("token_count") != total \
                or layer.get("expert_statistics") != expert_statistics(per_expert, k):
            raise ContractError(f"RouteTrace layer {li} derived fields are inconsistent")
    if document.get("route_payload_sha256") != payload_sha256(indices, weights, counts, spec.schema_version):
        raise ContractError("RouteTrace route payload SHA-256 is inconsistent")
    summary = {"event_count": len(events), "layer_count": spec.num_layers, "tokens_per_layer": total,
               "routed_token_decisions": total * spec.num_layers,
               "expert_assignments": total * spec.num_layers * k,
               "batch_shapes": [{"phase": "prefill", "batch_size": events[0]["batch_size"],
                                 "tokens_per_sequence": events[0]["tokens_per_sequence"], "occurrences": 1},
                                {"phase": "decode", "batch_size": events[1]["batch_size"],
                                 "tokens_per_sequence": events[1]["tokens_per_sequence"],
                                 "occurrences": len(events) - 1}]}
    if document.get("summary") != summary:
        raise ContractError("RouteTrace summary is inconsistent")
    return {"model_id": spec.model_id, "schema_version": spec.schema_version, "num_experts": spec.num_experts,
            "top_k": k, "token_counts": counts, "expert_indices": indices, "routing_weights": weights,
            "route_payload_sha256": document["route_payload_sha256"],
            "phases": [e["phase"] for e in events]}


@dataclass(frozen=True)
class ReplayEvent:
    event_index: int
    phase: str
    layer_index: int
    token_count: int
    expert_indices: np.ndarray   # int64 [tokens, k]
    routing_weights: np.ndarray  # float64 [tokens, k]


def replay(arrays: Mapping[str, Any]) -> Iterator[ReplayEvent]:
    """(event, layer) route tensors in replay order: event-major, then layer."""
    counts = np.asarray(arrays["token_counts"])
    bounds = np.concatenate(([0], np.cumsum(counts)))
    idx, w = arrays["expert_indices"], arrays["routing_weights"]
    phases = list(arrays["phases"])
    for ev in range(len(counts)):
        lo, hi = int(bounds[ev]), int(bounds[ev + 1])
        for layer in range(idx.shape[0]):
            yield ReplayEvent(ev, str(phases[ev]), layer, hi - lo, idx[layer, lo:hi], w[layer, lo:hi])


def load_arrays(path: str | Path) -> dict[str, Any]:
    """Dense routes stored by ``save_arrays`` (numpy, no pickled objects)."""
    with np.load(path, allow_pickle=False) as z:
        meta = json.loads(str(z["meta"]))
        return {**meta, "expert_indices": z["expert_indices"].astype(np.int64),
                "routing_weights": z["routing_weights"].astype(np.float64),
                "token_counts": z["token_counts"].astype(np.int64), "phases": str(z["phases"]).split(","),
                "num_experts": MODELS[meta["model_id"]].num_experts, "top_k": MODELS[meta["model_id"]].top_k}


def distinct_experts(arrays: Mapping[str, Any]) -> np.ndarray:
    """Distinct experts hit per (event, layer): [events, layers]."""
    counts = np.asarray(arrays["token_counts"])
    bounds = np.concatenate(([0], np.cumsum(counts)))
    idx = arrays["expert_indices"]
    out = np.zeros((len(counts), idx.shape[0]), dtype=np.int64)
    for ev in range(len(counts)):
        for layer in range(idx.shape[0]):
            out[ev, layer] = np.unique(idx[layer, bounds[ev]:bounds[ev + 1]]).size
    return out


__all__ = [
    "MODELS",
    "ReplayEvent",
    "distinct_experts",
    "expert_statistics",
    "load_arrays",
    "load_route_trace",
    "payload_sha256",
    "replay",
    "trace_arrays",
    "trace_model",
]
