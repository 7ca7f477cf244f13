"""RouteTrace validation and replay (CPU).

The fixture tests/golden/route_trace/olmoe_1b_7b_0125_128x32_greedy_v1.npz
holds the routes of the reference's committed trace
(benchmarks/traces/olmoe_1b_7b_0125_128x32_greedy_v1.json). It is pinned by
the document's own route payload SHA-256, recomputed here from the arrays,
and by statistics the document records (layer 0). A document rebuilt from the
arrays validates, and tampered copies are rejected as the reference's
validator rejects them (route_trace.py:304-360)."""

from __future__ import annotations

import copy
import math
from pathlib import Path

import numpy as np
import pytest

from uma_qmoe_amd.formats import ContractError
from uma_qmoe_amd.route_trace import (
    MODELS,
    distinct_experts,
    expert_statistics,
    load_arrays,
    payload_sha256,
    replay,
    trace_arrays,
)

FIXTURE = Path(__file__).resolve().parent / "golden" / "route_trace" / "olmoe_1b_7b_0125_128x32_greedy_v1.npz"


@pytest.fixture(scope="module")
def arrays():
    return load_arrays(FIXTURE)


def test_fixture_reproduces_the_documents_payload_hash(arrays):
    assert arrays["route_payload_sha256"] == "9ab4045d91156a24f8b26d044ac09b6eeade355026b59fc1279cf4fa7ddae354"
    got = payload_sha256(arrays["expert_indices"], arrays["routing_weights"], arrays["token_counts"],
                         arrays["schema_version"])
    assert got == arrays["route_payload_sha256"]
    # one changed weight or id changes the hash
    w = arrays["routing_weights"].copy()
    w[3, 5, 1] = np.nextafter(w[3, 5, 1], 1.0)
    assert payload_sha256(arrays["expert_indices"], w, arrays["token_counts"], 1) != got


def test_fixture_shape_and_recorded_layer0_statistics(arrays):
    idx = arrays["expert_indices"]
    assert idx.shape == (16, 159, 8) and list(arrays["token_counts"]) == [128] + [1] * 31
    assert arrays["phases"] == ["prefill"] + ["decode"] * 31
    stats = expert_statistics(np.bincount(idx[0].reshape(-1), minlength=64), 8)
    # as recorded in the document's layers[0].expert_statistics
    assert stats["hot_experts"] == [5, 18, 19, 41, 51, 30, 55, 12]
    assert stats["long_tail_experts"] == [0, 52, 29, 10, 39, 16, 17, 37]
    assert (stats["maximum_tokens"], stats["p95_tokens"], stats["mean_tokens"]) == (65, 64, 19.875)
    assert len(stats["empty_experts"]) == 32


def test_replay_order_and_distinct_experts(arrays):
    events = list(replay(arrays))
    assert len(events) == 32 * 16
    assert [(e.event_index, e.layer_index) for e in events[:3]] == [(0, 0), (0, 1), (0, 2)]
    assert events[16].event_index == 1 and events[16].token_count == 1 and events[0].token_count == 128
    d = distinct_experts(arrays)
    assert d.shape == (32, 16) and (d[1:] == 8).all() and (d[0] <= 64).all()
    for e in events[:20]:
        srt = np.sort(e.expert_indices, axis=1)
        assert (srt[:, 1:] != srt[:, :-1]).all()


def _document(arrays):
    """A RouteTrace document rebuilt from the arrays (the fields the
    validator recomputes)."""
    spec = MODELS[arrays["model_id"]]
    counts = arrays["token_counts"]
    events = [{"event_index": i, "phase": p, "decode_step": None if i == 0 else i - 1, "batch_size": 1,
               "tokens_per_sequence": int(t), "token_count": int(t)} for i, (p, t) in
              enumerate(zip(arrays["phases"], counts))]
    bounds = np.concatenate(([0], np.cumsum(counts)))
    layers = []
    for li in range(spec.num_layers):
        evs = [{"event_index": i, "token_count": int(counts[i]),
                "expert_indices": [int(v) for v in arrays["expert_indices"][li, bounds[i]:bounds[i + 1]].reshape(-1)],
                "routing_weights": [float(v) for v in arrays["routing_weights"][li, bounds[i]:bounds[i + 1]].reshape(-1)]}
               for i in range(len(counts))]
        per = np.bincount(arrays["expert_indices"][li].reshape(-1), minlength=spec.num_experts)
        layers.append({"layer_index": li, "top_k": spec.top_k, "token_count": int(counts.sum()), "events": evs,
                       "expert_statistics": expert_statistics(per, spec.top_k)})
    total = int(counts.sum())
    return {"schema_version": 1, "model": {"model_id": spec.model_id, "model_revision": spec.model_revision,
                                           "num_layers": 16, "num_experts": 64, "top_k": 8},
            "events": events, "layers": layers, "route_payload_sha256": arrays["route_payload_sha256"],
            "summary": {"event_count": 32, "layer_count": 16, "tokens_per_layer": total,
                        "routed_token_decisions": total * 16, "expert_assignments": total * 16 * 8,
                        "batch_shapes": [{"phase": "prefill", "batch_size": 1, "tokens_per_sequence": 128,
                                          "occurrences": 1},
                                         {"phase": "decode", "batch_size": 1, "tokens_per_sequence": 1,
                                          "occurrences": 31}]}}


def test_rebuilt_document_validates_and_tampering_is_rejected(arrays):
    doc = _document(arrays)
    again = trace_arrays(doc)
    assert np.array_equal(again["expert_indices"], arrays["expert_indices"])
    assert np.array_equal(again["routing_weights"], arrays["routing_weights"])

    def dup(d):
        row = d["layers"][2]["events"][5]["expert_indices"]
        row[1] = row[0]

    def oob(d):
        d["layers"][0]["events"][1]["expert_indices"][0] = 64

    def weight(d):
        d["layers"][0]["events"][1]["routing_weights"][0] = math.nan

    def stats(d):
        d["layers"][4]["expert_statistics"]["p95_tokens"] += 1

    def payload(d):
        w = d["layers"][7]["events"][9]["routing_weights"]
        w[0] = w[0] / 2

    def order(d):
        d["events"][3]["decode_step"] = 5

    for mutate, message in ((dup, "duplicate"), (oob, "exceeds"), (weight, "finite"), (stats, "derived"),
                            (payload, "payload SHA-256"), (order, "contiguous")):
        bad = copy.deepcopy(doc)
        mutate(bad)
        with pytest.raises(ContractError, match=message):
            trace_arrays(bad)
