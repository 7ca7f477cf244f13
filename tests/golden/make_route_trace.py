"""Writes tests/golden/route_trace/<trace_id>.npz from a RouteTrace document.

The reference commits one measured trace, benchmarks/traces/
olmoe_1b_7b_0125_128x32_greedy_v1.json (OLMoE-1B-7B-0125, batch 1, 128 prompt
tokens, 32 greedy output tokens: one 128-token prefill and 31 single-token
decode events over 16 layers, top-8 of 64 experts). The document is validated
completely by uma_qmoe_amd.route_trace (every derived field and the route
payload SHA-256 recomputed) and its routes are stored as data, no pickled
objects:

  meta             JSON text: trace_id, model_id, schema_version,
                   route_payload_sha256 (the document's), source file SHA-256
  expert_indices   uint8 [layers, tokens, k], events concatenated in order
  routing_weights  float64 [layers, tokens, k] (the document's values exactly)
  token_counts     int64 [events]
  phases           the events' phases as one comma-separated string

Run from the repository root, with the reference checkout present:
  python tests/golden/make_route_trace.py /root/reference/benchmarks/traces/olmoe_1b_7b_0125_128x32_greedy_v1.json
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "uma-qmoe_amd"))

from uma_qmoe_amd.route_trace import load_route_trace, trace_arrays  # noqa: E402


def main(path: str) -> Path:
    src = Path(path)
    doc = load_route_trace(src)
    arrays = trace_arrays(doc)
    out = HERE / "route_trace" / f"{doc['trace_id']}.npz"
    out.parent.mkdir(parents=True, exist_ok=True)
    meta = {"trace_id": doc["trace_id"], "model_id": arrays["model_id"], "schema_version": arrays["schema_version"],
            "route_payload_sha256": arrays["route_payload_sha256"],
            "source_sha256": hashlib.sha256(src.read_bytes()).hexdigest()}
    np.savez_compressed(out, meta=np.array(json.dumps(meta, sort_keys=True)),
                        expert_indices=arrays["expert_indices"].astype(np.uint8),
                        routing_weights=arrays["routing_weights"], token_counts=arrays["token_counts"],
                        phases=np.array(",".join(arrays["phases"])))
    return out


if __name__ == "__main__":
    print(main(sys.argv[1]))
