"""Agreement metrics and evidence records in the reference's reporting formats.

Metrics (src/uma_qmoe/reference_oracle.py:398-560), over float64 copies of
two tensors of one shape:

  absolute error  |ref - cand| per element;
  relative error  |ref - cand| / max(|ref|, epsilon);
  distributions   mean (exactly rounded sum), p50, p95, p99 and max, the
                  percentiles by nearest rank: sorted[max(0, ceil(q n) - 1)];
  cosine          dot / sqrt(|ref|^2 |cand|^2), 1 when both are zero, 0 when
                  one is, clipped to [-1, 1];
  route sets      per token, whether the k selected experts agree as a set,
                  and the mean overlap |A & B| / k.

Non-finite values are an error, not a metric. A quality policy (the fields
of benchmarks/policies/*_single_moe_layer_v1.yaml) is checked against these
metrics by ``check_policy``.

``kernel_evidence`` assembles the ``packed_q4_kernel_evidence`` document of
src/uma_qmoe/schemas/packed_q4_kernel_evidence.schema.json (producer:
benchmarks/runners/validate_packed_q4_kernel.py:201-221): the single-layer
timing samples with their median and nearest-rank p95, the compressed cache
of the backend (and a zero dequantized cache), the correctness results and
the gates. Two enumerations are widened for this target: ``target_id``
"mi355x" and platform "hip_gfx950"; everything else keeps the schema's
names, types and constants, which ``validate_kernel_evidence`` checks.
"""

from __future__ import annotations

from datetime import datetime, timezone
import hashlib
import math
import re
from typing import Any, Mapping, Sequence

import numpy as np

from .formats import ContractError

DEFAULT_EPSILON = 1e-12
# The north star's acceptance for a MoE layer output (bf16, fp32 accumulate).
NORTH_STAR = {"max_rel_l2": 1e-2, "max_absolute_error": 2e-2}
# benchmarks/policies/olmoe_q4_group128_halo3_single_moe_layer_v1.yaml:13-22
Q4_LAYER_POLICY = {"relative_error_epsilon": 1e-4, "max_absolute_error": 0.8, "max_relative_error": 200.0,
                   "max_p99_absolute_error": 0.075, "max_p99_relative_error": 8.0, "min_cosine_similarity": 0.999,
                   "min_router_top_k_set_agreement": 1.0}


def percentile(values: Any, q: float) -> float:
    """Nearest-rank percentile (reference_oracle.py:398-400)."""
    v = np.sort(np.asarray(values, dtype=np.float64).reshape(-1))
    if v.size == 0:
        raise ContractError("percentile of an empty sample")
    return float(v[max(0, math.ceil(q * v.size) - 1)])


def distribution(values: Any) -> dict[str, float]:
    v = np.asarray(values, dtype=np.float64).reshape(-1)
    return {"mean": math.fsum(v.tolist()) / v.size, "p50": percentile(v, 0.50), "p95": percentile(v, 0.95),
            "p99": percentile(v, 0.99), "max": float(v.max())}


def _as_f64(t: Any) -> np.ndarray:
    if hasattr(t, "detach"):
        import torch

        t = t.detach().cpu().to(torch.float64).numpy()
    return np.asarray(t, dtype=np.float64).reshape(-1)


def numeric_agreement(reference: Any, candidate: Any, *, epsilon: float = DEFAULT_EPSILON) -> dict[str, Any]:
    """Error distributions and cosine of one candidate tensor against its reference."""
    ref, cand = _as_f64(reference), _as_f64(candidate)
    if ref.shape != cand.shape:
        raise ContractError(f"tensor sizes differ: {ref.size} vs {cand.size}")
    if not (np.all(np.isfinite(ref)) and np.all(np.isfinite(cand))):
        raise ContractError("agreement metrics need finite values on both sides")
    if not (math.isfinite(epsilon) and epsilon > 0):
        raise ContractError("relative_error_epsilon must be finite and positive")
    absolute = np.abs(ref - cand)
    relative = absolute / np.maximum(np.abs(ref), epsilon)
    nr, nc = float(np.dot(ref, ref)), float(np.dot(cand, cand))
    if nr == 0.0 and nc == 0.0:
        cosine = 1.0
    elif nr == 0.0 or nc == 0.0:
        cosine = 0.0
    else:
        cosine = min(1.0, max(-1.0, float(np.dot(ref, cand)) / math.sqrt(nr * nc)))
    rel_l2 = math.sqrt(float(np.dot(ref - cand, ref - cand)) / max(nr, 1e-300))
    return {"element_count": int(ref.size), "finite": True, "absolute_error": distribution(absolute),
            "relative_error": distribution(relative), "cosine_similarity": cosine, "rel_l2": rel_l2}


def route_agreement(reference_indices: Any, candidate_indices: Any) -> dict[str, Any]:
    """Top-k set agreement of two [tokens, k] expert-index tensors."""
    ref = np.asarray(_as_f64(reference_indices), dtype=np.int64)
    cand = np.asarray(_as_f64(candidate_indices), dtype=np.int64)
    shape = tuple(reference_indices.shape)
    if len(shape) != 2 or tuple(candidate_indices.shape) != shape:
        raise ContractError("route tensors must both be [tokens, top_k]")
    k = shape[1]
    ref, cand = ref.reshape(shape), cand.reshape(shape)
    rs, cs = np.sort(ref, axis=1), np.sort(cand, axis=1)
    if np.any(rs[:, 1:] == rs[:, :-1]) or np.any(cs[:, 1:] == cs[:, :-1]):
        raise ContractError("route tensor contains duplicate expert ids in a top-k row")
    exact = np.all(rs == cs, axis=1)
    overlap = (ref[:, :, None] == cand[:, None, :]).any(axis=2).sum(axis=1) / k
    return {"decision_count": shape[0], "top_k": k, "exact_set_match_count": int(exact.sum()),
            "top_k_set_agreement": float(exact.mean()) if shape[0] else 1.0,
            "mean_set_overlap": float(overlap.mean()) if shape[0] else 1.0}


def check_policy(numeric: Mapping[str, Any], routes: Mapping[str, Any] | None, policy: Mapping[str, Any]) -> list[str]:
    """Names of the policy thresholds the metrics violate (empty: passed)."""
    failed = []
    limits = (("max_absolute_error", numeric["absolute_error"]["max"]),
              ("max_relative_error", numeric["relative_error"]["max"]),
              ("max_p99_absolute_error", numeric["absolute_error"]["p99"]),
              ("max_p99_relative_error", numeric["relative_error"]["p99"]))
    for name, value in limits:
        if policy.get(name) is not None and value > policy[name]:
            failed.append(name)
    if policy.get("min_cosine_similarity") is not None and numeric["cosine_similarity"] < policy["min_cosine_similarity"]:
        failed.append("min_cosine_similarity")
    want = policy.get("min_router_top_k_set_agreement")
    if want is not None and routes is not None and routes["top_k_set_agreement"] < want:
        failed.append("min_router_top_k_set_agreement")
    return failed


def timing(samples_ms: Sequence[float]) -> dict[str, Any]:
    """Median, nearest-rank p95/p99 and coefficient of variation of samples."""
    s = np.asarray(samples_ms, dtype=np.float64)
    if s.size < 3 or not np.all(s > 0):
        raise ContractError("timing needs at least three positive samples")
    mean = float(s.mean())
    return {"samples_milliseconds": [float(v) for v in s], "median_milliseconds": float(np.median(s)),
            "p95_milliseconds": percentile(s, 0.95), "p99_milliseconds": percentile(s, 0.99),
            "cv": float(s.std(ddof=1) / mean) if s.size > 1 else 0.0}


def tensor_sha256(t: Any) -> str:
    """SHA-256 of a tensor's float32 values (validate_packed_q4_kernel.py:57-59)."""
    return hashlib.sha256(np.ascontiguousarray(_as_f64(t).astype(np.float32)).tobytes()).hexdigest()


def kernel_evidence(*, target_id: str, platform: str, device_name: str, source_sha256: str, abi: str,
                    execution_strategy: str, model: Mapping[str, str], workload: Mapping[str, int],
                    projection_results: Sequence[Mapping[str, Any]], moe_forward: Mapping[str, Any],
                    acceptance: Mapping[str, float], samples_ms: Sequence[float], cache: Mapping[str, int],
                    prefill_moe_forward: Mapping[str, Any] | None = None,
                    prefill_samples_ms: Sequence[float] | None = None) -> dict[str, Any]:
    """The packed_q4_kernel_evidence document of one validation run."""
    def ok(r):
        return (r["finite"] and r["max_absolute_error"] <= acceptance["max_absolute_error"]
                and r["cosine_similarity"] >= acceptance["minimum_cosine_similarity"])

    t = timing(samples_ms)
    performance = {"scope": "single_moe_layer_microbenchmark", "samples_milliseconds": t["samples_milliseconds"],
                   "median_milliseconds": t["median_milliseconds"], "p95_milliseconds": t["p95_milliseconds"],
                   "compressed_cache_tensor_count": int(cache["tensor_count"]),
                   "compressed_cache_bytes": int(cache["device_storage_bytes"]),
                   "dequantized_weight_cache_bytes": int(cache["dequantized_weight_bytes"]),
                   "formal_tps_claim": False}
    gates = {"target_architecture": platform == "hip_gfx950", "target_compilation": True,
             "direct_packed_input": True, "no_dequantized_weight_cache": cache["dequantized_weight_bytes"] == 0,
             "projection_correctness": all(ok(r) for r in projection_results), "moe_correctness": ok(moe_forward),
             "performance_mode_executed": len(samples_ms) == workload["measured_iterations"]}
    correctness = {"projection_results": [dict(r) for r in projection_results], "moe_forward": dict(moe_forward),
                   "acceptance": dict(acceptance)}
    if prefill_moe_forward is not None:
        p = timing(prefill_samples_ms or [])
        performance.update({"prefill_samples_milliseconds": p["samples_milliseconds"],
                            "prefill_median_milliseconds": p["median_milliseconds"],
                            "prefill_p95_milliseconds": p["p95_milliseconds"]})
        correctness["prefill_moe_forward"] = dict(prefill_moe_forward)
        gates["prefill_moe_correctness"] = ok(prefill_moe_forward)
        gates["prefill_performance_mode_executed"] = len(prefill_samples_ms or []) == workload["measured_iterations"]
    gates["overall_passed"] = all(gates.values())
    return {
        "schema_version": 1,
        "kind": "packed_q4_kernel_evidence",
        "captured_at": datetime.now(timezone.utc).isoformat(timespec="seconds").replace("+00:00", "Z"),
        "target_id": target_id,
        "status": "passed" if gates["overall_passed"] else "failed",
        "model": dict(model),
        "kernel": {"platform": platform, "device_name": device_name, "source_sha256": source_sha256, "abi": abi,
                   "execution_strategy": execution_strategy, "compiled_for_target": True,
                   "reads_packed_weights_directly": True, "full_dequantized_weight_cache": False},
        "workload": dict(workload),
        "correctness": correctness,
        "performance": performance,
        "gates": gates,
    }


_HEX = {40: re.compile(r"^[0-9a-f]{40}$"), 64: re.compile(r"^[0-9a-f]{64}$")}


def _require(cond: bool, what: str) -> None:
    if not cond:
        raise ContractError(f"packed_q4_kernel_evidence: {what}")


def _only(obj: Any, required: set[str], optional: set[str], what: str) -> None:
    _require(isinstance(obj, dict), f"{what} must be an object")
    keys = set(obj)
    _require(required <= keys, f"{what} lacks {sorted(required - keys)}")
    _require(keys <= required | optional, f"{what} has unknown {sorted(keys - required - optional)}")


def _agreement_ok(r: Any, what: str, extra: set[str] = frozenset()) -> None:
    _only(r, {"finite", "max_absolute_error", "cosine_similarity"} | extra, set(), what)
    _require(isinstance(r["finite"], bool), f"{what}.finite")
    _require(r["max_absolute_error"] >= 0, f"{what}.max_absolute_error")
    _require(-1 <= r["cosine_similarity"] <= 1, f"{what}.cosine_similarity")


def validate_kernel_evidence(doc: Any) -> None:
    """The structural rules of packed_q4_kernel_evidence.schema.json (with the
    target enumerations widened as the module docstring says)."""
    _only(doc, {"schema_version", "kind", "captured_at", "target_id", "status", "model", "kernel", "workload",
                "correctness", "performance", "gates"}, set(), "document")
    _require(doc["schema_version"] == 1 and doc["kind"] == "packed_q4_kernel_evidence", "kind/version")
    datetime.fromisoformat(doc["captured_at"].replace("Z", "+00:00"))
    _require(doc["target_id"] in {"halo3", "local-halo", "spark1", "mi355x"}, "target_id")
    _require(doc["status"] in {"passed", "failed"}, "status")
    m = doc["model"]
    _only(m, {"model_id", "model_revision", "expert_pack_sha256"}, set(), "model")
    _require(bool(_HEX[40].match(m["model_revision"])) and bool(_HEX[64].match(m["expert_pack_sha256"])),
             "model hashes")
    k = doc["kernel"]
    _only(k, {"platform", "device_name", "source_sha256", "abi", "compiled_for_target",
              "reads_packed_weights_directly", "full_dequantized_weight_cache"}, {"execution_strategy"}, "kernel")
    _require(k["platform"] in {"hip_gfx1151", "cuda_sm121", "hip_gfx950"} and k["device_name"], "kernel platform")
    _require(bool(_HEX[64].match(k["source_sha256"])), "kernel source_sha256")
    w = doc["workload"]
    _only(w, {"layer_index", "tokens", "top_k", "unique_experts", "warmup_iterations", "measured_iterations"},
          {"prefill_tokens"}, "workload")
    _require(w["tokens"] >= 1 and w["warmup_iterations"] >= 1 and w["measured_iterations"] >= 3, "workload counts")
    c = doc["correctness"]
    _only(c, {"projection_results", "moe_forward", "acceptance"}, {"prefill_moe_forward"}, "correctness")
    _require(len(c["projection_results"]) == 3, "three projection results")
    for r in c["projection_results"]:
        _agreement_ok(r, "projection result", {"name", "shape"})
        _require(r["name"] in {"gate_proj", "up_proj", "down_proj"} and len(r["shape"]) == 2, "projection name/shape")
    for key in ("moe_forward", "prefill_moe_forward"):
        if key in c:
            _agreement_ok(c[key], key, {"output_sha256"})
            _require(bool(_HEX[64].match(c[key]["output_sha256"])), f"{key}.output_sha256")
    _only(c["acceptance"], {"max_absolute_error", "minimum_cosine_similarity"}, set(), "acceptance")
    p = doc["performance"]
    _only(p, {"scope", "samples_milliseconds", "median_milliseconds", "p95_milliseconds",
              "compressed_cache_tensor_count", "compressed_cache_bytes", "dequantized_weight_cache_bytes",
              "formal_tps_claim"}, {"prefill_samples_milliseconds", "prefill_median_milliseconds",
                                   "prefill_p95_milliseconds"}, "performance")
    _require(p["scope"] == "single_moe_layer_microbenchmark" and p["formal_tps_claim"] is False, "performance scope")
    _require(len(p["samples_milliseconds"]) >= 3 and all(v > 0 for v in p["samples_milliseconds"]), "samples")
    _require(p["compressed_cache_tensor_count"] >= 3 and p["compressed_cache_bytes"] >= 1, "compressed cache")
    _require(p["dequantized_weight_cache_bytes"] == 0, "dequantized weight cache must be 0")
    g = doc["gates"]
    _only(g, {"target_architecture", "target_compilation", "direct_packed_input", "no_dequantized_weight_cache",
              "projection_correctness", "moe_correctness", "performance_mode_executed", "overall_passed"},
          {"prefill_moe_correctness", "prefill_performance_mode_executed"}, "gates")
    _require(all(isinstance(v, bool) for v in g.values()), "gates are booleans")
    _require(g["overall_passed"] == all(v for n, v in g.items() if n != "overall_passed"), "overall gate")
    _require((doc["status"] == "passed") == g["overall_passed"], "status follows the gates")


__all__ = [
    "NORTH_STAR",
    "Q4_LAYER_POLICY",
    "check_policy",
    "distribution",
    "kernel_evidence",
    "numeric_agreement",
    "percentile",
    "route_agreement",
    "tensor_sha256",
    "timing",
    "validate_kernel_evidence",
]
