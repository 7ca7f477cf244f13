"""Agreement metrics and the kernel evidence record (CPU).

The metric functions are pinned by closed forms (nearest-rank percentiles of
1..n, cosine of scaled / negated / zero tensors, relative error of a scaled
tensor), by a plain-Python loop over a small case, and by the tolerance
envelope of the reference's Q4 single-layer policy; the evidence record by
the schema's structural rules (required fields, constants, gates)."""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

from uma_qmoe_amd.evidence import (
    Q4_LAYER_POLICY,
    check_policy,
    kernel_evidence,
    numeric_agreement,
    percentile,
    route_agreement,
    timing,
    validate_kernel_evidence,
)
from uma_qmoe_amd.formats import ContractError


def test_nearest_rank_percentiles_closed_form():
    v = np.arange(1, 101, dtype=np.float64)[::-1]
    assert (percentile(v, 0.5), percentile(v, 0.95), percentile(v, 0.99), percentile(v, 1.0)) == (50, 95, 99, 100)
    assert percentile([3.0, 1.0, 2.0], 0.5) == 2.0 and percentile([3.0, 1.0, 2.0], 0.95) == 3.0
    assert percentile([7.0], 0.01) == 7.0


def test_cosine_and_relative_error_closed_forms():
    g = torch.Generator().manual_seed(0)
    ref = torch.randn(64, generator=g)
    same = numeric_agreement(ref, ref)
    assert same["cosine_similarity"] == pytest.approx(1.0) and same["absolute_error"]["max"] == 0.0
    double = numeric_agreement(ref, 2 * ref)
    assert double["cosine_similarity"] == pytest.approx(1.0)
    assert double["relative_error"]["p50"] == pytest.approx(1.0) and double["relative_error"]["max"] == pytest.approx(1.0)
    assert numeric_agreement(ref, -ref)["cosine_similarity"] == pytest.approx(-1.0)
    zero = torch.zeros(8)
    assert numeric_agreement(zero, zero)["cosine_similarity"] == 1.0
    assert numeric_agreement(zero, torch.ones(8))["cosine_similarity"] == 0.0
    with pytest.raises(ContractError, match="finite"):
        numeric_agreement(ref, ref * float("nan"))


def test_metrics_match_a_plain_python_loop():
    g = torch.Generator().manual_seed(1)
    ref = torch.randn(37, generator=g).double()
    cand = ref + 0.01 * torch.randn(37, generator=g).double()
    eps = 1e-4
    absolute, relative = [], []
    dot = nr = nc = 0.0
    for a, b in zip(ref.tolist(), cand.tolist()):
        absolute.append(abs(a - b))
        relative.append(abs(a - b) / max(abs(a), eps))
        dot += a * b
        nr += a * a
        nc += b * b
    got = numeric_agreement(ref, cand, epsilon=eps)
    assert got["absolute_error"]["mean"] == pytest.approx(math.fsum(absolute) / 37, rel=1e-15)
    assert got["absolute_error"]["p99"] == sorted(absolute)[math.ceil(0.99 * 37) - 1]
    assert got["relative_error"]["p95"] == sorted(relative)[math.ceil(0.95 * 37) - 1]
    assert got["relative_error"]["max"] == max(relative)
    assert got["cosine_similarity"] == pytest.approx(dot / math.sqrt(nr * nc), rel=1e-14)


def test_route_set_agreement():
    ref = torch.tensor([[0, 1, 2, 3], [4, 5, 6, 7], [1, 2, 3, 4]])
    cand = torch.tensor([[3, 2, 1, 0], [4, 5, 6, 9], [8, 9, 10, 11]])
    r = route_agreement(ref, cand)
    assert r["decision_count"] == 3 and r["exact_set_match_count"] == 1
    assert r["top_k_set_agreement"] == pytest.approx(1 / 3)
    assert r["mean_set_overlap"] == pytest.approx((1 + 0.75 + 0) / 3)
    with pytest.raises(ContractError, match="duplicate"):
        route_agreement(torch.tensor([[0, 0]]), torch.tensor([[0, 1]]))


def test_policy_envelope():
    g = torch.Generator().manual_seed(2)
    ref = torch.randn(1000, generator=g)
    near = numeric_agreement(ref, ref + 0.01, epsilon=1e-4)
    assert check_policy(near, {"top_k_set_agreement": 1.0}, Q4_LAYER_POLICY) == []
    far = numeric_agreement(ref, ref + 0.5, epsilon=1e-4)
    failed = check_policy(far, {"top_k_set_agreement": 0.5}, Q4_LAYER_POLICY)
    assert "max_p99_absolute_error" in failed and "min_router_top_k_set_agreement" in failed


def _doc(**over):
    res = {"finite": True, "max_absolute_error": 0.01, "cosine_similarity": 0.9999}
    kw = dict(target_id="mi355x", platform="hip_gfx950", device_name="AMD Instinct MI355X", source_sha256="a" * 64,
              abi="q4-group128-packed-u8-fp32-scale-bf16-in-bf16-out-v1", execution_strategy="fused-persistent",
              model={"model_id": "allenai/OLMoE-1B-7B-0125", "model_revision": "b" * 40,
                     "expert_pack_sha256": "c" * 64},
              workload={"layer_index": 0, "tokens": 1, "prefill_tokens": 32, "top_k": 8, "unique_experts": 8,
                        "warmup_iterations": 3, "measured_iterations": 10},
              projection_results=[{**res, "name": n, "shape": [1024, 2048]} for n in ("gate_proj", "up_proj",
                                                                                      "down_proj")],
              moe_forward={**res, "output_sha256": "d" * 64}, acceptance={"max_absolute_error": 1.0,
                                                                         "minimum_cosine_similarity": 0.99},
              samples_ms=[0.02 + 0.001 * i for i in range(10)],
              cache={"tensor_count": 192, "device_storage_bytes": 64 * 3_342_336, "dequantized_weight_bytes": 0},
              prefill_moe_forward={**res, "output_sha256": "e" * 64}, prefill_samples_ms=[0.05] * 10)
    kw.update(over)
    return kernel_evidence(**kw)


def test_kernel_evidence_document_and_its_rules():
    doc = _doc()
    validate_kernel_evidence(doc)
    assert doc["status"] == "passed" and doc["gates"]["overall_passed"]
    assert doc["performance"]["median_milliseconds"] == pytest.approx(0.0245)
    assert doc["performance"]["p95_milliseconds"] == pytest.approx(0.029)
    bad = _doc(moe_forward={"finite": True, "max_absolute_error": 3.0, "cosine_similarity": 0.5,
                            "output_sha256": "d" * 64})
    validate_kernel_evidence(bad)
    assert bad["status"] == "failed" and not bad["gates"]["moe_correctness"]
    for mutate, message in ((lambda d: d["performance"].__setitem__("dequantized_weight_cache_bytes", 4),
                             "dequantized"),
                            (lambda d: d["performance"].pop("p95_milliseconds"), "lacks"),
                            (lambda d: d["gates"].__setitem__("overall_passed", False), "overall"),
                            (lambda d: d.__setitem__("extra", 1), "unknown"),
                            (lambda d: d["correctness"]["projection_results"].pop(), "three")):
        tampered = copy.deepcopy(doc)
        mutate(tampered)
        with pytest.raises(ContractError, match=message):
            validate_kernel_evidence(tampered)


def test_timing_summary():
    t = timing([1.0, 2.0, 3.0, 4.0])
    assert t["median_milliseconds"] == 2.5 and t["p95_milliseconds"] == 4.0
    assert t["cv"] == pytest.approx(np.std([1, 2, 3, 4], ddof=1) / 2.5)
    with pytest.raises(ContractError, match="three"):
        timing([1.0, 2.0])
