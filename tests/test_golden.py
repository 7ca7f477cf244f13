"""The golden fixtures (tests/golden/*.npz) against the CPU oracle.

The fixtures are regression anchors written by the oracle (make_golden.py);
the oracle itself is pinned in test_oracle_moe.py / test_oracle_codec.py.
Here: the seeds still regenerate the same weight bytes (SHA-256), the stored
input is the one the seeds give, the routes follow the explicit top-k rule on
the stored logits, and re-running the oracle reproduces the stored output.
"""

from __future__ import annotations

import pytest
import torch

from golden.make_golden import CASES, oracle_case, weights_digest
from golden_cases import load, names, regenerate
from oracle import moe as om


def test_every_case_has_a_fixture():
    assert sorted(CASES) == names()


@pytest.mark.parametrize("name", sorted(CASES))
def test_fixture_reproduces_from_seeds(name):
    fx = load(name)
    shape, layer, dense, x, layer_index, bias = regenerate(name)
    assert weights_digest(layer, dense) == fx["meta"]["weights_sha256"], "synthetic generator drifted"
    assert torch.equal(x.view(torch.int16), fx["x"].view(torch.int16))
    # selection is the explicit rule applied to the stored logits
    assert torch.equal(fx["indices"], om.topk_ordered(fx["logits"], shape.top_k))
    out, logits, weights, indices = oracle_case(shape, layer, dense, x, layer_index, bias)
    assert torch.equal(indices, fx["indices"])
    # same arithmetic on the same CPU library: at most one bf16 ulp apart
    for got, ref in ((logits, fx["logits"]), (weights, fx["weights"]), (out, fx["out"])):
        err = (got.float() - ref.float()).abs()
        assert bool((err <= ref.float().abs() * 2.0 ** -7 + 1e-6).all())
