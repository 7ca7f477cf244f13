"""Pins the oracle's MoE restatement (oracle/moe.py).

  * Transformers' own Qwen2MoeTopKRouter / Qwen2MoeExperts / Qwen2MoeMLP /
    Qwen2MoeRMSNorm (installed library, run on CPU) on the same weights;
  * the reference's stacked-expert fixture
    (tests/unit/test_fixed_model_runners.py:185-204) and fused gate/up order
    (tests/unit/test_custom_operator_lifecycle.py:70-112);
  * brute-force top-k on tiny inputs and forced ties (lower id wins);
  * invariants: k=1 with weight 1 is a single expert, zero weights give zero,
    slot order does not matter, a repeated expert adds its weights.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import codec as oc
from oracle import moe as om
from uma_qmoe_amd.formats import encode_target_tensor
from uma_qmoe_amd.packfile import memory_pack

H, I, IS, E, K = 128, 64, 96, 8, 2


def _pack(encoding: str, seed: int = 0, e: int = E, h: int = H, i: int = I, layer: int = 0):
    g = torch.Generator().manual_seed(seed)
    tensors, dense = {}, {}
    for ex in range(e):
        for proj, shape in (("gate_proj", (i, h)), ("up_proj", (i, h)), ("down_proj", (h, i))):
            w = torch.randn(shape, generator=g) * 0.05
            tensors[om.expert_name(layer, ex, proj)] = encode_target_tensor(w.numpy(), encoding)
    return memory_pack(tensors, {layer: encoding}, num_experts=e)


def _dense_experts(pack, layer: int, e: int):
    gate = torch.stack([torch.from_numpy(om.read_tensor(pack, om.expert_name(layer, x, "gate_proj"))) for x in range(e)])
    up = torch.stack([torch.from_numpy(om.read_tensor(pack, om.expert_name(layer, x, "up_proj"))) for x in range(e)])
    down = torch.stack([torch.from_numpy(om.read_tensor(pack, om.expert_name(layer, x, "down_proj"))) for x in range(e)])
    return gate, up, down


def _hf_config():
    from transformers.models.qwen2_moe.configuration_qwen2_moe import Qwen2MoeConfig

    return Qwen2MoeConfig(hidden_size=H, moe_intermediate_size=I, shared_expert_intermediate_size=IS, num_experts=E,
                          num_experts_per_tok=K, norm_topk_prob=False)


# ------------------------------------------------------------------ router --
def test_router_matches_brute_force_and_forced_ties():
    logits = torch.tensor([[0.5, 1.0, 1.0, -2.0, 1.0, 0.25], [3.0, 3.0, 3.0, 3.0, 3.0, 3.0]], dtype=torch.bfloat16)
    got = om.topk_ordered(logits, 3)
    for row, idx in zip(logits.float().tolist(), got.tolist()):
        brute = sorted(range(len(row)), key=lambda j: (-row[j], j))[:3]
        assert idx == brute
    assert got.tolist() == [[1, 2, 4], [0, 1, 2]]


def test_router_matches_transformers_on_tie_free_inputs():
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeTopKRouter

    cfg = _hf_config()
    router = Qwen2MoeTopKRouter(cfg)
    g = torch.Generator().manual_seed(11)
    with torch.no_grad():
        router.weight.copy_(torch.randn(E, H, generator=g) * 0.1)
    x = torch.randn(64, H, generator=g)
    with torch.no_grad():
        hf_logits, hf_w, hf_i = router(x)
    logits, w, idx = om.router(x, router.weight.detach(), K)
    assert torch.equal(logits, hf_logits)
    probs = F.softmax(hf_logits.float(), -1)
    for t in range(x.shape[0]):
        top = probs[t].sort(descending=True).values
        if top[K - 1] == top[K]:
            continue  # tie at the boundary: torch.topk order is implementation-defined
        assert set(idx[t].tolist()) == set(hf_i[t].tolist())
        np.testing.assert_allclose(w[t].float().sort().values.numpy(), hf_w[t].float().sort().values.numpy(), rtol=1e-6)


def test_router_weights_are_softmax_probabilities():
    g = torch.Generator().manual_seed(3)
    x = torch.randn(16, H, generator=g).to(torch.bfloat16)
    wr = (torch.randn(E, H, generator=g) * 0.1).to(torch.bfloat16)
    logits, w, idx = om.router(x, wr, K)
    l64 = logits.double()
    p = torch.exp(l64 - l64.max(-1, keepdim=True).values)
    p = p / p.sum(-1, keepdim=True)
    expect = p.gather(-1, idx)
    assert torch.allclose(w.double(), expect, rtol=1e-2, atol=0)
    _, wn, _ = om.router(x, wr, K, norm_topk_prob=True)
    assert torch.allclose(wn.double().sum(-1), torch.ones(16, dtype=torch.float64), atol=1e-2)


# ----------------------------------------------------------------- experts --
def test_stacked_expert_fixture_from_reference():
    # tests/unit/test_fixed_model_runners.py:185-204: one stacked expert
    gate_up = torch.arange(2 * 4 * 3, dtype=torch.float32).reshape(2, 4, 3)
    down = torch.arange(2 * 3 * 2, dtype=torch.float32).reshape(2, 3, 2)
    x = torch.arange(6, dtype=torch.float32).reshape(2, 3)
    gate, up = F.linear(x, gate_up[1]).chunk(2, dim=-1)
    expected = F.linear(F.silu(gate) * up, down[1])
    tensors = {}
    for e in range(2):
        tensors[om.expert_name(0, e, "gate_proj")] = encode_target_tensor(gate_up[e, :2].numpy(), "bf16_le")
        tensors[om.expert_name(0, e, "up_proj")] = encode_target_tensor(gate_up[e, 2:].numpy(), "bf16_le")
        tensors[om.expert_name(0, e, "down_proj")] = encode_target_tensor(down[e].numpy(), "bf16_le")
    pack = memory_pack(tensors, {0: "bf16_le"})
    out = om.streaming_reference(x, torch.ones(2, 1, dtype=torch.int64), torch.ones(2, 1), 0, pack, num_experts=2)
    assert torch.equal(out, expected)  # fp32 hidden: the accumulator is fp32 too


def test_fused_gate_up_puts_gate_rows_first():
    # tests/unit/test_custom_operator_lifecycle.py:70-112: one fused linear,
    # chunk(2) -> (gate, up), silu(gate) * up
    g = torch.full((2, 3), 1.0)
    u = torch.full((2, 3), 2.0)
    x = torch.ones(1, 3)
    out = om._fused_gate_up(x, torch.cat((g, u)))
    assert torch.allclose(out, F.silu(torch.full((1, 2), 3.0)) * 6.0)


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
@torch.no_grad()
def test_experts_match_transformers(encoding):
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeExperts

    pack = _pack(encoding, seed=7)
    gate, up, down = _dense_experts(pack, 0, E)
    experts = Qwen2MoeExperts(_hf_config())
    with torch.no_grad():
        experts.gate_up_proj.copy_(torch.cat((gate, up), dim=1))
        experts.down_proj.copy_(down)
    g = torch.Generator().manual_seed(1)
    x = torch.randn(24, H, generator=g).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(24)])
    w = torch.rand(24, K, generator=g).to(torch.bfloat16)
    ours = om.streaming_reference(x, idx, w, 0, pack, num_experts=E)
    hf = experts(x.float(), idx, w.float())
    assert ours.dtype == torch.bfloat16
    assert om.rel_l2(ours, hf) < 4e-3
    assert om.max_abs(ours, hf) < 2e-2


@torch.no_grad()
def test_block_matches_transformers_sparse_moe_block():
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeSparseMoeBlock

    pack = _pack("q4_group128", seed=9)
    gate, up, down = _dense_experts(pack, 0, E)
    blk = Qwen2MoeSparseMoeBlock(_hf_config())
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        blk.experts.gate_up_proj.copy_(torch.cat((gate, up), dim=1))
        blk.experts.down_proj.copy_(down)
        for p in (blk.gate.weight, blk.shared_expert.gate_proj.weight, blk.shared_expert.up_proj.weight,
                  blk.shared_expert.down_proj.weight, blk.shared_expert_gate.weight):
            p.copy_((torch.randn(p.shape, generator=g) * 0.1).to(torch.bfloat16).float())
    blk = blk.to(torch.bfloat16)
    x = torch.randn(1, 12, H, generator=g).to(torch.bfloat16)
    layer = {
        "router": blk.gate.weight.detach(),
        "top_k": K,
        "num_experts": E,
        "shared_gate": blk.shared_expert.gate_proj.weight.detach(),
        "shared_up": blk.shared_expert.up_proj.weight.detach(),
        "shared_down": blk.shared_expert.down_proj.weight.detach(),
        "shared_expert_gate": blk.shared_expert_gate.weight.detach(),
    }
    out, logits, w, idx = om.qwen_block(x, layer, pack, 0)
    # the Transformers block on the same routes (topk tie order is theirs)
    _, hf_w, hf_i = blk.gate(x.reshape(-1, H))
    assert torch.equal(logits, F.linear(x.reshape(-1, H), blk.gate.weight))
    routed = blk.experts(x.reshape(-1, H), idx, w)
    shared = torch.sigmoid(blk.shared_expert_gate(x.reshape(-1, H))) * blk.shared_expert(x.reshape(-1, H))
    hf = (routed + shared).reshape(x.shape)
    assert om.rel_l2(out, hf) < 1e-2
    assert om.max_abs(out, hf) < 2e-2


# -------------------------------------------------------------- invariants --
def test_invariants_single_zero_permutation_linearity():
    pack = _pack("q4_group128", seed=4)
    gate, up, down = _dense_experts(pack, 0, E)
    g = torch.Generator().manual_seed(8)
    x = torch.randn(6, H, generator=g).to(torch.bfloat16)
    # k=1, weight 1: a single expert's FFN
    idx1 = torch.full((6, 1), 3, dtype=torch.int64)
    out1 = om.streaming_reference(x, idx1, torch.ones(6, 1, dtype=torch.bfloat16), 0, pack, num_experts=E)
    xf = x.float()
    single = F.linear(F.silu(F.linear(xf, gate[3])) * F.linear(xf, up[3]), down[3])
    assert torch.equal(out1, single.to(torch.bfloat16))
    # zero weights
    idx = torch.tensor([[0, 5]] * 6)
    zero = om.streaming_reference(x, idx, torch.zeros(6, 2, dtype=torch.bfloat16), 0, pack, num_experts=E)
    assert torch.count_nonzero(zero) == 0
    # slot permutation
    w = torch.rand(6, 2, generator=g).to(torch.bfloat16)
    a = om.streaming_reference(x, idx, w, 0, pack, num_experts=E)
    b = om.streaming_reference(x, idx.flip(-1), w.flip(-1), 0, pack, num_experts=E)
    assert torch.equal(a, b)
    # a repeated expert contributes both weights
    rep = om.streaming_reference(x, torch.tensor([[2, 2]] * 6), w, 0, pack, num_experts=E)
    one = om.streaming_reference(x, torch.tensor([[2]] * 6), (w.float().sum(-1, keepdim=True)).to(torch.bfloat16), 0,
                                 pack, num_experts=E)
    assert om.rel_l2(rep, one) < 1e-2


def test_rmsnorm_matches_transformers():
    from transformers.models.qwen2_moe.modeling_qwen2_moe import Qwen2MoeRMSNorm

    x = (torch.randn(3, H) * 3).to(torch.bfloat16)
    norm = Qwen2MoeRMSNorm(H, eps=1e-6).to(torch.bfloat16)
    assert torch.equal(om.rmsnorm(x, 1e-6), norm(x))


def test_validation_messages_follow_reference():
    pack = _pack("q4_group128", seed=1, e=2)
    x = torch.zeros(1, 2048, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="Qwen routes must have shape"):
        om.qwen_streaming_reference(x, torch.zeros(1, 3, dtype=torch.int64), torch.zeros(1, 3), 0, pack)
    with pytest.raises(RuntimeError, match="invalid Qwen expert"):
        om.qwen_streaming_reference(x, torch.full((1, 4), 60), torch.zeros(1, 4), 0, pack)
    with pytest.raises(RuntimeError, match="layer_index"):
        om.olmoe_streaming_reference(x, torch.zeros(1, 8, dtype=torch.int64), torch.zeros(1, 8), 16, pack)


def test_route_permutation_matches_reference_torch_calls():
    """The counting sort equals the reference's stable argsort + bincount +
    cumsum (src/uma_qmoe/native_backend.py:530-543) on valid ids, and drops
    out-of-range ids while keeping the rest stable."""
    g = torch.Generator().manual_seed(7)
    for t, k, e in [(1, 4, 60), (5, 8, 64), (64, 4, 60), (33, 2, 256)]:
        idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
        order, offsets = om.route_permutation(idx, e)
        flat = idx.reshape(-1)
        assert order == torch.argsort(flat, stable=True).tolist()
        ref_offsets = torch.cat((torch.zeros(1, dtype=torch.int64), torch.bincount(flat, minlength=e).cumsum(0)))
        assert offsets == ref_offsets.tolist()
    # duplicates within a token and across tokens keep route order
    order, offsets = om.route_permutation(torch.tensor([[2, 2], [1, 2]]), 3)
    assert order == [2, 0, 1, 3] and offsets == [0, 0, 1, 4]
    # invalid ids vanish; E+1 offsets still cover [0, E]
    order, offsets = om.route_permutation(torch.tensor([[3, -1], [70, 3], [0, 5]]), 8)
    assert order == [4, 0, 3, 5] and offsets == [0, 1, 1, 1, 3, 3, 4, 4, 4]
