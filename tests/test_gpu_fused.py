"""The single-token fused MoE block kernel (one persistent launch per layer).

Checks, through the C ABI:
  * the fused and the multi-kernel paths both match the golden fixtures
    (selection bit-exact given logits);
  * repeated launches on one workspace are bit-identical and leave the sync
    words clean (the kernel's last wave resets them; the sticky error word
    stays zero);
  * the result does not depend on how the CUs are split between the routed and
    the shared experts: every row is computed by one wave with the same
    lane/column mapping, whatever the split;
  * renormalised top-k and top-k = 1 / 8 on a shape without shared expert.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from golden.make_golden import weights_digest
from golden_cases import load, regenerate
from oracle import moe as om
from test_gpu_kernels import DEV, assert_close, dense_to_cpu, dense_to_dev, note, to_dev
from uma_qmoe_amd import _native
from uma_qmoe_amd import synthetic as syn

pytestmark = pytest.mark.gpu


@pytest.fixture()
def fused_default(hip_ext):
    yield hip_ext
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, 1)


def _block(hip_ext, layer, dense, x, shape, ws=None):
    out, logits, weights, indices = hip_ext.moe_layer(layer, dense, x, shape.top_k, shape.norm_topk_prob, workspace=ws)
    torch.cuda.synchronize()
    return out.cpu(), logits.cpu(), weights.cpu(), indices.cpu()


@pytest.mark.parametrize("name", ["c1_t1", "c2_t1", "c3_l0_t1", "c3_l16_t1"])
@pytest.mark.parametrize("fused", [1, 0])
def test_both_paths_match_golden(fused_default, name, fused):
    hip_ext = fused_default
    note(f"fused={fused} {name}")
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, fused)
    fx = load(name)
    shape, layer, dense, x, layer_index, _ = regenerate(name)
    assert weights_digest(layer, dense) == fx["meta"]["weights_sha256"]
    out, logits, weights, indices = _block(hip_ext, to_dev(layer), dense_to_dev(dense), fx["x"].to(DEV), shape)
    assert torch.equal(indices, om.topk_ordered(logits, shape.top_k))
    ref_l = fx["logits"].float()
    assert bool(((logits.float() - ref_l).abs() <= ref_l.abs() * 2.0 ** -7 + 1e-30).all())
    if torch.equal(indices, fx["indices"]):
        assert_close(out, fx["out"], f"{name} fused={fused}")
    else:
        lay = {"router": dense.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
               "shared_gate": dense.shared_gate, "shared_up": dense.shared_up, "shared_down": dense.shared_down,
               "shared_expert_gate": dense.shared_expert_gate}
        ref, *_ = om.qwen_block(fx["x"], lay, syn.DeviceLayerReader({layer_index: layer}), layer_index,
                                routes=(weights, indices))
        assert_close(out, ref, f"{name} fused={fused} (gpu routes)")


def test_repeat_and_grid_size_are_bit_identical(fused_default):
    hip_ext = fused_default
    note("fused repeat / grid size c2")
    shape = syn.C2
    layer = syn.build_experts(shape, device=DEV, seed=11)
    dense = syn.build_dense(shape, device=DEV, seed=11)
    x = syn.hidden_states(shape, 1, device=DEV, seed=11)
    ws = hip_ext.new_workspace(DEV, 1, shape.hidden, shape.intermediate, shape.shared_intermediate,
                            shape.num_experts, shape.top_k)
    first = _block(hip_ext, layer, dense, x, shape, ws)
    for _ in range(4):
        again = _block(hip_ext, layer, dense, x, shape, ws)
        for a, b in zip(first, again):
            assert torch.equal(a.view(torch.uint8) if a.dtype == torch.bfloat16 else a,
                               b.view(torch.uint8) if b.dtype == torch.bfloat16 else b)
    hip_ext.workspace_status(ws)
    # one launch epoch per workgroup (one workgroup per CU), each advanced once per launch
    cus = torch.cuda.get_device_properties(DEV).multi_processor_count
    sync = ws[: 4 * (64 + cus)].view(torch.int32).cpu()
    assert int(sync[4]) == 0, "error word raised"
    assert int(sync[5]) == 0, "a launch was marked as expired"
    assert torch.equal(sync[64:64 + cus], torch.full((cus,), 5, dtype=torch.int32)), "epochs"
    assert not torch.isnan(first[0].float()).any(), "poisoned output without an expired wait"
    # the fused result is within tolerance of the multi-kernel path
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, 0)
    multi = _block(hip_ext, layer, dense, x, shape, ws)
    assert torch.equal(multi[3], first[3])
    assert_close(first[0], multi[0], "fused vs multi-kernel", rel=5e-3, mx=1e-2)


@pytest.mark.parametrize("k,norm,enc", [(1, False, "q4_group128"), (8, True, "q4_group128"),
                                        (2, False, "q8_group128"), (3, True, "bf16_le")])
def test_fused_topk_variants_match_oracle(fused_default, k, norm, enc):
    hip_ext = fused_default
    note(f"fused k={k} norm={norm} {enc}")
    shape = syn.MoEShape(f"fused_k{k}", 2048, 16, k, 256, encoding=enc, norm_topk_prob=norm)
    layer = syn.build_experts(shape, seed=k)
    dense = syn.build_dense(shape, seed=k)
    x = syn.hidden_states(shape, 1, seed=k)
    out, logits, weights, indices = _block(hip_ext, to_dev(layer), dense_to_dev(dense), x.to(DEV), shape)
    assert torch.equal(indices, om.topk_ordered(logits, k))
    probs = torch.softmax(logits.float(), -1).gather(-1, indices)
    if norm:
        probs = probs / probs.sum(-1, keepdim=True)
    assert (weights.float() - probs).abs().max() <= 2.0 ** -8 * probs.max() + 1e-6
    lay = {"router": dense.router, "top_k": k, "num_experts": shape.num_experts, "norm_topk_prob": norm}
    ref, *_ = om.olmoe_block(x, lay, syn.DeviceLayerReader({0: layer}), 0, routes=(weights, indices))
    assert_close(out, ref, f"fused k={k}")


def _norm_case(case):
    if case == "c1":
        return syn.C1, 0
    if case == "c2":
        return syn.C2, 0
    layer_index = int(case.split("_l")[1])
    return syn.c3_layer_shape(layer_index), layer_index


# (tokens, fused option): one token on the fused kernel and on the multi-kernel
# path; three tokens take the multi-kernel path whatever the option
@pytest.mark.parametrize("tokens,fused", [(1, 1), (1, 0), (2, 1), (3, 1)])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("case", ["c1", "c2", "c3_l0", "c3_l16"])
def test_norm_block_matches_oracle(fused_default, case, weighted, tokens, fused):
    """MoE(RMSNorm(x)) in one call (folded into the fused kernel's activation
    staging: one launch per token up to two tokens) against the oracle's
    RMSNorm followed by its block, given the device's routes."""
    hip_ext = fused_default
    note(f"norm block {case} weighted={weighted} tokens={tokens} fused={fused}")
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, fused)
    shape, layer_index = _norm_case(case)
    layer = syn.build_experts(shape, layer=layer_index, device=DEV)
    dense = syn.build_dense(shape, layer=layer_index, device=DEV)
    # a residual stream is far from unit RMS: scale it, so a missing norm shows
    x = (syn.hidden_states(shape, tokens, tag="norm").float() * 7.5).to(torch.bfloat16)
    w = None
    if weighted:
        w = (1.0 + syn.normal((shape.hidden,), seed=5, std=0.25)).to(torch.bfloat16)
    out, logits, weights, indices = hip_ext.norm_moe_layer(layer, dense, x.to(DEV), shape.top_k, 1e-6,
                                                           None if w is None else w.to(DEV))
    torch.cuda.synchronize()
    out, logits, weights, indices = out.cpu(), logits.cpu(), weights.cpu(), indices.cpu()
    xn = om.rmsnorm(x, 1e-6, w)
    dense_c = dense_to_cpu(dense)
    ref_logits = torch.nn.functional.linear(xn, dense_c.router).float()
    # the device's sum of squares may round differently, moving a normalised
    # element by one bf16 ulp: its effect on a logit is far below 2^-12
    assert bool(((logits.float() - ref_logits).abs() <= ref_logits.abs() * 2.0 ** -7 + 2.0 ** -12).all())
    assert torch.equal(indices, om.topk_ordered(logits, shape.top_k))
    lay = {"router": dense_c.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense_c.shared_gate, "shared_up": dense_c.shared_up, "shared_down": dense_c.shared_down,
           "shared_expert_gate": dense_c.shared_expert_gate}
    ref, *_ = om.qwen_block(xn, lay, syn.DeviceLayerReader({layer_index: layer}), layer_index,
                            routes=(weights, indices))
    assert_close(out, ref, f"norm block {case} weighted={weighted} tokens={tokens} fused={fused}")
