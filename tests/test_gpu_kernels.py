"""GPU parity of the HIP kernels (through the C ABI) against the CPU oracle.

Tolerances (north star): outputs rel-L2 <= 1e-2 and max-abs <= 2e-2 in bf16
with fp32 accumulation; expert indices bit-exact given identical logits;
permutation and index work bit-exact.
"""

from __future__ import annotations

import sys
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import codec as oc
from oracle import moe as om
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.native_backend import DenseBlock, DeviceExperts

pytestmark = pytest.mark.gpu

REL_L2 = 1e-2
MAX_ABS = 2e-2
DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(layer: DeviceExperts) -> DeviceExperts:
    mv = lambda t: None if t is None else t.to(DEV)
    return replace(layer, gate=mv(layer.gate), gate_scales=mv(layer.gate_scales), up=mv(layer.up),
                   up_scales=mv(layer.up_scales), down=mv(layer.down), down_scales=mv(layer.down_scales))


def dense_to_dev(d: DenseBlock) -> DenseBlock:
    mv = lambda t: None if t is None else t.to(DEV)
    return DenseBlock(mv(d.router), mv(d.shared_gate), mv(d.shared_up), mv(d.shared_down), mv(d.shared_expert_gate))


def dense_to_cpu(d: DenseBlock) -> DenseBlock:
    mv = lambda t: None if t is None else t.cpu()
    return DenseBlock(mv(d.router), mv(d.shared_gate), mv(d.shared_up), mv(d.shared_down), mv(d.shared_expert_gate))


def assert_close(got: torch.Tensor, ref: torch.Tensor, what: str, rel=REL_L2, mx=MAX_ABS):
    r = om.rel_l2(got.cpu(), ref.cpu())
    m = om.max_abs(got.cpu(), ref.cpu())
    print(f"  {what}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    assert torch.isfinite(got.float()).all(), what
    assert r <= rel, f"{what}: rel-L2 {r}"
    assert m <= mx, f"{what}: max-abs {m}"


def assert_bf16_rounded(got: torch.Tensor, ref: torch.Tensor, what: str, rel=4e-3, slack=2e-3):
    """For a single bf16-rounded output of an FP32 sum: each element may differ
    from the exact value by one bf16 rounding (half an ulp, at most 2^-8 of its
    magnitude) plus a small absolute slack for the FP32 summation order."""
    g, r = got.cpu().float(), ref.cpu().float()
    err = (g - r).abs()
    bound = r.abs() * 2.0 ** -8 + slack
    worst = float((err - bound).max())
    print(f"  {what}: rel_l2={om.rel_l2(g, r):.3e} max_abs={float(err.max()):.3e} worst_over_bound={worst:.3e}",
          flush=True)
    assert torch.isfinite(g).all(), what
    assert om.rel_l2(g, r) <= rel, f"{what}: rel-L2"
    assert worst <= 0.0, f"{what}: an element exceeds one bf16 rounding + {slack}"


def assert_weights_follow_logits(logits, weights, indices, norm=False, what="routing weights"):
    """weights == bf16(softmax_f32(logits)[indices]) (renormalised over the k
    selected when ``norm``), to one bf16 ulp; indices bit-exact given the logits."""
    lc, wc, ic = logits.cpu(), weights.cpu(), indices.cpu()
    assert torch.equal(ic, om.topk_ordered(lc, ic.shape[-1])), f"{what}: indices"
    p = torch.softmax(lc.float(), dim=-1).gather(-1, ic)
    if norm:
        p = p / p.sum(-1, keepdim=True)
    ref = p.to(torch.bfloat16).view(torch.int16).int()
    got = wc.to(torch.bfloat16).view(torch.int16).int()
    ulps = int((ref - got).abs().max())
    print(f"  {what}: max bf16 ulp difference {ulps}", flush=True)
    assert ulps <= 1, f"{what}: weights differ from softmax(logits) by {ulps} ulp"


# ------------------------------------------------------------------ linear --
@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
@pytest.mark.parametrize("rows,n,k", [(1, 64, 2048), (3, 96, 1408), (7, 40, 768), (4, 256, 5632)])
def test_linear_matches_oracle(hip_ext, encoding, rows, n, k):
    note(f"linear {encoding} rows={rows} n={n} k={k}")
    g = torch.Generator().manual_seed(rows * 1000 + n + k)
    w = torch.randn(1, n, k, generator=g) * 0.02
    data, scales = syn.encode_projection(w, encoding)
    x = torch.randn(rows, k, generator=g).to(torch.bfloat16)
    if encoding == "q4_group128":
        deq = oc.q4_dequantize(data.numpy().tobytes(), scales.numpy().tobytes(), (n, k))
        got = hip_ext.q4_linear(x.to(DEV), data[0].to(DEV), scales[0].to(DEV), n, k, 128)
    elif encoding == "q8_group128":
        deq = oc.q8_dequantize(data.numpy().tobytes(), scales.numpy().tobytes(), (n, k))
        got = hip_ext.q8_linear(x.to(DEV), data[0].to(DEV), scales[0].to(DEV), n, k, 128)
    else:
        deq = data[0].float().numpy()
        got = hip_ext.bf16_linear(x.to(DEV), data[0].to(DEV))
    ref = x.float() @ torch.from_numpy(deq).T
    assert_bf16_rounded(got, ref, "linear")


def test_q4_kernel_decodes_reserved_minus_eight(hip_ext):
    """The codec rejects -8, but the kernel decodes full two's complement
    (reference kernel src/uma_qmoe/native/packed_q4_kernel.cu:62-70)."""
    note("q4 -8 decode")
    n, k = 8, 256
    rng = np.random.default_rng(0)
    codes = rng.integers(-8, 8, size=(n, k)).astype(np.int8)
    codes[:, 0] = -8
    nib = (codes.astype(np.int16) & 0xF).astype(np.uint8).reshape(n, k // 2, 2)
    packed = torch.from_numpy(nib[..., 0] | (nib[..., 1] << 4))
    scales = torch.from_numpy(rng.uniform(0.001, 0.01, size=(n * k // 128,)).astype(np.float32))
    x = torch.randn(2, k).to(torch.bfloat16)
    got = hip_ext.q4_linear(x.to(DEV), packed.to(DEV), scales.to(DEV), n, k, 128)
    deq = codes.astype(np.float32) * np.repeat(scales.numpy(), 128).reshape(n, k)
    ref = x.float() @ torch.from_numpy(deq).T
    assert_bf16_rounded(got, ref, "q4 with -8")


def test_q4_groups_crossing_rows(hip_ext):
    """Scale groups run over the flattened tensor (src/uma_qmoe/q4.py:146-159):
    with K=64 and group 128 one group spans two rows."""
    note("q4 flattened groups K=64")
    n, k = 16, 64
    w = torch.randn(n, k) * 0.02
    packed, scales = oc.q4_quantize(w.numpy(), 128)
    x = torch.randn(3, k).to(torch.bfloat16)
    got = hip_ext.q4_linear(x.to(DEV), torch.frombuffer(bytearray(packed), dtype=torch.uint8).to(DEV),
                            torch.frombuffer(bytearray(scales), dtype=torch.float32).to(DEV), n, k, 128)
    ref = x.float() @ torch.from_numpy(oc.q4_dequantize(packed, scales, (n, k))).T
    assert_bf16_rounded(got, ref, "crossing groups")


# ----------------------------------------------------------------- routing --
@pytest.mark.parametrize("t,k,e", [(1, 4, 60), (5, 8, 64), (512, 4, 60), (256, 8, 128), (33, 2, 256), (384, 8, 128),
                                   (1000, 4, 60)])
def test_route_permute_is_a_stable_sort(hip_ext, t, k, e):
    note(f"permute t={t} k={k} e={e}")
    g = torch.Generator().manual_seed(t + k + e)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
    order, offsets = hip_ext.route_permute(idx.to(DEV), e)
    flat = idx.reshape(-1)
    assert torch.equal(order.cpu(), torch.argsort(flat, stable=True))
    counts = torch.bincount(flat, minlength=e)
    assert torch.equal(offsets.cpu(), torch.cat((torch.zeros(1, dtype=torch.int64), counts.cumsum(0))))


def test_route_permute_drops_invalid_ids(hip_ext):
    note("permute invalid ids")
    idx = torch.tensor([[3, -1], [70, 3], [0, 5]])
    order, offsets = hip_ext.route_permute(idx.to(DEV), 8)
    ref_order, ref_offsets = om.route_permutation(idx, 8)
    assert ref_order == [4, 0, 3, 5] and ref_offsets == [0, 1, 1, 1, 3, 3, 4, 4, 4]
    assert order.cpu()[: int(offsets[-1])].tolist() == ref_order
    assert offsets.cpu().tolist() == ref_offsets
    # many routes (the workgroup-parallel sort), ids out of range sprinkled in
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(-3, 70, (700, 4), generator=g)
    order, offsets = hip_ext.route_permute(idx.to(DEV), 64)
    ref_order, ref_offsets = om.route_permutation(idx, 64)
    assert order.cpu()[: int(offsets[-1])].tolist() == ref_order
    assert offsets.cpu().tolist() == ref_offsets


@pytest.mark.parametrize("t,e,k", [(1, 60, 4), (7, 64, 8), (64, 128, 8)])
def test_router_topk_bit_exact_given_logits(hip_ext, t, e, k):
    note(f"router t={t} e={e} k={k}")
    g = torch.Generator().manual_seed(e * t)
    x = torch.randn(t, 2048, generator=g).to(torch.bfloat16)
    w = (torch.randn(e, 2048, generator=g) * 0.02).to(torch.bfloat16)
    logits, weights, indices = hip_ext.router_topk(x.to(DEV), w.to(DEV), k)
    logits, weights, indices = logits.cpu(), weights.cpu(), indices.cpu()
    ref_logits = torch.nn.functional.linear(x, w)
    # logits: fp32 accumulation in a different order; at most one bf16 ulp apart
    ulp = (ref_logits.float().abs() * 2.0 ** -7).clamp_min(2.0 ** -126)
    assert ((logits.float() - ref_logits.float()).abs() <= ulp).all()
    # selection is bit-exact given the kernel's own logits
    assert torch.equal(indices, om.topk_ordered(logits, k))
    probs = torch.softmax(logits.float(), -1).gather(-1, indices)
    assert (weights.float() - probs).abs().max() <= 2.0 ** -8 * probs.max() + 1e-6


def test_router_forced_ties_go_to_lower_id(hip_ext):
    note("router forced ties")
    g = torch.Generator().manual_seed(9)
    base = (torch.randn(4, 2048, generator=g) * 0.02).to(torch.bfloat16)
    w = base[torch.tensor([0, 1, 1, 2, 1, 3, 3, 0])]  # identical rows -> identical logits
    x = torch.randn(16, 2048, generator=g).to(torch.bfloat16)
    logits, _, indices = hip_ext.router_topk(x.to(DEV), w.to(DEV), 3)
    assert torch.equal(indices.cpu(), om.topk_ordered(logits.cpu(), 3))
    lc = logits.cpu().float()
    for tt in range(16):
        sel = indices.cpu()[tt].tolist()
        for a, b in zip(sel, sel[1:]):
            assert lc[tt, a] > lc[tt, b] or (lc[tt, a] == lc[tt, b] and a < b)


# ----------------------------------------------------------------- experts --
SMALL = syn.MoEShape("small_q4", 256, 8, 2, 128)


def _routes(t, k, e, seed):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
    w = torch.rand(t, k, generator=g).to(torch.bfloat16)
    return idx, w


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
@pytest.mark.parametrize("t", [1, 2, 3, 4, 9])
def test_moe_forward_small(hip_ext, encoding, t):
    note(f"moe_forward small {encoding} t={t}")
    shape = replace(SMALL, encoding=encoding)
    layer = syn.build_experts(shape, seed=t)
    reader = syn.DeviceLayerReader({0: layer})
    x = syn.hidden_states(shape, t, seed=t)
    idx, w = _routes(t, shape.top_k, shape.num_experts, t)
    got = hip_ext.moe_forward(to_dev(layer), x.to(DEV), idx.to(DEV), w.to(DEV))
    ref = om.streaming_reference(x, idx, w, 0, reader, num_experts=shape.num_experts)
    assert_close(got, ref, f"{encoding} t={t}")


def test_moe_forward_edge_cases(hip_ext):
    note("moe_forward edge cases")
    layer = syn.build_experts(SMALL, seed=3)
    dl = to_dev(layer)
    reader = syn.DeviceLayerReader({0: layer})
    x = syn.hidden_states(SMALL, 4, seed=3)
    # duplicate expert inside one token
    idx = torch.tensor([[2, 2], [1, 7], [7, 1], [0, 0]])
    w = torch.tensor([[0.5, 0.25], [0.3, 0.7], [0.7, 0.3], [1.0, 0.0]]).to(torch.bfloat16)
    got = hip_ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV))
    ref = om.streaming_reference(x, idx, w, 0, reader, num_experts=8)
    assert_close(got, ref, "duplicates")
    # zero weights -> zero output
    z = hip_ext.moe_forward(dl, x.to(DEV), idx.to(DEV), torch.zeros_like(w).to(DEV))
    assert torch.count_nonzero(z) == 0
    # an invalid expert id contributes nothing (the reference kernel skips it)
    bad = torch.tensor([[2, 99], [1, 7], [7, 1], [0, -3]])
    got_bad = hip_ext.moe_forward(dl, x.to(DEV), bad.to(DEV), w.to(DEV))
    keep = torch.tensor([[2, 0], [1, 7], [7, 1], [0, 0]])
    wk = w.clone()
    wk[0, 1] = 0
    wk[3, 1] = 0
    ref_bad = om.streaming_reference(x, keep, wk, 0, reader, num_experts=8)
    assert_close(got_bad, ref_bad, "invalid ids")
    # no tokens
    empty = hip_ext.moe_forward(dl, x[:0].to(DEV), idx[:0].to(DEV), w[:0].to(DEV))
    assert empty.shape == (0, SMALL.hidden)
    # int32 indices and k=1
    got1 = hip_ext.moe_forward(dl, x.to(DEV), idx[:, :1].to(torch.int32).to(DEV), w[:, :1].to(DEV))
    ref1 = om.streaming_reference(x, idx[:, :1], w[:, :1], 0, reader, num_experts=8)
    assert_close(got1, ref1, "k=1 int32")


@pytest.mark.parametrize("name,t", [("c1", 1), ("c1", 3), ("c2", 1), ("c2", 4), ("c5", 1)])
def test_moe_forward_benchmark_shapes(hip_ext, name, t):
    shape = syn.CONFIGS[name]
    note(f"moe_forward {shape.name} t={t}")
    layer = syn.build_experts(shape, device=DEV)
    reader = syn.DeviceLayerReader({0: layer})
    x = syn.hidden_states(shape, t)
    idx, w = _routes(t, shape.top_k, shape.num_experts, 17 + t)
    got = hip_ext.moe_forward(layer, x.to(DEV), idx.to(DEV), w.to(DEV))
    ref = om.streaming_reference(x, idx, w, 0, reader, num_experts=shape.num_experts)
    assert_close(got, ref, f"{shape.name} t={t}")


# expert counts at which the shared-expert gate column (index E) of the router
# output falls on lane 0 of the second and of the fifth 64-column slice
GATE_COLUMN_SHAPES = {"e64_shared": syn.MoEShape("e64_shared", 256, 64, 2, 128, 128),
                      "e256_shared": syn.MoEShape("e256_shared", 256, 256, 2, 128, 128)}


@pytest.mark.parametrize("name,t", [("c2", 1), ("c1", 1), ("c2", 3), ("e64_shared", 3), ("e256_shared", 3)])
def test_moe_layer_matches_oracle_block(hip_ext, name, t):
    """Whole block: router + routed + shared + sigmoid gate, one C-ABI call."""
    shape = GATE_COLUMN_SHAPES[name] if name in GATE_COLUMN_SHAPES else syn.CONFIGS[name]
    note(f"moe_layer {shape.name} t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    reader = syn.DeviceLayerReader({0: layer})
    x = syn.hidden_states(shape, t)
    out, logits, weights, indices = hip_ext.moe_layer(layer, dense, x.to(DEV), shape.top_k)
    logits_c, weights_c, indices_c = logits.cpu(), weights.cpu(), indices.cpu()
    assert torch.equal(indices_c, om.topk_ordered(logits_c, shape.top_k))
    dense_c = DenseBlock(*(None if v is None else v.cpu() for v in (
        dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate)))
    ref_logits = torch.nn.functional.linear(x, dense_c.router)
    ulp = (ref_logits.float().abs() * 2.0 ** -7).clamp_min(2.0 ** -126)
    assert ((logits_c.float() - ref_logits.float()).abs() <= ulp).all()
    lay = {"router": dense_c.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense_c.shared_gate, "shared_up": dense_c.shared_up, "shared_down": dense_c.shared_down,
           "shared_expert_gate": dense_c.shared_expert_gate}
    ref, *_ = om.qwen_block(x, lay, reader, 0, routes=(weights_c, indices_c))
    assert_close(out, ref, f"{shape.name} block t={t}")


@pytest.mark.parametrize("t", [768, 769])
def test_block_topk_permute_fusion_boundary(hip_ext, t):
    """768 tokens x top-4 = 3072 routes take the top-k and the permutation in
    one launch (the last workgroup to finish its top-k permutes), 769 tokens
    take two launches. Indices follow the kernel's logits exactly, sampled
    tokens match the oracle block, and a second call on the same workspace
    (whose completion counter the first call must leave at zero) gives the
    same bits."""
    shape = syn.MoEShape("routes_3072", 256, 16, 4, 128, 128)
    note(f"top-k + permute fusion boundary t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    reader = syn.DeviceLayerReader({0: layer})
    x = syn.hidden_states(shape, t, seed=5)
    out, logits, weights, indices = hip_ext.moe_layer(layer, dense, x.to(DEV), shape.top_k)
    out = out.clone()
    logits_c, weights_c, indices_c = logits.cpu(), weights.cpu(), indices.cpu()
    assert_weights_follow_logits(logits_c, weights_c, indices_c, False, f"fusion boundary t={t}")
    dense_c = DenseBlock(*(None if v is None else v.cpu() for v in (
        dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate)))
    lay = {"router": dense_c.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense_c.shared_gate, "shared_up": dense_c.shared_up, "shared_down": dense_c.shared_down,
           "shared_expert_gate": dense_c.shared_expert_gate}
    pick = torch.randperm(t, generator=torch.Generator().manual_seed(t))[:16].sort().values
    ref, *_ = om.qwen_block(x[pick], lay, reader, 0, routes=(weights_c[pick], indices_c[pick]))
    assert_close(out.cpu()[pick], ref, f"sampled tokens t={t}")
    again = hip_ext.moe_layer(layer, dense, x.to(DEV), shape.top_k)[0]
    assert torch.equal(again, out)


@pytest.mark.parametrize("layer_index", [0, 16])
def test_c3_stack_layer_encodings(hip_ext, layer_index):
    """c3: routed BF16 (layers 0-15) and Q8 (layers 16-23) blocks with shared expert."""
    shape = syn.c3_layer_shape(layer_index)
    note(f"c3 layer {layer_index} {shape.encoding}")
    layer = syn.build_experts(shape, layer=layer_index, device=DEV)
    dense = syn.build_dense(shape, layer=layer_index, device=DEV)
    reader = syn.DeviceLayerReader({layer_index: layer})
    x = om.rmsnorm(syn.hidden_states(shape, 1, tag="c3"), 1e-6)
    xr = hip_ext.rmsnorm(syn.hidden_states(shape, 1, tag="c3").to(DEV), 1e-6)
    # rsqrt differs in the last fp32 bits; after the bf16 cast at most one ulp apart
    assert ((xr.cpu().float() - x.float()).abs() <= x.float().abs() * 2.0 ** -7 + 1e-30).all()
    out, logits, weights, indices = hip_ext.moe_layer(layer, dense, xr, shape.top_k)
    dense_c = DenseBlock(*(None if v is None else v.cpu() for v in (
        dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate)))
    lay = {"router": dense_c.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense_c.shared_gate, "shared_up": dense_c.shared_up, "shared_down": dense_c.shared_down,
           "shared_expert_gate": dense_c.shared_expert_gate}
    ref, *_ = om.qwen_block(x, lay, reader, layer_index, routes=(weights.cpu(), indices.cpu()))
    assert_close(out, ref, f"c3 layer {layer_index}")


def test_c3_stack_chain(hip_ext):
    """c3 stack driver: x <- MoE_l(RMSNorm(x)) chained on the device through
    BF16 layers 0 and 15 and Q8 layers 16 and 23 for two decode steps. Every
    layer is checked against the oracle given the same device input and the
    device's routes (a free-running bf16 chain drifts by the rounding of every
    layer, which a fixed tolerance cannot tell from a defect)."""
    layer_ids = (0, 15, 16, 23)
    parts = {}
    for l in layer_ids:
        shape = syn.c3_layer_shape(l)
        layer = syn.build_experts(shape, layer=l, device=DEV)
        dense = syn.build_dense(shape, layer=l, device=DEV)
        dense_c = DenseBlock(*(None if v is None else v.cpu() for v in (
            dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate)))
        lay = {"router": dense_c.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
               "shared_gate": dense_c.shared_gate, "shared_up": dense_c.shared_up,
               "shared_down": dense_c.shared_down, "shared_expert_gate": dense_c.shared_expert_gate}
        parts[l] = (shape, layer, dense, lay, syn.DeviceLayerReader({l: layer}))
    x_g = syn.hidden_states(syn.c3_layer_shape(0), 1, tag="c3_chain").to(DEV)
    for step in range(2):
        for l in layer_ids:
            shape, layer, dense, lay, reader = parts[l]
            note(f"c3 chain step {step} layer {l} {shape.encoding}")
            x_in = x_g.cpu()
            n_g = hip_ext.rmsnorm(x_g, 1e-6)
            n_o = om.rmsnorm(x_in, 1e-6)
            assert ((n_g.cpu().float() - n_o.float()).abs() <= n_o.float().abs() * 2.0 ** -7 + 1e-30).all()
            x_g, _, weights, indices = hip_ext.moe_layer(layer, dense, n_g, shape.top_k)
            ref, *_ = om.qwen_block(n_g.cpu(), lay, reader, l, routes=(weights.cpu(), indices.cpu()))
            assert_close(x_g, ref, f"c3 chain step {step} layer {l}")


def test_workspace_reused_across_token_counts(hip_ext):
    """One zero-filled workspace serves calls of 1, 2, 32, 3 and 1 tokens in a
    row (fused single-token launches, then the multi-launch path with the
    side stream and the fused top-k + permutation): every call gives the same
    bits as the same call on a fresh workspace, so the synchronisation words
    each path leaves behind sit where the next token count looks for them."""
    shape = syn.C2
    note("workspace reuse across token counts")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    counts = (1, 2, 32, 3, 1)

    def ws_bytes(t):
        return hip_ext.lib.uqm_moe_workspace_bytes(t, shape.hidden, shape.intermediate, shape.shared_intermediate,
                                                   shape.num_experts, shape.top_k)

    shared_ws = torch.zeros(max(ws_bytes(t) for t in counts), dtype=torch.uint8, device=DEV)
    for i, t in enumerate(counts):
        x = syn.hidden_states(shape, t, seed=90 + i).to(DEV)
        got = [v.clone() for v in hip_ext.moe_layer(layer, dense, x, shape.top_k, workspace=shared_ws)]
        fresh = torch.zeros(ws_bytes(t), dtype=torch.uint8, device=DEV)
        ref = hip_ext.moe_layer(layer, dense, x, shape.top_k, workspace=fresh)
        for a, b, what in zip(got, ref, ("out", "logits", "weights", "indices")):
            assert torch.equal(a, b), f"t={t} {what}"
