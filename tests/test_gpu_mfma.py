"""GPU parity of the MFMA grouped-GEMM path and of the streaming GEMV path
(multi-token calls) against the CPU oracle and against the workgroup-staged
batched-GEMV path (independent HIP implementations of the same projections).

Tolerances: rel-L2 <= 1e-2, max-abs <= 2e-2 against the oracle (north star);
the two HIP paths compute the same FP32 sums in different orders, so their
bf16 outputs agree to a few bf16 ulps.
"""

from __future__ import annotations

import sys
from dataclasses import replace

import pytest
import torch

from oracle import moe as om
from test_gpu_kernels import assert_weights_follow_logits
from uma_qmoe_amd import _native
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.native_backend import DenseBlock, DeviceExperts

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
REL_L2 = 1e-2
MAX_ABS = 2e-2
# the smallest shape the grouped-GEMM paths take (K >= 768 for both projections)
MID = syn.MoEShape("mid", 1024, 16, 4, 768)


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(layer: DeviceExperts) -> DeviceExperts:
    mv = lambda t: None if t is None else t.to(DEV)
    return replace(layer, gate=mv(layer.gate), gate_scales=mv(layer.gate_scales), up=mv(layer.up),
                   up_scales=mv(layer.up_scales), down=mv(layer.down), down_scales=mv(layer.down_scales))


def dense_cpu(d: DenseBlock) -> DenseBlock:
    return DenseBlock(*(None if v is None else v.cpu() for v in (
        d.router, d.shared_gate, d.shared_up, d.shared_down, d.shared_expert_gate)))


def layout_of(shape, d: DenseBlock) -> dict:
    return {"router": d.router, "top_k": shape.top_k, "num_experts": shape.num_experts, "shared_gate": d.shared_gate,
            "shared_up": d.shared_up, "shared_down": d.shared_down, "shared_expert_gate": d.shared_expert_gate,
            "norm_topk_prob": shape.norm_topk_prob}


def close(got, ref, what, rel=REL_L2, mx=MAX_ABS):
    r = om.rel_l2(got.cpu(), ref.cpu())
    m = om.max_abs(got.cpu(), ref.cpu())
    print(f"  {what}: rel_l2={r:.3e} max_abs={m:.3e}", flush=True)
    assert torch.isfinite(got.float()).all(), what
    assert r <= rel, f"{what}: rel-L2 {r}"
    assert m <= mx, f"{what}: max-abs {m}"


def within_ulps(got, ref, what, ulps=2, rel=5e-3):
    """Two HIP paths that sum the same FP32 products in different orders:
    every bf16 output within `ulps` bf16 ulps of the other path's, rel-L2 <=
    rel. The ulp is that of the larger magnitude (2^(e - 7) for |y| in
    [2^e, 2^(e+1))), at least the ulp of the outputs' RMS: near zero the sums'
    rounding error follows the size of their terms, not of the result."""
    a, b = got.cpu().float(), ref.cpu().float()
    r = om.rel_l2(a, b)
    rms = b.pow(2).mean().sqrt().item()
    mag = torch.maximum(a.abs(), b.abs()).clamp_min(max(rms, 2.0 ** -126))
    ulp = torch.exp2(torch.floor(torch.log2(mag)) - 7)
    worst = ((a - b).abs() / ulp).max().item()
    print(f"  {what}: rel_l2={r:.3e} max_ulps={worst:.1f}", flush=True)
    assert torch.isfinite(a).all(), what
    assert r <= rel, f"{what}: rel-L2 {r}"
    assert worst <= ulps, f"{what}: {worst} bf16 ulps"


def routes(t, k, e, seed, hot=None, hot_share=0.0):
    g = torch.Generator().manual_seed(seed)
    idx = torch.stack([torch.randperm(e, generator=g)[:k] for _ in range(t)])
    if hot is not None:
        take = torch.rand(t, generator=g) < hot_share
        idx[take, 0] = hot
        # keep each token's experts distinct
        for r in torch.nonzero(take).flatten().tolist():
            row = idx[r]
            for s in range(1, k):
                if row[s] == hot:
                    row[s] = next(c for c in range(e) if c not in row.tolist())
    w = torch.rand(t, k, generator=g).to(torch.bfloat16)
    return idx, w


STREAM_DEFAULT = 32  # UQM_OPT_STREAM_MAX_ROUTES default (routes per call)
STREAM_ALWAYS = 1 << 30


def restore_defaults(ext) -> None:
    ext.set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, 2)
    ext.set_option(_native.UQM_OPT_FUSED_DECODE, 1)
    ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, STREAM_DEFAULT)


@pytest.fixture
def mfma_on(hip_ext):
    # two-token blocks would take the fused kernel once per token; the
    # streaming GEMV would take the calls with few routes per expert
    hip_ext.set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, 2)
    hip_ext.set_option(_native.UQM_OPT_FUSED_DECODE, 0)
    hip_ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, 0)
    yield hip_ext
    restore_defaults(hip_ext)


def both_paths(ext, fn):
    """(MFMA grouped GEMMs, workgroup-staged GEMV) results of fn."""
    ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, 0)
    ext.set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, 2)
    a = fn()
    ext.set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, 0)
    b = fn()
    ext.set_option(_native.UQM_OPT_MFMA_MIN_TOKENS, 2)
    torch.cuda.synchronize()
    return a, b


def streamed(ext, fn, threshold=STREAM_ALWAYS):
    """fn's result with the routed projections on the streaming GEMV."""
    ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, threshold)
    try:
        out = fn()
        torch.cuda.synchronize()
    finally:
        ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, 0)
    return out


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
@pytest.mark.parametrize("t", [2, 16, 37, 100, 300])
def test_routed_matches_oracle_and_gemv(mfma_on, encoding, t):
    """Routed experts on the grouped-GEMM kernel against the oracle and the
    GEMV path."""
    ext = mfma_on
    shape = replace(MID, encoding=encoding)
    note(f"mfma routed {encoding} t={t}")
    layer = syn.build_experts(shape, seed=t)
    dl = to_dev(layer)
    x = syn.hidden_states(shape, t, seed=t)
    idx, w = routes(t, shape.top_k, shape.num_experts, 100 + t)
    got, gemv = both_paths(ext, lambda: ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV)))
    ref = om.streaming_reference(x, idx, w, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got, ref, f"mfma vs oracle {encoding} t={t}")
    close(got, gemv, f"mfma vs gemv {encoding} t={t}", rel=5e-3, mx=1e-2)


@pytest.mark.parametrize("encoding", ["q4_group128", "q8_group128", "bf16_le"])
@pytest.mark.parametrize("t", [1, 2, 3, 16, 37, 100])
def test_stream_matches_oracle_and_mfma(mfma_on, encoding, t):
    """Routed experts on the streaming GEMV (forced for every route count, so
    experts with more routes than a wave holds take several passes, and rows
    of 24 chunks leave most lanes idle) against the oracle and the MFMA and
    staged-GEMV paths."""
    ext = mfma_on
    shape = replace(MID, encoding=encoding)
    note(f"stream routed {encoding} t={t}")
    layer = syn.build_experts(shape, seed=t)
    dl = to_dev(layer)
    x = syn.hidden_states(shape, t, seed=t)
    idx, w = routes(t, shape.top_k, shape.num_experts, 100 + t)
    call = lambda: ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV))
    got = streamed(ext, call)
    mfma, gemv = both_paths(ext, call)
    ref = om.streaming_reference(x, idx, w, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got, ref, f"stream vs oracle {encoding} t={t}")
    close(got, gemv, f"stream vs gemv {encoding} t={t}", rel=5e-3, mx=1e-2)
    if t >= 2:
        close(got, mfma, f"stream vs mfma {encoding} t={t}", rel=5e-3, mx=1e-2)
    # invalid ids contribute nothing on this path too
    idx2 = idx.clone()
    idx2[::3, 0] = -1
    got2 = streamed(ext, lambda: ext.moe_forward(dl, x.to(DEV), idx2.to(DEV), w.to(DEV)))
    w2 = w.clone()
    w2[::3, 0] = 0
    ref2 = om.streaming_reference(x, idx, w2, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got2, ref2, f"stream dropped ids {encoding} t={t}")


@pytest.mark.parametrize("t", [3, 5, 8])
def test_qwen_block_stream_decode(mfma_on, t):
    """c2 shapes at batch 3, 5 and 8 with the default threshold (at most 32
    routes, so the streaming GEMV takes the routed experts): against the
    oracle block and the MFMA path, eagerly and replayed from a HIP graph."""
    ext = mfma_on
    shape = syn.C2
    note(f"stream qwen block t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, t, seed=90 + t).to(DEV)
    out, logits, weights, indices = [v.clone() for v in
                                     streamed(ext, lambda: ext.moe_layer(layer, dense, x, shape.top_k), STREAM_DEFAULT)]
    assert_weights_follow_logits(logits, weights, indices, False, f"c2 stream block t={t}")
    ref, *_ = om.qwen_block(x.cpu(), layout_of(shape, dense_cpu(dense)), syn.DeviceLayerReader({0: layer}), 0,
                            routes=(weights.cpu(), indices.cpu()))
    close(out, ref, f"c2 stream block t={t}")
    mfma = ext.moe_layer(layer, dense, x, shape.top_k)[0]
    close(out, mfma, f"c2 stream vs mfma t={t}", rel=5e-3, mx=1e-2)
    ws = torch.zeros(ext.lib.uqm_moe_workspace_bytes(t, shape.hidden, shape.intermediate, shape.shared_intermediate,
                                                     shape.num_experts, shape.top_k), dtype=torch.uint8, device=DEV)
    ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, STREAM_DEFAULT)
    try:
        res = torch.empty_like(x)
        ext.moe_layer(layer, dense, x, shape.top_k, out=res, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(res, out), "workspace call"
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ext.moe_layer(layer, dense, x, shape.top_k, out=res, workspace=ws)
        for rep in range(3):
            res.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(res, out), f"graph replay {rep}"
            ext.moe_layer(layer, dense, x, shape.top_k, workspace=ws)
        del graph
    finally:
        ext.set_option(_native.UQM_OPT_STREAM_MAX_ROUTES, 0)


@pytest.mark.parametrize("encoding", ["q4_group128", "bf16_le"])
def test_hot_expert_spans_many_tiles(mfma_on, encoding):
    """One expert takes ~85% of 300 tokens (k=2): it is split into many route
    tiles that share its weight rows; idle experts get no tile."""
    ext = mfma_on
    shape = replace(MID, encoding=encoding, top_k=2)
    note(f"mfma hot expert {encoding}")
    layer = syn.build_experts(shape, seed=5)
    dl = to_dev(layer)
    t = 300
    x = syn.hidden_states(shape, t, seed=5)
    idx, w = routes(t, 2, shape.num_experts, 7, hot=5, hot_share=0.85)
    got = ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV))
    ref = om.streaming_reference(x, idx, w, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got, ref, f"hot expert {encoding}")
    # invalid ids are dropped on this path too
    idx2 = idx.clone()
    idx2[::7, 1] = -1
    got2 = ext.moe_forward(dl, x.to(DEV), idx2.to(DEV), w.to(DEV))
    w2 = w.clone()
    w2[::7, 1] = 0
    idx3 = idx.clone()
    ref2 = om.streaming_reference(x, idx3, w2, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got2, ref2, f"dropped ids {encoding}")


def test_48_route_tiles(mfma_on):
    """Q4, 32 experts x 1024 rows, 300 tokens top-4: 37.5 routes per expert on
    average, so the routed projections take 48-route tiles (3 x 16 tokens per
    MFMA item; every expert's rows x 32 experts fill the 256 CUs). One expert
    takes ~30% of the tokens (three tiles, the last one partial); the others
    fill 25-46 of one tile. Against the oracle and the GEMV path."""
    ext = mfma_on
    shape = syn.MoEShape("tile48", 2048, 32, 4, 1024)
    note("mfma 48-route tiles")
    layer = syn.build_experts(shape, seed=11)
    dl = to_dev(layer)
    t = 300
    x = syn.hidden_states(shape, t, seed=11)
    idx, w = routes(t, 4, shape.num_experts, 13, hot=3, hot_share=0.3)
    counts = torch.bincount(idx.flatten(), minlength=shape.num_experts)
    assert 32 < idx.numel() / shape.num_experts <= 48 and counts.max() > 96 and counts.min() > 0
    got, got_g = both_paths(ext, lambda: ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV)))
    ref = om.streaming_reference(x, idx, w, 0, syn.DeviceLayerReader({0: layer}), num_experts=shape.num_experts)
    close(got, ref, "48-route tiles")
    close(got, got_g, "48-route tiles mfma vs gemv", rel=5e-3, mx=1e-2)


# K / 128 odd in both projections (H = 1152: 9 scale groups, I = 896: 7)
ODD = syn.MoEShape("odd_k", 1152, 40, 4, 896)


@pytest.mark.parametrize("t", [6, 32, 200, 400])
def test_q4_odd_group_count(mfma_on, t):
    """Q4 projections whose K holds an odd number of 128-element scale groups,
    so the 16-route gate/up tiles cannot take two-group steps (K a multiple of
    256; the MID shape's gate/up and the c2 block's at batch 16 and 32 take
    them) and run one group per step. The planner takes (gate/up; down): t=6
    64-row items (down with two K-split partials when the items are few); t=32
    128-row items, 16-route tiles; t=200 32-route tiles; t=400 48-route tiles.
    Against the oracle and the GEMV path."""
    ext = mfma_on
    note(f"mfma odd group count t={t}")
    layer = syn.build_experts(ODD, seed=60 + t)
    dl = to_dev(layer)
    x = syn.hidden_states(ODD, t, seed=60 + t)
    idx, w = routes(t, ODD.top_k, ODD.num_experts, 160 + t)
    got, gemv = both_paths(ext, lambda: ext.moe_forward(dl, x.to(DEV), idx.to(DEV), w.to(DEV)))
    ref = om.streaming_reference(x, idx, w, 0, syn.DeviceLayerReader({0: layer}), num_experts=ODD.num_experts)
    close(got, ref, f"odd groups vs oracle t={t}")
    close(got, gemv, f"odd groups mfma vs gemv t={t}", rel=5e-3, mx=1e-2)


@pytest.mark.parametrize("t", [2, 16, 32])
def test_qwen_block_batched_decode(mfma_on, t):
    """c2 shapes at batch 2, 16 and 32: router, routed Q4 experts and the BF16
    shared expert on the MFMA path, against the oracle block."""
    ext = mfma_on
    shape = syn.C2
    note(f"mfma qwen block t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, t, seed=40 + t)
    (out, logits, weights, indices), (out_g, *_rest) = both_paths(
        ext, lambda: ext.moe_layer(layer, dense, x.to(DEV), shape.top_k))
    assert_weights_follow_logits(logits, weights, indices, False, f"c2 block t={t}")
    ref, *_ = om.qwen_block(x, layout_of(shape, dense_cpu(dense)), syn.DeviceLayerReader({0: layer}), 0,
                            routes=(weights.cpu(), indices.cpu()))
    close(out, ref, f"c2 block t={t}")
    close(out, out_g, f"c2 block mfma vs gemv t={t}", rel=5e-3, mx=1e-2)


@pytest.mark.parametrize("t", [4, 32, 160])
def test_shared_expert_side_stream(mfma_on, t):
    """The shared expert forked onto the library's side stream (the default)
    gives the same bits as the in-order run on the caller's stream, eagerly and
    replayed from a HIP graph (several replays, eager work in between). At 160
    tokens the shared expert takes the dense kernel."""
    ext = mfma_on
    shape = syn.C2
    note(f"shared expert side stream t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, t, seed=70 + t).to(DEV)
    ws = torch.zeros(ext.lib.uqm_moe_workspace_bytes(t, shape.hidden, shape.intermediate, shape.shared_intermediate,
                                                     shape.num_experts, shape.top_k), dtype=torch.uint8, device=DEV)
    try:
        ext.set_option(_native.UQM_OPT_OVERLAP_SHARED, 0)
        ref = [v.clone() for v in ext.moe_layer(layer, dense, x, shape.top_k, workspace=ws)]
        ext.set_option(_native.UQM_OPT_OVERLAP_SHARED, 1)
        got = ext.moe_layer(layer, dense, x, shape.top_k, workspace=ws)
        for a, b, what in zip(got, ref, ("out", "logits", "weights", "indices")):
            assert torch.equal(a, b), f"eager {what}"
        out = torch.empty_like(x)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            ext.moe_layer(layer, dense, x, shape.top_k, out=out, workspace=ws)
        for rep in range(3):
            out.zero_()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref[0]), f"graph replay {rep}"
            # eager work between replays
            ext.moe_layer(layer, dense, x, shape.top_k, workspace=ws)
        del graph
    finally:
        ext.set_option(_native.UQM_OPT_OVERLAP_SHARED, 1)


RAGGED = syn.MoEShape("dense_ragged", 1088, 8, 2, 256, 1344, encoding="bf16_le")


@pytest.mark.parametrize("which,t", [("ragged", 128), ("ragged", 200), ("ragged", 300), ("c2", 200), ("c2", 384),
                                     ("c2", 1000)])
def test_dense_shared_expert(mfma_on, which, t):
    """From 128 tokens the shared expert takes the dense kernel: 4-wave items
    of 128 weight rows x 128 tokens, or 8-wave items of 256 tokens where they
    take fewer rounds over the CUs. The ragged shape has partial 128-token
    tiles, a hidden size of 1088 (the down projection's last 128-row block
    half full) and 1344 shared rows (21 K stages in the down projection: no K
    split); c2 at 200 tokens splits the down projection's K in four; at 384
    tokens the gate/up takes 8-wave items (the second 256-token tile half
    full); at 1000 tokens both projections take 8-wave items, the down
    projection with its K split in four. Against the oracle on sampled tokens
    (the last token always among them) and against the GEMV path on every
    token."""
    ext = mfma_on
    shape = RAGGED if which == "ragged" else syn.C2
    note(f"dense shared expert {which} t={t}")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, t, seed=90 + t)
    (out, logits, weights, indices), (out_g, *_rest) = both_paths(
        ext, lambda: ext.moe_layer(layer, dense, x.to(DEV), shape.top_k))
    within_ulps(out, out_g, f"dense shared {which} t={t} vs gemv")
    pick = torch.randperm(t, generator=torch.Generator().manual_seed(t))[:12]
    pick = torch.unique(torch.cat([pick, torch.tensor([t - 1])]))
    ref, *_ = om.qwen_block(x[pick], layout_of(shape, dense_cpu(dense)), syn.DeviceLayerReader({0: layer}), 0,
                            routes=(weights.cpu()[pick], indices.cpu()[pick]))
    close(out.cpu()[pick], ref, f"dense shared {which} t={t} sampled tokens vs oracle")


def test_c4_prefill_512_tokens(mfma_on):
    """c4: 512 tokens through the whole block (MFMA routed + shared). Every
    token's result depends only on its own routes, so 16 sampled tokens are
    checked against the oracle, all 512 against the GEMV path, and the top-k
    selection of all 512 against the kernel's own logits."""
    ext = mfma_on
    shape = syn.C4
    note("mfma c4 T=512")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape, device=DEV)
    x = syn.hidden_states(shape, 512, seed=4)
    (out, logits, weights, indices), (out_g, *_rest) = both_paths(
        ext, lambda: ext.moe_layer(layer, dense, x.to(DEV), shape.top_k))
    assert_weights_follow_logits(logits, weights, indices, False, "c4 (512 tokens)")
    close(out, out_g, "c4 mfma vs gemv (512 tokens)", rel=5e-3, mx=1e-2)
    pick = torch.randperm(512, generator=torch.Generator().manual_seed(9))[:16].sort().values
    ref, *_ = om.qwen_block(x[pick], layout_of(shape, dense_cpu(dense)), syn.DeviceLayerReader({0: layer}), 0,
                            routes=(weights.cpu()[pick], indices.cpu()[pick]))
    close(out.cpu()[pick], ref, "c4 sampled tokens vs oracle")


def test_c5_zipf_256_tokens(mfma_on):
    """c5: 256 tokens, 128 experts, top-8, Zipf-biased routes (hot experts with
    > 100 routes next to experts with 0-2)."""
    ext = mfma_on
    shape = syn.C5
    note("mfma c5 T=256 zipf")
    layer = syn.build_experts(shape, device=DEV)
    dense = syn.build_dense(shape)
    x = syn.hidden_states(shape, 256, seed=5)
    bias = syn.zipf_router_bias(shape)
    lg = (torch.nn.functional.linear(x, dense.router).float() + bias).to(torch.bfloat16)
    idx = om.topk_ordered(lg, shape.top_k)
    w = torch.softmax(lg.float(), -1).gather(-1, idx).to(torch.bfloat16)
    counts = torch.bincount(idx.flatten(), minlength=shape.num_experts)
    print(f"  routes per expert: max={int(counts.max())} zero={int((counts == 0).sum())}", flush=True)
    assert int(counts.max()) > 100
    got, gemv = both_paths(ext, lambda: ext.moe_forward(layer, x.to(DEV), idx.to(DEV), w.to(DEV)))
    close(got, gemv, "c5 mfma vs gemv (256 tokens)", rel=5e-3, mx=1e-2)
    pick = torch.randperm(256, generator=torch.Generator().manual_seed(11))[:16].sort().values
    ref = om.streaming_reference(x[pick], idx[pick], w[pick], 0, syn.DeviceLayerReader({0: layer}),
                                 num_experts=shape.num_experts)
    close(got.cpu()[pick], ref, "c5 sampled tokens vs oracle")
