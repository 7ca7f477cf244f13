"""uqm_moe_layer_noalloc (the library's static scratch array, no workspace,
no allocation) against uqm_moe_layer on fresh workspaces, through the C ABI.

Calls in a row on the same scratch, each smaller than the one before (a
32-token MFMA call, a 3-token call, a single-token fused call): outputs,
logits, routing weights and indices equal the workspace entry point's bit
for bit, and the routed output is within the north-star tolerance of the
oracle. A call needing more than the array holds fails cleanly and leaves
the next call correct. A graph captured after the first (eager) call
replays to the eager bits with eager calls in between.
"""

from __future__ import annotations

import pytest
import torch

from oracle import moe as om
from test_gpu_kernels import DEV, assert_close, note
from uma_qmoe_amd import _native
from uma_qmoe_amd import synthetic as syn

pytestmark = pytest.mark.gpu


def _same(a, b, what):
    for x, y, name in zip(a, b, ("out", "logits", "weights", "indices")):
        assert torch.equal(x, y), f"{what}: {name} differs from uqm_moe_layer"


def _fresh(hip_ext, layer, dense, x, shape):
    ws = hip_ext.new_workspace(DEV, x.shape[0], shape.hidden, shape.intermediate, shape.shared_intermediate,
                               shape.num_experts, shape.top_k)
    return [t.clone() for t in hip_ext.moe_layer(layer, dense, x, shape.top_k, workspace=ws)]


def test_noalloc_matches_the_workspace_entry_point(hip_ext):
    shape = syn.C2
    layer = syn.build_experts(shape, device=DEV, seed=31)
    dense = syn.build_dense(shape, device=DEV, seed=31)
    reader = syn.DeviceLayerReader({0: layer})
    lay = {"router": dense.router.cpu(), "top_k": 4, "num_experts": 60, "shared_gate": dense.shared_gate.cpu(),
           "shared_up": dense.shared_up.cpu(), "shared_down": dense.shared_down.cpu(),
           "shared_expert_gate": dense.shared_expert_gate.cpu()}
    for t in (32, 3, 1):
        note(f"no-alloc c2 T={t}")
        x = syn.hidden_states(shape, t, seed=100 + t)
        got = [v.clone() for v in hip_ext.moe_layer_noalloc(layer, dense, x.to(DEV), 4)]
        ref = _fresh(hip_ext, layer, dense, x.to(DEV), shape)
        torch.cuda.synchronize()
        _same(got, ref, f"T={t}")
        pick = slice(0, min(t, 4))
        oracle, *_ = om.qwen_block(x[pick], lay, reader, 0, routes=(got[2].cpu()[pick], got[3].cpu()[pick]))
        assert_close(got[0].cpu()[pick], oracle, f"no-alloc T={t} vs oracle")
    # more than the scratch array holds: refused before any launch, nothing changed
    big = torch.zeros(1000, shape.hidden, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(_native.NativeError, match="uqm_moe_layer_noalloc"):
        hip_ext.moe_layer_noalloc(layer, dense, big, 4)
    x = syn.hidden_states(shape, 2, seed=7).to(DEV)
    _same([v.clone() for v in hip_ext.moe_layer_noalloc(layer, dense, x, 4)], _fresh(hip_ext, layer, dense, x, shape),
          "after the refused call")


def test_noalloc_replays_from_a_graph(hip_ext):
    shape = syn.C2
    layer = syn.build_experts(shape, device=DEV, seed=32)
    dense = syn.build_dense(shape, device=DEV, seed=32)
    x = syn.hidden_states(shape, 4, seed=9).to(DEV)
    outs = [torch.empty_like(x), torch.empty((4, 60), dtype=torch.bfloat16, device=DEV),
            torch.empty((4, 4), dtype=torch.bfloat16, device=DEV), torch.empty((4, 4), dtype=torch.int64, device=DEV)]
    eager = [v.clone() for v in hip_ext.moe_layer_noalloc(layer, dense, x, 4)]
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        hip_ext.moe_layer_noalloc(layer, dense, x, 4, out=outs[0], logits=outs[1], weights=outs[2], indices=outs[3])
    for rep in range(3):
        for o in outs:
            o.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _same(outs, eager, f"graph replay {rep}")
        hip_ext.moe_layer_noalloc(layer, dense, x[:1], 4)  # eager work on the same scratch in between
    del graph
