"""The reference's measured OLMoE routes (RouteTrace fixture) replayed
through the HIP routed-expert op at c1 shapes, against the oracle on the
same routes: the 128-token prefill event (sampled tokens) and decode events
of three layers; and the whole 32-event x 16-layer replay twice, bit for bit
the same, every output finite."""

from __future__ import annotations

from pathlib import Path

import pytest
import torch

from oracle import moe as om
from test_gpu_kernels import DEV, assert_close, note
from uma_qmoe_amd import synthetic as syn
from uma_qmoe_amd.route_trace import load_arrays, replay

pytestmark = pytest.mark.gpu

FIXTURE = Path(__file__).resolve().parent / "golden" / "route_trace" / "olmoe_1b_7b_0125_128x32_greedy_v1.npz"


@pytest.fixture(scope="module")
def trace_layers():
    arrays = load_arrays(FIXTURE)
    layers = {l: syn.build_experts(syn.C1, layer=l, device=DEV) for l in range(16)}
    return arrays, layers


def _call(hip_ext, layer, ev, x):
    idx = torch.from_numpy(ev.expert_indices).to(DEV)
    w = torch.from_numpy(ev.routing_weights).to(torch.bfloat16).to(DEV)
    return hip_ext.moe_forward(layer, x.to(DEV), idx, w)


@pytest.mark.parametrize("layer_index", [0, 7, 15])
def test_trace_routes_match_oracle(hip_ext, trace_layers, layer_index):
    arrays, layers = trace_layers
    reader = syn.DeviceLayerReader({layer_index: layers[layer_index]})
    events = [e for e in replay(arrays) if e.layer_index == layer_index and e.event_index < 4]
    for ev in events:
        note(f"trace layer {layer_index} event {ev.event_index} ({ev.phase}, {ev.token_count} tokens)")
        x = syn.hidden_states(syn.C1, ev.token_count, seed=ev.event_index, tag="trace_test")
        out = _call(hip_ext, layers[layer_index], ev, x)
        pick = slice(0, ev.token_count) if ev.token_count <= 8 else torch.arange(0, ev.token_count, 16)
        idx = torch.from_numpy(ev.expert_indices)[pick]
        w = torch.from_numpy(ev.routing_weights).to(torch.bfloat16)[pick]
        ref = om.streaming_reference(x[pick], idx, w, layer_index, reader, num_experts=64).to(torch.bfloat16)
        assert_close(out.cpu()[pick], ref, f"trace layer {layer_index} event {ev.event_index}")


def test_whole_trace_replays_deterministically(hip_ext, trace_layers):
    arrays, layers = trace_layers
    first, second = [], []
    for runs in (first, second):
        for ev in replay(arrays):
            x = syn.hidden_states(syn.C1, ev.token_count, seed=ev.event_index, tag="trace_test")
            runs.append(_call(hip_ext, layers[ev.layer_index], ev, x))
        torch.cuda.synchronize()
    assert len(first) == 32 * 16
    for a, b in zip(first, second):
        assert torch.isfinite(a.float()).all()
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
