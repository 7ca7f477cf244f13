"""Qwen host integration on the GPU: the tiny checkpoint of qwen_tiny loaded
with performance_mode=True (every MoE block in the HIP library, fused into one
op or in the reference's structure around qwen_moe_forward) against
Transformers' model with the pack's dequantized experts on the CPU; and greedy
decode replayed from one HIP graph per token against the same steps run
eagerly."""

from __future__ import annotations

import sys

import pytest
import torch

from oracle import moe as om
from qwen_tiny import ARCH, MANIFEST, prompt, reference_model, write_checkpoint
from uma_qmoe_amd.custom_op import REGISTRY
from uma_qmoe_amd.native_backend import install_packed_q4_backend
from uma_qmoe_amd.qwen_host import DecodeGraph, load_fixed_qwen

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def note(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def checkpoint(tmp_path_factory):
    d = tmp_path_factory.mktemp("qwen_tiny_gpu")
    pack, model, q4 = write_checkpoint(d)
    return d, pack, reference_model(model, q4)


@pytest.fixture(autouse=True)
def _backend():
    install_packed_q4_backend()
    yield
    REGISTRY.uninstall("hip_gfx950")


@pytest.mark.parametrize("fused_block", [True, False])
def test_host_on_gpu_matches_transformers(checkpoint, fused_block):
    d, pack, ref = checkpoint
    note(f"qwen host gpu fused_block={fused_block}")
    ids = prompt(6)
    with load_fixed_qwen(d, pack, model_manifest_sha256=MANIFEST, device=DEV, performance_mode=True,
                         architecture=ARCH, fused_block=fused_block) as host:
        with torch.no_grad():
            for n in (6, 1):  # a prompt (multi-token kernels), then one token (fused kernel)
                got = host.model(input_ids=ids[:, :n].to(DEV)).logits.float().cpu()
                want = ref(input_ids=ids[:, :n]).logits.float()
                r = om.rel_l2(got, want)
                print(f"  n={n}: rel_l2={r:.3e}", flush=True)
                assert torch.isfinite(got).all()
                assert r <= 2e-2, f"logits n={n}: rel-L2 {r}"
                assert torch.equal(got[0, -1].argmax(), want[0, -1].argmax())


def test_decode_graph_replays_the_eager_steps(checkpoint):
    """Eager cached steps against the whole sequence run again without a
    cache, and the graph replays against the eager steps."""
    d, pack, _ref = checkpoint
    note("qwen host decode graph")
    ids = prompt(6).to(DEV)
    steps = 8
    with load_fixed_qwen(d, pack, model_manifest_sha256=MANIFEST, device=DEV, performance_mode=True,
                         architecture=ARCH) as host:
        eager = DecodeGraph(host.model, max_len=32)
        first = eager.prefill(ids)
        toks_e, logits_e = [first], []
        seq = torch.cat([ids, first], 1)
        for i in range(steps):
            toks_e.append(eager.step_eager())
            logits_e.append(eager.logits.clone())
            with torch.no_grad():
                full = host.model(input_ids=seq).logits[0, -1].float()
            r = om.rel_l2(logits_e[-1].cpu(), full.cpu())
            assert r <= 2e-2, f"eager step {i} against the uncached sequence: rel-L2 {r}"
            seq = torch.cat([seq, toks_e[-1]], 1)
        graph = DecodeGraph(host.model, max_len=32)
        first_g = graph.prefill(ids)
        assert torch.equal(first_g, first)
        graph.capture()
        toks_g, logits_g = [first_g], []
        for _ in range(steps):
            toks_g.append(graph.replay().clone())
            logits_g.append(graph.logits.clone())
            torch.cuda.synchronize()
        for i in range(steps):
            assert torch.equal(toks_g[i + 1], toks_e[i + 1]), f"token {i}"
            r = om.rel_l2(logits_g[i].cpu(), logits_e[i].cpu())
            assert r <= 1e-3, f"step {i}: rel-L2 {r}"
        assert graph.next_position == 6 + steps
