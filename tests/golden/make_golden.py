"""Writes the golden fixtures under tests/golden/ from the CPU oracle.

Each fixture is one ``<case>.npz`` (numpy, no pickled objects) holding:
  meta      JSON text: shape, seeds, token count, SHA-256 of the encoded
            weights the seeds regenerate (so a changed generator is caught)
  x         bf16 words [T, H] (uint16) — the block input
  logits    bf16 words [T, E] — oracle router logits (CPU F.linear in bf16)
  weights   bf16 words [T, k] — routing weights
  indices   int64 [T, k]      — selected experts (larger logit, then lower id)
  out       bf16 words [T, H] — oracle block output

Weights are not stored: they are regenerated bit-identically on the CPU from
the seeds by uma_qmoe_amd.synthetic and checked against the stored digest.
Run from the repository root:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import hashlib
import json
import sys
from dataclasses import asdict, replace
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for _p in (ROOT, ROOT / "uma-qmoe_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

from oracle import moe as om  # noqa: E402
from uma_qmoe_amd import synthetic as syn  # noqa: E402

SEED = syn.SEED


def _bits(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16).copy()
    return t.numpy().copy()


def weights_digest(layer, dense) -> str:
    h = hashlib.sha256()
    tensors = [layer.gate, layer.gate_scales, layer.up, layer.up_scales, layer.down, layer.down_scales]
    if dense is not None:
        tensors += [dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate]
    for t in tensors:
        if t is not None:
            h.update(_bits(t).tobytes())
    return h.hexdigest()


# name -> (shape, tokens, layer index, rmsnorm input, zipf bias)
CASES = {
    "tiny_q4": (syn.MoEShape("tiny_q4", 256, 8, 2, 128, 128, "q4_group128"), 5, 0, False),
    "tiny_q8": (syn.MoEShape("tiny_q8", 256, 8, 2, 128, 128, "q8_group128"), 5, 0, False),
    "tiny_bf16": (syn.MoEShape("tiny_bf16", 256, 8, 2, 128, 128, "bf16_le"), 5, 0, False),
    "c1_t1": (syn.C1, 1, 0, False),
    "c2_t1": (syn.C2, 1, 0, False),
    "c4_t16": (replace(syn.C4, name=syn.C2.name), 16, 0, False),
    "c5_t8": (syn.C5, 8, 0, False),
    "c3_l0_t1": (syn.c3_layer_shape(0), 1, 0, True),
    "c3_l16_t1": (syn.c3_layer_shape(16), 1, 16, True),
}


def case_inputs(name: str):
    """Regenerates (shape, layer, dense, x, layer_index, bias) of a case on the CPU."""
    shape, tokens, layer_index, norm = CASES[name]
    layer = syn.build_experts(shape, layer=layer_index, seed=SEED)
    dense = syn.build_dense(shape, layer=layer_index, seed=SEED)
    x = syn.hidden_states(shape, tokens, seed=SEED, tag=f"golden_{name}")
    if norm:
        x = om.rmsnorm(x, 1e-6)
    bias = syn.zipf_router_bias(shape, seed=SEED) if shape.zipf_s else None
    return shape, layer, dense, x, layer_index, bias


def oracle_case(shape, layer, dense, x, layer_index, bias):
    lay = {"router": dense.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense.shared_gate, "shared_up": dense.shared_up, "shared_down": dense.shared_down,
           "shared_expert_gate": dense.shared_expert_gate, "norm_topk_prob": shape.norm_topk_prob}
    reader = syn.DeviceLayerReader({layer_index: layer})
    routes = None
    if bias is not None:
        logits = (torch.nn.functional.linear(x, dense.router).float() + bias).to(torch.bfloat16)
        probs = torch.softmax(logits.float(), -1)
        idx = om.topk_ordered(logits, shape.top_k)
        routes = (probs.gather(-1, idx).to(torch.bfloat16), idx)
    out, logits, weights, indices = om.qwen_block(x, lay, reader, layer_index, routes=routes)
    if bias is not None:
        logits = (logits.float() + bias).to(torch.bfloat16)
    return out, logits, weights, indices


def main(names=None) -> None:
    for name in names or CASES:
        shape, layer, dense, x, layer_index, bias = case_inputs(name)
        out, logits, weights, indices = oracle_case(shape, layer, dense, x, layer_index, bias)
        meta = {"case": name, "shape": asdict(shape), "tokens": int(x.shape[0]), "layer_index": layer_index,
                "seed": SEED, "zipf_bias_scale": 1.0 if bias is not None else None,
                "weights_sha256": weights_digest(layer, dense),
                "generator": "uma_qmoe_amd.synthetic (torch CPU generators), oracle.moe.qwen_block"}
        np.savez_compressed(HERE / f"{name}.npz", meta=np.array(json.dumps(meta, sort_keys=True)), x=_bits(x),
                            logits=_bits(logits), weights=_bits(weights), indices=_bits(indices.to(torch.int64)),
                            out=_bits(out))
        print(f"wrote {name}.npz", flush=True)


if __name__ == "__main__":
    main(sys.argv[1:] or None)
