"""A tiny Qwen2MoE checkpoint on disk for the host-integration tests: the
Transformers config, the dense BF16 tensors in one safetensors shard with the
checkpoint index (which also lists the per-expert tensor names, as a real
Qwen1.5-MoE checkpoint does), and the routed experts as a Q4 ExpertPack. The
fixed model's expert count and top-k (60, 4) are kept; everything else is
small. ``reference_model`` is the same model in Transformers with its experts
set to the pack's dequantized weights: what the host must reproduce."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

from uma_qmoe_amd.formats import decode, quantize_q4
from uma_qmoe_amd.packfile import write_expert_pack
from uma_qmoe_amd.qwen_host import QWEN_MODEL_ID, QWEN_MODEL_REVISION

LAYERS, EXPERTS, TOP_K = 2, 60, 4
ARCH = ("qwen2_moe", LAYERS, EXPERTS, TOP_K)
MANIFEST = "2" * 64
SHARD = "model-00001-of-00001.safetensors"


def config():
    from transformers import Qwen2MoeConfig

    return Qwen2MoeConfig(vocab_size=512, hidden_size=256, intermediate_size=512, moe_intermediate_size=128,
                          shared_expert_intermediate_size=256, num_hidden_layers=LAYERS, num_attention_heads=4,
                          num_key_value_heads=4, num_experts=EXPERTS, num_experts_per_tok=TOP_K,
                          norm_topk_prob=False, max_position_embeddings=256, tie_word_embeddings=False,
                          decoder_sparse_step=1, mlp_only_layers=[], rms_norm_eps=1e-6)


def _random_model(seed: int):
    from transformers import Qwen2MoeForCausalLM

    torch.manual_seed(seed)
    model = Qwen2MoeForCausalLM(config())
    with torch.no_grad():
        for name, p in model.named_parameters():
            if name.endswith("norm.weight") or "layernorm" in name:
                p.copy_(1.0 + 0.1 * torch.randn_like(p))
            else:
                p.copy_(0.05 * torch.randn_like(p))
    return model.to(torch.bfloat16).eval()


def _expert_q4(model):
    """{pack name: Q4Tensor} of every routed expert (gate = first half of
    gate_up_proj, as Qwen2MoeExperts.forward splits it)."""
    out = {}
    for l, layer in enumerate(model.model.layers):
        gu = layer.mlp.experts.gate_up_proj.detach().float()
        down = layer.mlp.experts.down_proj.detach().float()
        inter = gu.shape[1] // 2
        for e in range(EXPERTS):
            for proj, w in (("gate_proj", gu[e, :inter]), ("up_proj", gu[e, inter:]), ("down_proj", down[e])):
                out[f"model.layers.{l}.mlp.experts.{e}.{proj}.weight"] = quantize_q4(w.numpy())
    return out


def write_checkpoint(directory: Path, seed: int = 7):
    """Writes config.json, the dense shard, its index and ``experts.uqep``
    under ``directory``; returns (pack path, the random model)."""
    from safetensors.torch import save_file

    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    model = _random_model(seed)
    model.config.save_pretrained(directory)
    dense = {k: v.contiguous() for k, v in model.state_dict().items() if ".mlp.experts." not in k}
    save_file(dense, str(directory / SHARD))
    q4 = _expert_q4(model)
    weight_map = {name: SHARD for name in dense}
    weight_map.update({name: SHARD for name in q4})
    (directory / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))
    pack = directory / "experts.uqep"
    write_expert_pack(pack, sorted(q4.items()), model_id=QWEN_MODEL_ID, model_revision=QWEN_MODEL_REVISION,
                      model_manifest_sha256=MANIFEST)
    return pack, model, q4


def reference_model(model, q4):
    """The random model with every routed expert replaced by its dequantized
    Q4 weights (BF16, as Transformers holds them)."""
    import copy

    ref = copy.deepcopy(model)
    with torch.no_grad():
        for l, layer in enumerate(ref.model.layers):
            gu = layer.mlp.experts.gate_up_proj
            inter = gu.shape[1] // 2
            for e in range(EXPERTS):
                def deq(proj):
                    t = q4[f"model.layers.{l}.mlp.experts.{e}.{proj}.weight"]
                    return torch.from_numpy(np.asarray(
                        decode_q4(t), dtype=np.float32)).to(torch.bfloat16)
                gu[e, :inter] = deq("gate_proj")
                gu[e, inter:] = deq("up_proj")
                layer.mlp.experts.down_proj[e] = deq("down_proj")
    return ref


def decode_q4(t):
    from uma_qmoe_amd.formats import TargetTensor

    return decode(TargetTensor(tuple(t.shape), "q4_group128", t.packed, t.scales, t.group_size))


def prompt(n: int, seed: int = 3):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, config().vocab_size, (1, n), generator=g)
