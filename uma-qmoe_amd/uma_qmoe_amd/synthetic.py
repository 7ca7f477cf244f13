"""Seeded synthetic MoE layers for the benchmark configurations.

Weights are drawn N(0, 0.02) in float32 and encoded with the canonical codecs
(Q4 [-7, 7] absmax/7, Q8 absmax/127, BF16 round-to-nearest-even); router
weights are BF16 N(0, 0.02); hidden states are BF16 N(0, 1). Every tensor has
its own generator seeded from (seed, layer, name), so a layer can be rebuilt
bit-identically on any device from the same seed.

Configurations (shapes of the fixed models: src/uma_qmoe/fixed_models.py:32-55):
  c1  OLMoE layer, H 2048, E 64, k 8, I 1024, no shared expert, Q4, 1 token
  c2  Qwen1.5-MoE layer, H 2048, E 60, k 4, I 1408, shared 5632 BF16, Q4, 1 token
  c3  24-layer Qwen stack: routed BF16 in layers 0-15, Q8 in 16-23
  c4  c2 shapes at 512 tokens (and 32)
  c5  H 2048, E 128, k 8, I 768, no shared expert, Q4, 256 tokens, router
      logits biased so expert popularity follows Zipf(s=1.1)
"""

from __future__ import annotations

from dataclasses import dataclass, field, replace
import hashlib
from typing import Any

from .native_backend import EXPERT_NAME, DenseBlock, DeviceExperts
from .formats import TargetTensor, encode_projection

SEED = 20260920
WEIGHT_STD = 0.02


@dataclass(frozen=True)
class MoEShape:
    name: str
    hidden: int
    num_experts: int
    top_k: int
    intermediate: int
    shared_intermediate: int = 0
    encoding: str = "q4_group128"
    tokens: int = 1
    norm_topk_prob: bool = False
    zipf_s: float | None = None
    group_size: int = 128

    @property
    def has_shared(self) -> bool:
        return self.shared_intermediate > 0


C1 = MoEShape("c1_olmoe_w4a16", 2048, 64, 8, 1024)
C2 = MoEShape("c2_qwen_w4a16", 2048, 60, 4, 1408, 5632)
C4 = replace(C2, name="c4_qwen_w4a16_prefill", tokens=512)
C5 = MoEShape("c5_finegrained_w4a16_zipf", 2048, 128, 8, 768, tokens=256, zipf_s=1.1)
C3_LAYERS = 24
C3_STEPS = 32


def c3_layer_shape(layer: int) -> MoEShape:
    return replace(C2, name=f"c3_qwen_stack_l{layer}", encoding="bf16_le" if layer < 16 else "q8_group128")


CONFIGS = {"c1": C1, "c2": C2, "c4": C4, "c5": C5}


def _seed(seed: int, *parts: Any) -> int:
    h = hashlib.sha256(repr((seed, *parts)).encode()).digest()
    return int.from_bytes(h[:8], "little") & ((1 << 63) - 1)


def _generator(device: Any, seed: int):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def normal(shape, *, seed: int, std: float = WEIGHT_STD, device: Any = "cpu"):
    import torch

    return torch.randn(shape, generator=_generator(device, seed), device=device, dtype=torch.float32) * std


def hidden_states(shape: MoEShape, tokens: int | None = None, *, seed: int = SEED, device: Any = "cpu", tag: str = "x"):
    import torch

    t = shape.tokens if tokens is None else tokens
    return normal((t, shape.hidden), seed=_seed(seed, shape.name, tag), std=1.0, device=device).to(torch.bfloat16)


def build_experts(shape: MoEShape, *, layer: int = 0, seed: int = SEED, device: Any = "cpu",
                  chunk: int = 8) -> DeviceExperts:
    """All routed experts of one layer, encoded, expert-major, on ``device``.

    Experts are generated ``chunk`` at a time (generator per expert), which
    bounds the float32 staging memory.
    """
    import torch

    out = {}
    dims = {"gate_proj": (shape.intermediate, shape.hidden), "up_proj": (shape.intermediate, shape.hidden),
            "down_proj": (shape.hidden, shape.intermediate)}
    for proj, (rows, cols) in dims.items():
        datas, scales = [], []
        for e0 in range(0, shape.num_experts, chunk):
            ws = [normal((rows, cols), seed=_seed(seed, shape.name, layer, e, proj), device=device)
                  for e in range(e0, min(shape.num_experts, e0 + chunk))]
            d, s = encode_projection(torch.stack(ws), shape.encoding, shape.group_size)
            datas.append(d)
            if s is not None:
                scales.append(s)
            del ws
        out[proj] = (torch.cat(datas), torch.cat(scales) if scales else None)
    return DeviceExperts(shape.encoding, shape.group_size, shape.num_experts, shape.hidden, shape.intermediate,
                         out["gate_proj"][0], out["gate_proj"][1], out["up_proj"][0], out["up_proj"][1],
                         out["down_proj"][0], out["down_proj"][1])


def build_dense(shape: MoEShape, *, layer: int = 0, seed: int = SEED, device: Any = "cpu") -> DenseBlock:
    import torch

    def bf(rows, cols, tag):
        return normal((rows, cols), seed=_seed(seed, shape.name, layer, tag), device=device).to(torch.bfloat16)

    router = bf(shape.num_experts, shape.hidden, "router")
    if not shape.has_shared:
        return DenseBlock(router)
    i = shape.shared_intermediate
    return DenseBlock(router, bf(i, shape.hidden, "shared_gate"), bf(i, shape.hidden, "shared_up"),
                      bf(shape.hidden, i, "shared_down"), bf(1, shape.hidden, "shared_expert_gate"))


def zipf_router_bias(shape: MoEShape, scale: float = 1.0, *, seed: int = SEED, device: Any = "cpu"):
    """Per-expert logit bias b_e = scale * log(rank_e ** -s) over a seeded
    random ranking of the experts (float32 [E])."""
    import torch

    ranks = torch.randperm(shape.num_experts, generator=_generator("cpu", _seed(seed, shape.name, "zipf"))) + 1
    bias = scale * (-(shape.zipf_s or 1.0)) * torch.log(ranks.to(torch.float32))
    return bias.to(device)


def algorithmic_bytes(experts: DeviceExperts, dense: DenseBlock | None, distinct_experts: int) -> int:
    """Weight bytes one layer call must read: each distinct routed expert once,
    plus router and shared expert (activations are < 0.1% and not counted)."""
    total = experts.bytes_per_expert() * distinct_experts
    if dense is not None:
        for t in (dense.router, dense.shared_gate, dense.shared_up, dense.shared_down, dense.shared_expert_gate):
            if t is not None:
                total += t.numel() * t.element_size()
    return total


@dataclass
class DeviceLayerReader:
    """Pack-reader view (``tensor_views``/``layer_encoding``) over staged device
    tensors, copying one expert matrix to the host on demand. Lets the
    operator boundary and checkers read a synthetic layer without a file."""

    layers: dict[int, DeviceExperts]
    model: dict[str, Any] = field(default_factory=dict)
    mapping_count: int = 1

    @property
    def header(self) -> dict[str, Any]:
        return {"quantization": {"group_size": 128}, "model": dict(self.model)}

    def layer_encoding(self, layer_index: int) -> str:
        return self.layers[int(layer_index)].encoding

    def tensor_views(self, name: str):
        import re

        import numpy as np
        import torch

        m = re.fullmatch(r"model\.layers\.(\d+)\.mlp\.experts\.(\d+)\.(gate_proj|up_proj|down_proj)\.weight", name)
        if m is None or int(m.group(1)) not in self.layers:
            raise KeyError(name)
        layer = self.layers[int(m.group(1))]
        e = int(m.group(2))
        if e >= layer.num_experts:
            raise KeyError(name)
        proj = m.group(3)
        data = {"gate_proj": layer.gate, "up_proj": layer.up, "down_proj": layer.down}[proj][e]
        scales = {"gate_proj": layer.gate_scales, "up_proj": layer.up_scales, "down_proj": layer.down_scales}[proj]
        shape = [layer.intermediate_size, layer.hidden_size] if proj != "down_proj" else [layer.hidden_size, layer.intermediate_size]
        d = data.detach().cpu()
        if d.dtype == torch.bfloat16:
            d = d.view(torch.int16)
        raw = memoryview(np.ascontiguousarray(d.numpy()).reshape(-1).view(np.uint8))
        sc = memoryview(np.ascontiguousarray(scales[e].detach().cpu().numpy()).view(np.uint8)) if scales is not None else memoryview(b"")
        meta = {"shape": shape, "encoding": layer.encoding, "group_size": layer.group_size if layer.encoding != "bf16_le" else None}
        return raw, sc, meta

    def close(self) -> None:
        pass


def pack_tensors(layers: dict[int, DeviceExperts]):
    """(name, TargetTensor) of every routed-expert matrix of staged layers, in
    the order the pack writers store them (layer, expert, gate/up/down): the
    bytes of the synthetic layers as a pack would hold them."""
    reader = DeviceLayerReader(layers)
    for index in sorted(layers):
        for name in expert_names(index, layers[index].num_experts):
            data, scales, meta = reader.tensor_views(name)
            yield name, TargetTensor(tuple(meta["shape"]), meta["encoding"], bytes(data), bytes(scales),
                                     meta["group_size"])


def expert_names(layer: int, num_experts: int):
    for e in range(num_experts):
        for proj in ("gate_proj", "up_proj", "down_proj"):
            yield EXPERT_NAME.format(layer=layer, expert=e, proj=proj)
