"""Qwen1.5-MoE host over the HIP MoE operator, with HIP-graph decode.

Follows the reference's fixed-Qwen host (src/uma_qmoe/qwen_compressed_loader.py:45-299):
``load_fixed_qwen`` builds the Transformers Qwen2MoE model on the meta device,
replaces every layer's MoE block with ``QuantizedQwenMoEBlock`` bound to one
registered expert pack, loads only the dense BF16 tensors from the
checkpoint's safetensors shards (the per-expert tensors are skipped: the pack
holds them), and never holds a BF16 expert parameter. ``DecodeGraph`` captures
one greedy decode step of the whole model over a static KV cache in a HIP graph
(embedding, attention, the library's MoE blocks, head, argmax, and the advance
of the token and position buffers), so that a replay is one token with no host
work in between (the reference's TPOT runner,
benchmarks/runners/run_compressed_qwen_baseline.py, decodes eagerly).
"""

from __future__ import annotations

import itertools
import json
import re
from dataclasses import dataclass
from pathlib import Path
from typing import Any, Iterator, Mapping

from .formats import ENCODINGS, ContractError

QWEN_MODEL_ID = "Qwen/Qwen1.5-MoE-A2.7B"
QWEN_MODEL_REVISION = "1a758c50ecb6350748b9ce0a99d2352fd9fc11c9"  # fixed_models.py:44-55
# (model_type, layers, routed experts, top-k) of the fixed Qwen model
QWEN_ARCHITECTURE = ("qwen2_moe", 24, 60, 4)

_EXPERT_WEIGHT = re.compile(r"^model\.layers\.\d+\.mlp\.experts\.\d+\.(?:down_proj|gate_proj|up_proj)\.weight$")
_TARGET_MAGIC = b"UQMOTPK1"


def is_qwen_expert_tensor_name(name: str) -> bool:
    """True for the per-expert checkpoint tensors the pack replaces
    (qwen_compressed_loader.py:32-35,96-97)."""
    return _EXPERT_WEIGHT.fullmatch(name) is not None


def _torch():
    import torch

    return torch


def _block_class():
    torch = _torch()

    class QuantizedQwenMoEBlock(torch.nn.Module):
        """Qwen router, shared expert and shared-expert gate plus the packed
        routed experts of one layer (qwen_compressed_loader.py:45-86).

        With ``fused_block`` (the default) the whole block runs as one
        ``uma_qmoe::moe_block`` op: router, top-k, routed experts, shared expert
        and its sigmoid gate in the library (one kernel launch per token at one
        or two tokens). Without it the block has the reference's structure: the
        shared expert and the router in torch around ``qwen_moe_forward``."""

        def __init__(self, gate: Any, shared_expert: Any, shared_expert_gate: Any, *, layer_index: int,
                     pack_handle: int, performance_mode: bool, fused_block: bool = True) -> None:
            super().__init__()
            self.gate = gate
            self.shared_expert = shared_expert
            self.shared_expert_gate = shared_expert_gate
            self.layer_index = layer_index
            self.pack_handle = pack_handle
            self.performance_mode = performance_mode
            self.fused_block = fused_block

        def forward(self, hidden_states: Any) -> Any:
            batch_size, sequence_length, hidden_size = hidden_states.shape
            flattened = hidden_states.reshape(-1, hidden_size)
            if self.fused_block:
                shared = self.shared_expert
                out = torch.ops.uma_qmoe.moe_block(
                    flattened, self.gate.weight, shared.gate_proj.weight, shared.up_proj.weight,
                    shared.down_proj.weight, self.shared_expert_gate.weight, int(self.gate.top_k),
                    bool(self.gate.norm_topk_prob), self.layer_index, self.pack_handle, self.performance_mode)[0]
            else:
                shared_output = self.shared_expert(flattened)
                _logits, routing_weights, selected_experts = self.gate(flattened)
                out = torch.ops.uma_qmoe.qwen_moe_forward(flattened, selected_experts, routing_weights,
                                                          self.layer_index, self.pack_handle, self.performance_mode)
                out.add_(torch.sigmoid(self.shared_expert_gate(flattened)) * shared_output)
            return out.reshape(batch_size, sequence_length, hidden_size)

    return QuantizedQwenMoEBlock


_BLOCK = None


def quantized_block(*args: Any, **kwargs: Any) -> Any:
    """A ``QuantizedQwenMoEBlock`` (the class is built on first use, so that
    importing this module does not import torch)."""
    global _BLOCK
    if _BLOCK is None:
        _BLOCK = _block_class()
    return _BLOCK(*args, **kwargs)


def replace_moe_blocks(model: Any, pack_handle: int, *, performance_mode: bool, fused_block: bool = True) -> int:
    """Swaps every layer's MoE block for a QuantizedQwenMoEBlock over the
    pack; returns the number replaced."""
    n = 0
    for layer_index, layer in enumerate(model.model.layers):
        original = layer.mlp
        layer.mlp = quantized_block(original.gate, original.shared_expert, original.shared_expert_gate,
                                    layer_index=layer_index, pack_handle=pack_handle,
                                    performance_mode=performance_mode, fused_block=fused_block)
        n += 1
    return n


def restore_nonpersistent_buffers(model: Any, config: Any, device: Any) -> None:
    """Rebuilds the rotary embedding, whose frequencies are not in the
    state dict and so are uninitialised after ``to_empty``
    (compressed_loader.py:136-166)."""
    torch = _torch()
    rotary = model.model.rotary_emb
    model.model.rotary_emb = type(rotary)(config=config).to(device=device)
    persistent = set(model.state_dict())
    nonpersistent = {name: b for name, b in model.named_buffers() if name not in persistent}
    if any(b.is_meta or not bool(torch.isfinite(b).all()) for b in nonpersistent.values()):
        raise ContractError("fixed Qwen non-persistent buffers are not initialized")


@dataclass(frozen=True)
class QwenCheckpointIndex:
    """What a Qwen checkpoint directory's safetensors index says about the
    tensors a compressed host needs.

    ``dense`` maps every tensor the host model materialises (its state dict)
    to the shard that holds it; ``experts`` are the per-expert tensors the
    index lists and the pack replaces. ``read`` refuses an index whose dense
    set is not exactly the model's (qwen_compressed_loader.py:99-122 keeps
    the same refusal and message)."""

    root: Path
    dense: Mapping[str, str]
    experts: frozenset

    @classmethod
    def read(cls, root: Path, wanted: set[str]) -> "QwenCheckpointIndex":
        try:
            entries = json.loads((root / "model.safetensors.index.json").read_text(encoding="utf-8"))["weight_map"]
        except (OSError, json.JSONDecodeError, KeyError, TypeError) as exc:
            raise ContractError("cannot load fixed Qwen Safetensors index") from exc
        if not isinstance(entries, dict):
            raise ContractError("fixed Qwen weight_map must be an object")
        if not all(isinstance(k, str) and isinstance(v, str) and v for k, v in entries.items()):
            raise ContractError("fixed Qwen weight_map entries must be strings")
        experts = frozenset(filter(is_qwen_expert_tensor_name, entries))
        dense = {name: shard for name, shard in entries.items() if name not in experts}
        if dense.keys() != wanted:
            missing, unexpected = sorted(wanted - dense.keys()), sorted(dense.keys() - wanted)
            raise ContractError(f"fixed Qwen dense checkpoint set mismatch: missing={missing[:8]!r}, "
                                f"unexpected={unexpected[:8]!r}")
        return cls(root, dense, experts)

    def tensors(self) -> Iterator[tuple[str, Any]]:
        """(name, CPU tensor) of every dense tensor, one shard open at a time,
        shards and names in sorted order."""
        from safetensors import safe_open

        by_shard: dict[str, list[str]] = {}
        for name in sorted(self.dense):
            by_shard.setdefault(self.dense[name], []).append(name)
        for shard in sorted(by_shard):
            with safe_open(self.root / shard, framework="pt", device="cpu") as source:
                for name in by_shard[shard]:
                    yield name, source.get_tensor(name)


def expected_expert_tensors(layers: int, experts: int, hidden: int, intermediate: int) -> dict[str, tuple[int, int]]:
    """{name: shape} of the routed-expert tensors of a Qwen MoE model: gate and
    up [intermediate, hidden], down [hidden, intermediate] per layer and expert
    (the set target_pack.py:738-775 requires of the fixed model, 24 x 60 x 3)."""
    shapes = {"gate_proj": (intermediate, hidden), "up_proj": (intermediate, hidden), "down_proj": (hidden, intermediate)}
    return {f"model.layers.{l}.mlp.experts.{e}.{p}.weight": s
            for l in range(layers) for e in range(experts) for p, s in shapes.items()}


def _tensor_table(reader: Any) -> dict[str, tuple[tuple[int, ...], str]]:
    """{name: (shape, encoding)} of every tensor of a TargetPack reader (its
    header's table; an in-memory pack has none and is asked per tensor)."""
    entries = reader.header.get("tensors")
    if entries is None:
        return {n: (tuple(t.shape), t.encoding) for n in reader.names() for t in (reader.tensor(n),)}
    return {t["name"]: (tuple(t["shape"]), t["encoding"]) for t in entries}


def require_complete_target_pack(reader: Any, *, layers: int, experts: int, hidden: int, intermediate: int) -> None:
    """Refuses a TargetPack that does not hold exactly the model's routed
    experts at their shapes, or whose per-encoding tensor counts disagree
    with its layer policy (TargetPackReader.validate_fixed_qwen_complete,
    target_pack.py:738-775, with the fixed model's sizes as arguments and
    the same messages)."""
    want = expected_expert_tensors(layers, experts, hidden, intermediate)
    table = _tensor_table(reader)
    have = {name: shape for name, (shape, _enc) in table.items()}
    if have != want:
        missing, unexpected = sorted(want.keys() - have.keys()), sorted(have.keys() - want.keys())
        wrong = sorted(n for n in want.keys() & have.keys() if want[n] != have[n])
        raise ContractError(f"TargetPack fixed Qwen tensor set mismatch: missing={missing[:8]!r}, "
                            f"unexpected={unexpected[:8]!r}, wrong_shape={wrong[:8]!r}")
    per_layer = [reader.layer_encoding(l) for l in range(layers)]
    policy = {enc: 3 * experts * per_layer.count(enc) for enc in sorted(ENCODINGS)}
    stored = {enc: sum(e == enc for _shape, e in table.values()) for enc in sorted(ENCODINGS)}
    declared = reader.header.get("encoding_tensor_counts", stored)
    if not policy == stored == declared:
        raise ContractError("TargetPack fixed Qwen policy counts are inconsistent")


def pack_vma_count(path: Path | None) -> int:
    """Memory mappings of ``path`` in this process (/proc/self/maps); -1 when
    that cannot be read or the pack has no file (compressed_loader.py:125-133)."""
    if path is None:
        return -1
    target = str(Path(path).resolve())
    try:
        maps = Path("/proc/self/maps").read_text(encoding="utf-8")
    except OSError:
        return -1
    return sum(line.endswith(target) or f"{target} " in line for line in maps.splitlines())


class FixedQwenHost:
    """A loaded host model, the pack its MoE blocks read and the pack's
    operator handle. ``close`` (or leaving the ``with`` block) unregisters
    the handle — waiting for calls in flight — and closes the pack; a second
    close does nothing."""

    def __init__(self, model: Any, expert_pack: Any, pack_handle: int, evidence: dict[str, Any]) -> None:
        self.model = model
        self.expert_pack = expert_pack
        self.pack_handle = pack_handle
        self.evidence = evidence
        self._open = True

    def close(self) -> None:
        from .custom_op import unregister_expert_pack

        if self._open:
            self._open = False
            unregister_expert_pack(self.pack_handle)
            self.expert_pack.close()

    def __enter__(self) -> "FixedQwenHost":
        return self

    def __exit__(self, *_exc: Any) -> None:
        self.close()


def _open_pack(expert_pack: Any, model_id: str, model_revision: str, manifest: str,
               policy: str | None) -> tuple[Any, Path | None]:
    """The pack reader (opened here from a path, else the reader given) and
    the file it maps, if known. A TargetPack needs the policy id, an
    ExpertPack refuses one (qwen_compressed_loader.py:170-195 messages)."""
    from .packfile import ExpertPackReader, TargetPackReader

    if not isinstance(expert_pack, (str, Path)):
        return expert_pack, getattr(expert_pack, "path", None)
    path = Path(expert_pack)
    try:
        with path.open("rb") as f:
            is_target = f.read(8) == _TARGET_MAGIC
    except OSError as exc:
        raise ContractError(f"cannot read compressed Qwen pack {path}: {exc}") from exc
    expected = dict(expected_model_id=model_id, expected_model_revision=model_revision,
                    expected_model_manifest_sha256=manifest)
    if is_target and not policy:
        raise ContractError("Qwen TargetPack loading requires a policy id")
    if not is_target and policy is not None:
        raise ContractError("Qwen ExpertPack cannot satisfy a TargetPack policy id")
    reader = TargetPackReader(path, expected_policy_id=policy, **expected) if is_target else ExpertPackReader(
        path, **expected)
    return reader, path


def _host_model(config: Any, pack_handle: int, device: Any, *, performance_mode: bool, fused_block: bool) -> Any:
    """The Transformers model built on the meta device with every MoE block
    swapped for the quantized block, then materialised (uninitialised) on
    ``device`` with its non-persistent buffers rebuilt. No expert parameter
    is ever allocated."""
    torch = _torch()
    from transformers import AutoModelForCausalLM

    with torch.device("meta"):
        model = AutoModelForCausalLM.from_config(config, dtype=torch.bfloat16, trust_remote_code=False)
    replace_moe_blocks(model, pack_handle, performance_mode=performance_mode, fused_block=fused_block)
    model.to_empty(device=device)
    restore_nonpersistent_buffers(model, config, device)
    return model


def _fill_dense(model: Any, index: QwenCheckpointIndex, device: Any) -> tuple[int, int]:
    """Copies every dense checkpoint tensor into the model (BF16, the
    destination's shape); returns (tensor count, bytes)."""
    torch = _torch()
    slots = model.state_dict(keep_vars=True)
    count = nbytes = 0
    with torch.no_grad():
        for name, value in index.tensors():
            if value.dtype != torch.bfloat16:
                raise ContractError(f"dense tensor {name!r} is not BF16")
            slot = slots[name]
            if slot.shape != value.shape:
                raise ContractError(f"dense tensor {name!r} shape mismatch")
            slot.copy_(value.to(device=device))
            count += 1
            nbytes += value.numel() * value.element_size()
    if count != len(slots):
        raise ContractError("not every Qwen dense checkpoint tensor was loaded")
    return count, nbytes


def load_fixed_qwen(model_directory: str | Path, expert_pack: Any, *, model_manifest_sha256: str,
                    device: str = "cuda:0", performance_mode: bool = False, target_policy_id: str | None = None,
                    fused_block: bool = True, architecture: tuple = QWEN_ARCHITECTURE,
                    model_id: str = QWEN_MODEL_ID, model_revision: str = QWEN_MODEL_REVISION) -> FixedQwenHost:
    """A Qwen MoE host: the dense BF16 tensors of a local checkpoint directory
    in a Transformers model whose MoE blocks run the HIP operator over one
    expert pack (the fixed-model loader of qwen_compressed_loader.py:143-299,
    with the same refusals and evidence keys). ``expert_pack`` is a pack file
    or an open reader; ``architecture`` is the (model_type, layers, experts,
    top-k) the checkpoint must have, the fixed model's by default.

    The pack is checked before anything is built: one mapping (one VMA when
    its file is known) and, for a TargetPack, exactly the model's routed
    experts. The model's layout is then fixed by the config, the dense
    tensors are streamed shard by shard, and the result is checked: every
    block replaced, every dense tensor loaded, the index's expert tensors
    all skipped, no expert or meta tensor left."""
    torch = _torch()
    from transformers import AutoConfig

    from .custom_op import register_expert_pack, register_moe_forward, unregister_expert_pack
    from .packfile import MemoryTargetPack, TargetPackReader

    root = Path(model_directory)
    config = AutoConfig.from_pretrained(root, local_files_only=True, trust_remote_code=False)
    arch = tuple(getattr(config, f, None) for f in ("model_type", "num_hidden_layers", "num_experts",
                                                     "num_experts_per_tok"))
    if arch != tuple(architecture):
        raise ContractError(f"unexpected fixed Qwen architecture {arch!r}")
    _model_type, layers, experts, _top_k = arch
    reader, pack_path = _open_pack(expert_pack, model_id, model_revision, model_manifest_sha256, target_policy_id)
    opened_here = isinstance(expert_pack, (str, Path))
    try:
        if getattr(reader, "mapping_count", None) != 1:
            raise ContractError("compressed Qwen host mapped ExpertPack more than once")
        vmas = pack_vma_count(pack_path)
        if vmas not in (1, -1):
            raise ContractError("compressed Qwen host observed multiple ExpertPack VMAs")
        if isinstance(reader, (TargetPackReader, MemoryTargetPack)):
            require_complete_target_pack(reader, layers=layers, experts=experts, hidden=config.hidden_size,
                                         intermediate=config.moe_intermediate_size)
    except BaseException:
        if opened_here:
            reader.close()
        raise
    register_moe_forward()
    handle = register_expert_pack(reader)
    try:
        model = _host_model(config, handle, device, performance_mode=performance_mode, fused_block=fused_block)
        index = QwenCheckpointIndex.read(root, set(model.state_dict()))
        dense_count, dense_bytes = _fill_dense(model, index, device)
        blocks = sum(isinstance(layer.mlp, _BLOCK) for layer in model.model.layers)
        expert_params = [n for n, _ in model.named_parameters() if ".mlp.experts." in n]
        failures = [
            (blocks != layers, "compressed Qwen host did not replace every MoE block"),
            (len(index.experts) != layers * experts * 3,
             f"expected to skip {layers * experts * 3} Qwen expert tensors, skipped {len(index.experts)}"),
            (bool(expert_params), "compressed Qwen host still contains expert Parameters"),
            (any(t.is_meta for t in itertools.chain(model.parameters(), model.buffers())),
             "compressed Qwen host contains meta tensors"),
        ]
        for failed, message in failures:
            if failed:
                raise ContractError(message)
        model.eval()
        evidence = {
            "model_id": model_id,
            "model_revision": model_revision,
            "device": str(device),
            "performance_mode": performance_mode,
            "fused_block": fused_block,
            "dense_tensor_count": dense_count,
            "dense_tensor_bytes": dense_bytes,
            "skipped_expert_tensor_count": len(index.experts),
            "loaded_expert_tensor_count": 0,
            "expert_parameter_count": len(expert_params),
            "quantized_moe_block_count": blocks,
            "model_parameter_bytes": sum(p.numel() * p.element_size() for p in model.parameters()),
            "expert_pack_mapping_count": reader.mapping_count,
            "expert_pack_vma_count": vmas,
        }
        if pack_path is not None:
            evidence["expert_pack_size_bytes"] = Path(pack_path).stat().st_size
        if str(device).startswith("cuda"):
            evidence["torch_allocated_bytes"] = int(torch.cuda.memory_allocated(device))
            evidence["torch_reserved_bytes"] = int(torch.cuda.memory_reserved(device))
        return FixedQwenHost(model, reader, handle, evidence)
    except BaseException:
        unregister_expert_pack(handle)
        if opened_here:
            reader.close()
        raise


class DecodeGraph:
    """Greedy decode of a (host) Qwen2MoE model with one HIP graph per token.

    ``prefill`` runs the prompt eagerly into a static KV cache of
    ``max_len`` positions and primes the token and position buffers;
    ``capture`` records one decode step — the model on the current token at
    the current position, the argmax of the last logits written back into the
    token buffer, the position advanced — so every ``replay`` produces the
    next token with no host work. ``logits`` holds the last step's logits
    (fp32 [vocab]) and ``token`` the token it chose."""

    def __init__(self, model: Any, *, max_len: int) -> None:
        torch = _torch()
        from transformers import StaticCache

        self.model = model
        self.device = next(model.parameters()).device
        self.max_len = int(max_len)
        self.cache = StaticCache(config=model.config, max_cache_len=self.max_len)
        self.token = torch.zeros((1, 1), dtype=torch.long, device=self.device)
        self.position = torch.zeros((1,), dtype=torch.long, device=self.device)
        self.next_position = 0  # host copy of ``position`` (no sync per token)
        self.logits = None
        self.graph = None
        # the stream the warm-up and the capture run on: the library's
        # per-stream workspace is then allocated (and zero-filled) by the
        # warm-up, outside the graph
        self.stream = torch.cuda.Stream(device=self.device)

    def _forward(self, input_ids: Any, cache_position: Any) -> Any:
        out = self.model(input_ids=input_ids, past_key_values=self.cache, cache_position=cache_position,
                         use_cache=True)
        return out.logits[0, -1].float()

    def prefill(self, prompt_ids: Any) -> Any:
        """Runs the prompt ([1, n] token ids on the device) and returns the
        first generated token (the prompt's greedy continuation)."""
        torch = _torch()
        n = int(prompt_ids.shape[1])
        if n < 1 or n >= self.max_len:
            raise ContractError("prompt must be non-empty and shorter than the cache")
        with torch.no_grad():
            logits = self._forward(prompt_ids, torch.arange(n, device=self.device))
            self.token.copy_(logits.argmax().view(1, 1))
            self.position.fill_(n)
        self.next_position = n
        self.logits = logits
        return self.token.clone()

    def _step(self) -> Any:
        logits = self._forward(self.token, self.position)
        self.token.copy_(logits.argmax().view(1, 1))
        self.position.add_(1)
        return logits

    def step_eager(self) -> Any:
        """One decode step without the graph (the same operations)."""
        torch = _torch()
        if self.next_position >= self.max_len:
            raise ContractError("the static cache is full")
        with torch.no_grad():
            self.logits = self._step()
        self.next_position += 1
        return self.token.clone()

    def _counters(self) -> list[Any]:
        """The device-side state a step advances: the token and position
        buffers and each cache layer's fill counter (Transformers' StaticLayer
        writes new keys at its own ``cumulative_length``, not at
        ``cache_position``)."""
        torch = _torch()
        counters = [self.token, self.position]
        for layer in getattr(self.cache, "layers", ()):
            c = getattr(layer, "cumulative_length", None)
            if torch.is_tensor(c):
                counters.append(c)
        return counters

    def capture(self) -> None:
        """Records one decode step. The cache, token and position buffers
        must be those of a prefilled sequence with at least two free positions
        (the warm-up step on a side stream writes the next position; the
        token, position and cache fill counters are put back afterwards)."""
        torch = _torch()
        if self.next_position + 2 > self.max_len:
            raise ContractError("no room in the cache to capture a decode step")
        counters = self._counters()
        saved = [c.clone() for c in counters]
        self.stream.wait_stream(torch.cuda.current_stream())
        with torch.no_grad(), torch.cuda.stream(self.stream):
            self._step()
            if [c.data_ptr() for c in self._counters()] != [c.data_ptr() for c in counters]:
                raise ContractError("the decode step replaced a cache counter instead of advancing it in place")
            for c, v in zip(counters, saved):
                c.copy_(v)
        torch.cuda.current_stream().wait_stream(self.stream)
        graph = torch.cuda.CUDAGraph()
        with torch.no_grad(), torch.cuda.graph(graph, stream=self.stream):
            self.logits = self._step()
        # capture ran nothing: the buffers still hold the prefilled state
        self.graph = graph

    def replay(self) -> Any:
        """One token: returns the token buffer (device, [1, 1]) after the step."""
        if self.graph is None:
            raise ContractError("capture() a decode step first")
        if self.next_position >= self.max_len:
            raise ContractError("the static cache is full")
        self.graph.replay()
        self.next_position += 1
        return self.token


__all__ = [
    "DecodeGraph",
    "FixedQwenHost",
    "QWEN_ARCHITECTURE",
    "QWEN_MODEL_ID",
    "QWEN_MODEL_REVISION",
    "is_qwen_expert_tensor_name",
    "load_fixed_qwen",
    "quantized_block",
    "replace_moe_blocks",
    "restore_nonpersistent_buffers",
]
