"""Validation run of the packed-Q4 HIP path that writes a
``packed_q4_kernel_evidence`` document.

The steps, gates and document are those of the reference's validator
(benchmarks/runners/validate_packed_q4_kernel.py:95-221), run on MI355X:

  1. three projections of layer 0, expert 0 (gate and up on
     ``linspace(-0.5, 0.5, 2048)`` and ``linspace(0.25, -0.25, 2048)``, down
     on ``linspace(-0.75, 0.75, 1024)``) through the backend's ``q4_linear``,
     against ``F.linear`` on the BF16-dequantised weight;
  2. ``moe_forward`` at one token (``linspace(-0.5, 0.5, 2048)``, experts
     0..7, weight 0.125 each) in performance mode against correctness mode;
  3. the same at 32 tokens (``linspace(-0.5, 0.5, 32 * 2048)``);
  4. timing samples of both performance-mode calls (HIP events);
  5. gates: every agreement within max-abs 1.0 and cosine >= 0.99, the
     platform, the compressed cache with no dequantised cache, all samples
     taken.

Correctness mode is the library's own (``native_backend.CorrectnessPath``:
every expert of the layer dequantised transiently to BF16 by a HIP kernel,
then the BF16 expert kernels), as the reference compares its performance
backend with its transient-dequantisation path. The document's ``target_id``
is "mi355x" and its platform "hip_gfx950" (the two enumerations the schema
widens for this target); everything else keeps the reference's fields.

Usage: ``python -m uma_qmoe_amd.validate_kernel --expert-pack PACK
--model-manifest-sha256 HEX --output PATH [--warmup-iterations 3]
[--measured-iterations 10]``. It refuses to overwrite ``--output``.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import math
from pathlib import Path
from typing import Any, Callable

from . import _native
from .evidence import kernel_evidence, tensor_sha256, validate_kernel_evidence
from .formats import ContractError

MODEL_ID = "allenai/OLMoE-1B-7B-0125"
MODEL_REVISION = "9b0c1aa87e34a20052389dce1f0cf01da783f654"
ABI = f"q4-group128-packed-u8-fp32-scale-bf16-in-bf16-out-uqm-abi{_native.ABI_VERSION}"
EXECUTION_STRATEGY = "decode-fused-persistent-one-launch-prefill-grouped-mfma-stream-k"
ACCEPTANCE = {"max_absolute_error": 1.0, "minimum_cosine_similarity": 0.99}
LAYER, TOP_K, PREFILL_TOKENS = 0, 8, 32


def file_sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with Path(path).open("rb") as f:
        for block in iter(lambda: f.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


def agreement(candidate: Any, reference: Any) -> dict[str, Any]:
    """finite / max-abs / cosine of a candidate against its reference (both
    as float64; a non-finite candidate reports max-abs 1e30 and cosine 0, so
    it fails the gates)."""
    import torch

    c = candidate.detach().double().reshape(-1).cpu()
    r = reference.detach().double().reshape(-1).cpu()
    finite = bool(torch.isfinite(c).all())
    if not finite:
        return {"finite": False, "max_absolute_error": 1e30, "cosine_similarity": 0.0}
    nc, nr = float(c.dot(c)), float(r.dot(r))
    cos = 1.0 if nc == nr == 0.0 else 0.0 if nc == 0.0 or nr == 0.0 else float(c.dot(r)) / math.sqrt(nc * nr)
    return {"finite": True, "max_absolute_error": float((c - r).abs().max()) if c.numel() else 0.0,
            "cosine_similarity": min(1.0, max(-1.0, cos))}


def time_calls(torch: Any, call: Callable[[], Any], warmup: int, measured: int) -> list[float]:
    """Milliseconds of each of ``measured`` calls (HIP events on the current
    stream, one synchronisation per sample) after ``warmup`` calls."""
    for _ in range(warmup):
        call()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    samples = []
    for _ in range(measured):
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record(stream)
        call()
        stop.record(stream)
        stop.synchronize()
        samples.append(float(start.elapsed_time(stop)))
    return samples


def run(expert_pack: Path, *, model_manifest_sha256: str, warmup: int = 3, measured: int = 10,
        target_id: str = "mi355x", model_id: str = MODEL_ID, model_revision: str = MODEL_REVISION) -> dict[str, Any]:
    """Runs the validation on ``cuda:0`` and returns the validated document."""
    import torch
    import torch.nn.functional as F

    from .custom_op import register_expert_pack, register_moe_forward, unregister_expert_pack
    from .formats import decode_target_tensor
    from .native_backend import install_packed_q4_backend, native_kernel_source_sha256
    from .packfile import ExpertPackReader

    if warmup < 1 or measured < 3:
        raise ContractError("packed Q4 timing requires >=1 warmup and >=3 measured samples")
    if not torch.cuda.is_available():
        raise RuntimeError("packed Q4 validation requires a HIP device")
    dev = torch.device("cuda:0")
    register_moe_forward()
    backend = install_packed_q4_backend()
    reader = ExpertPackReader(expert_pack, expected_model_id=model_id, expected_model_revision=model_revision,
                              expected_model_manifest_sha256=model_manifest_sha256)
    handle = register_expert_pack(reader)
    try:
        inputs = {"gate_proj": (-0.5, 0.5), "up_proj": (0.25, -0.25), "down_proj": (-0.75, 0.75)}
        projections = []
        with torch.inference_mode():
            for proj, (lo, hi) in inputs.items():
                name = f"model.layers.{LAYER}.mlp.experts.0.{proj}.weight"
                weight = torch.from_numpy(decode_target_tensor(reader.tensor(name))).to(dev, torch.bfloat16)
                x = torch.linspace(lo, hi, weight.shape[1], dtype=torch.float32).reshape(1, -1).to(dev,
                                                                                                      torch.bfloat16)
                got = backend.q4_linear(x, handle, name)
                result = agreement(got, F.linear(x, weight))
                result.update({"name": proj, "shape": list(weight.shape)})
                projections.append(result)

            hidden_size = int(projections[0]["shape"][1])

            def routed(tokens: int):
                x = torch.linspace(-0.5, 0.5, tokens * hidden_size, dtype=torch.float32, device=dev)
                x = x.reshape(tokens, hidden_size).to(torch.bfloat16)
                experts = torch.arange(TOP_K, dtype=torch.int64, device=dev).repeat(tokens, 1)
                weights = torch.full((tokens, TOP_K), 0.125, dtype=torch.bfloat16, device=dev)
                return x, experts, weights

            def compare(tokens: int) -> dict[str, Any]:
                x, experts, weights = routed(tokens)
                slow = torch.ops.uma_qmoe.moe_forward(x, experts, weights, LAYER, handle, False)
                fast = torch.ops.uma_qmoe.moe_forward(x, experts, weights, LAYER, handle, True)
                torch.cuda.synchronize()
                result = agreement(fast, slow)
                result["output_sha256"] = tensor_sha256(fast)
                return result

            decode, prefill = compare(1), compare(PREFILL_TOKENS)
            args1, args32 = routed(1), routed(PREFILL_TOKENS)
            samples = time_calls(torch, lambda: torch.ops.uma_qmoe.moe_forward(*args1, LAYER, handle, True),
                                 warmup, measured)
            prefill_samples = time_calls(
                torch, lambda: torch.ops.uma_qmoe.moe_forward(*args32, LAYER, handle, True), warmup, measured)
        cache = backend.cache_summary()
        doc = kernel_evidence(
            target_id=target_id, platform=backend.platform, device_name=torch.cuda.get_device_name(dev),
            source_sha256=native_kernel_source_sha256(), abi=ABI, execution_strategy=EXECUTION_STRATEGY,
            model={"model_id": model_id, "model_revision": model_revision,
                   "expert_pack_sha256": file_sha256(expert_pack)},
            workload={"layer_index": LAYER, "tokens": 1, "prefill_tokens": PREFILL_TOKENS, "top_k": TOP_K,
                      "unique_experts": TOP_K, "warmup_iterations": warmup, "measured_iterations": measured},
            projection_results=projections, moe_forward=decode, acceptance=ACCEPTANCE, samples_ms=samples,
            cache=cache, prefill_moe_forward=prefill, prefill_samples_ms=prefill_samples)
        validate_kernel_evidence(doc)
        return doc
    finally:
        unregister_expert_pack(handle)
        reader.close()


def main(argv: list[str] | None = None) -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    parser.add_argument("--expert-pack", type=Path, required=True)
    parser.add_argument("--model-manifest-sha256", required=True)
    parser.add_argument("--target-id", default="mi355x", choices=("mi355x",))
    parser.add_argument("--warmup-iterations", type=int, default=3)
    parser.add_argument("--measured-iterations", type=int, default=10)
    parser.add_argument("--output", type=Path, required=True)
    args = parser.parse_args(argv)
    if args.output.exists():
        raise SystemExit("refusing to overwrite packed Q4 kernel evidence")
    doc = run(args.expert_pack, model_manifest_sha256=args.model_manifest_sha256, warmup=args.warmup_iterations,
              measured=args.measured_iterations, target_id=args.target_id)
    args.output.parent.mkdir(parents=True, exist_ok=True)
    args.output.write_text(json.dumps(doc, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    print(json.dumps({"status": doc["status"], "gates": doc["gates"]}, sort_keys=True))
    return 0 if doc["gates"]["overall_passed"] else 1


if __name__ == "__main__":
    raise SystemExit(main())
