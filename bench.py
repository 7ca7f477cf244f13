"""MoE-layer benchmark on one MI355X (contract: one JSON line on stdout).

Workload: one Qwen1.5-MoE-A2.7B-shaped MoE block,
W4A16 routed experts (60 x [1408 x 2048], top-4, Q4 group-128 with FP32
scales) plus the BF16 shared expert (5632) and its sigmoid gate, decode batch
1, seeded synthetic weights N(0, 0.02). A step is one MoE block call on one
token: router, top-k, permutation, routed gate/up/SiLU/down, shared expert,
combine. R distinct layer instances (R x bytes >= 1 GiB) are rotated so that
the 256 MB MALL cannot serve the weights; the R calls are captured in one HIP
graph, which the timed region replays.

``value`` is microseconds per token per MoE layer (lower is better). The
roofline is HBM: algorithmic bytes = weight bytes one call must read (each
selected expert once + router + shared expert + shared gate).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "uma-qmoe_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBPS = 8000.0


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=240)
    ap.add_argument("--warmup", type=int, default=24)
    ap.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5", "trace", "qwen", "pack"],
                    help="c2 (default): Qwen W4A16 decode; c1: OLMoE decode; c3: 24-layer Qwen stack (BF16/Q8 routed "
                         "experts), decode; c4: Qwen prefill, 512 tokens; c5: 128-expert top-8 layer, 256 tokens "
                         "with Zipf-skewed routes (routed experts only); trace: the reference's measured OLMoE "
                         "RouteTrace (128-token prefill + 31 decode tokens over 16 layers) replayed through "
                         "c1-shaped Q4 layers; qwen: end-to-end greedy decode of a Qwen1.5-MoE-A2.7B-shaped model "
                         "(synthetic weights) through the host integration, one HIP graph per token; pack: open, "
                         "validate and stage a Q4 TargetPack of c2 layers with the library's pack reader")
    ap.add_argument("--tokens", type=int, default=0, help="tokens per call (0: the config's own)")
    ap.add_argument("--rotate-bytes", type=float, default=1.1e9)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-batch32", dest="batch32", action="store_false",
                    help="skip the batch-32 decode measurement reported beside the batch-1 value")
    ap.add_argument("--multi-kernel", action="store_true",
                    help="one- and two-token calls take the multi-launch path (UQM_OPT_FUSED_DECODE = 0) "
                         "instead of the fused kernel")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="only run 8 device-to-device copies of BYTES bytes (calibrates rocprofv3 "
                         "FETCH_SIZE / WRITE_SIZE against a kernel of known traffic) and exit")
    return ap.parse_args()


def counter_collection_active(environ=None) -> bool:
    """Whether this process runs under rocprofv3 hardware-counter collection
    (--pmc or a counter input file), which sets ROCPROF_COUNTER_COLLECTION and
    ROCPROF_COUNTERS / ROCPROF_COUNTER_GROUPS in the profiled program's
    environment."""
    env = os.environ if environ is None else environ
    flag = str(env.get("ROCPROF_COUNTER_COLLECTION", "")).strip().lower()
    return flag not in ("", "0", "false", "no", "off") or bool(env.get("ROCPROF_COUNTERS")) or bool(
        env.get("ROCPROF_COUNTER_GROUPS"))


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _time_calls(fn, seconds: float, least: int, most: int):
    times = []
    start = time.perf_counter()
    while time.perf_counter() - start < seconds or len(times) < least:
        t0 = time.perf_counter_ns()
        fn()
        times.append((time.perf_counter_ns() - t0) / 1e3)
        if len(times) >= most:
            break
    times.sort()
    return times[len(times) // 2], len(times)


def cpu_baseline(shape, seconds: float, ext=None):
    """The oracle (reference CPU correctness path restated) on the host cores,
    two rows, ~``seconds`` of work in all: (i) as the reference runs it,
    transient dequantization on every call, FP32 FFN, BF16 index_add_, BF16
    shared expert; (ii) the same arithmetic on weights dequantized to FP32
    once (a compute-only CPU bound). With ``ext``, the same token also runs
    through the HIP block once and the reference_oracle agreement metrics of
    the two outputs (same routes) and of the two routings are returned."""
    import torch

    from oracle import moe as om
    from uma_qmoe_amd import synthetic as syn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    progress(f"cpu baseline: {shape.name} on {cores} host cores")
    layer = syn.build_experts(shape, seed=syn.SEED + 1)
    dense = syn.build_dense(shape, seed=syn.SEED + 1)
    reader = syn.DeviceLayerReader({0: layer})
    lay = {"router": dense.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
           "shared_gate": dense.shared_gate, "shared_up": dense.shared_up, "shared_down": dense.shared_down,
           "shared_expert_gate": dense.shared_expert_gate}
    x = syn.hidden_states(shape, 1)
    for _ in range(2):
        om.qwen_block(x, lay, reader, 0)
    med, n = _time_calls(lambda: om.qwen_block(x, lay, reader, 0), seconds / 2, 5, 200)
    weights_of = om.predequantized(reader, 0, shape.num_experts)
    om.qwen_block(x, lay, reader, 0, weights_of=weights_of)
    med_pre, n_pre = _time_calls(lambda: om.qwen_block(x, lay, reader, 0, weights_of=weights_of), seconds / 2, 5, 2000)
    row = {
        "value": round(med, 1),
        "unit": "us/token",
        "cores": cores,
        "kind": "port",
        "sample": f"median of {n} single-token {shape.name} block calls (oracle, dequantize per call)",
        "cpu_model": cpu_model(),
        "predequantized": {"value": round(med_pre, 1), "unit": "us/token",
                           "sample": f"median of {n_pre} calls with every expert dequantized to FP32 once"},
    }
    agreement = None
    if ext is not None:
        from uma_qmoe_amd.evidence import NORTH_STAR, Q4_LAYER_POLICY, check_policy, numeric_agreement, route_agreement

        dev = torch.device("cuda:0")
        mv = lambda t: None if t is None else t.to(dev)  # noqa: E731
        layer_d = syn.DeviceExperts(layer.encoding, layer.group_size, layer.num_experts, layer.hidden_size,
                                    layer.intermediate_size, *(mv(t) for t in (layer.gate, layer.gate_scales, layer.up,
                                                                               layer.up_scales, layer.down,
                                                                               layer.down_scales)))
        dense_d = syn.DenseBlock(*(mv(t) for t in (dense.router, dense.shared_gate, dense.shared_up, dense.shared_down,
                                                   dense.shared_expert_gate)))
        out, _logits, w, idx = ext.moe_layer(layer_d, dense_d, x.to(dev), shape.top_k)
        torch.cuda.synchronize()
        ref_same, *_ = om.qwen_block(x, lay, reader, 0, routes=(w.cpu(), idx.cpu()), weights_of=weights_of)
        _ref, _rl, _rw, ref_idx = om.qwen_block(x, lay, reader, 0, weights_of=weights_of)
        numeric = numeric_agreement(ref_same, out.cpu(), epsilon=Q4_LAYER_POLICY["relative_error_epsilon"])
        routes = route_agreement(ref_idx, idx.cpu())
        agreement = {
            "scope": f"one {shape.name} token, HIP block vs oracle on the same routes; routes vs the oracle's own",
            "output": numeric,
            "routes": routes,
            "policy": "olmoe_q4_group128_halo3_single_moe_layer_v1 thresholds",
            "policy_failures": check_policy(numeric, routes, Q4_LAYER_POLICY),
            "north_star_ok": numeric["rel_l2"] <= NORTH_STAR["max_rel_l2"]
            and numeric["absolute_error"]["max"] <= NORTH_STAR["max_absolute_error"],
        }
    return row, agreement


BASELINE_METRIC = "MoE layer \u00b5s/token + achieved HBM GB/s (% peak), Qwen-MoE shape, batch 1 & 32"


# Sources of the single-token fused kernel: a profile of it stays valid while
# these hash to the digest recorded with the measurement.
FUSED_KERNEL_SOURCES = ("uqm_fused.hip", "uqm_device.h", "uqm_internal.h")


def fused_kernel_source_sha256() -> str:
    """SHA-256 over FUSED_KERNEL_SOURCES (name, NUL, bytes, in that order)."""
    import hashlib

    digest = hashlib.sha256()
    for name in FUSED_KERNEL_SOURCES:
        digest.update(name.encode("utf-8"))
        digest.update(b"\0")
        digest.update((ROOT / "uma-qmoe_amd" / "csrc" / name).read_bytes())
    return digest.hexdigest()


def profiled_traffic(workload: str):
    """HBM bytes per launch of the fused kernel from the committed rocprofv3
    summary (profiles/moe_decode_fused_c2.md), only while the kernel's sources
    still hash to the digest recorded with the measurement."""
    import re

    path = ROOT / "profiles" / "moe_decode_fused_c2.md"
    if not path.is_file():
        return None
    m = re.search(r"```json\n(.*?)\n```", path.read_text(), re.S)
    if m is None:
        return None
    data = json.loads(m.group(1))
    if data.get("workload") != workload or data.get("source_sha256") != fused_kernel_source_sha256():
        return None
    return int(data["traffic_bytes_per_launch"])


MFMA_PEAK_TFLOPS = 2500.0  # dense bf16


def layer_flops(shape, tokens: int, routes: int) -> float:
    """Multiply-adds x 2 of one block call: router, routed gate/up/down per
    route, shared gate/up/down per token."""
    f = 2.0 * shape.hidden * shape.num_experts * tokens
    f += 6.0 * shape.hidden * shape.intermediate * routes
    f += 6.0 * shape.hidden * shape.shared_intermediate * tokens
    return f


def zipf_routes(torch, syn, shape, x, dense):
    """Top-k routes of a Zipf-biased router (c5): logits = bf16(x W_r^T + b).
    Only the workload's routing pattern matters here, not tie order."""
    bias = syn.zipf_router_bias(shape, device=x.device)
    vals = (torch.nn.functional.linear(x, dense.router).float() + bias).to(torch.bfloat16).float()
    idx = torch.topk(vals, shape.top_k, dim=-1).indices
    w = torch.softmax(vals, -1).gather(-1, idx).to(torch.bfloat16)
    return idx.to(torch.int64).contiguous(), w.contiguous()


def progress(msg: str) -> None:
    """One line per bench phase on stderr (the JSON line alone goes to stdout)."""
    print(f"[bench {time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


CV_LIMIT = 0.03
MIN_SAMPLES = 10
MIN_TIMED_CALLS = 1300  # >= 100 replays of the 13-instance rotation in all samples together


def sample_plan(steps: int) -> int:
    """Samples of exactly ``steps`` layer calls each: at least MIN_SAMPLES,
    and enough that all samples together time >= MIN_TIMED_CALLS calls."""
    return max(MIN_SAMPLES, math.ceil(MIN_TIMED_CALLS / max(1, steps)))


def timed_samples(torch, run_calls, steps: int, warmup: int, samples: int, stream=None):
    """``warmup`` untimed calls, then ``samples`` timings of exactly ``steps``
    calls each, bracketed by device synchronisations, with HIP events on the
    stream the kernels run on. ``run_calls(n)`` enqueues n calls. Returns the
    per-sample milliseconds."""
    run_calls(warmup)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    out = []
    for _ in range(samples):
        torch.cuda.synchronize()
        start.record(stream)
        run_calls(steps)
        stop.record(stream)
        torch.cuda.synchronize()
        out.append(start.elapsed_time(stop))
    return out


def sample_stats(per_call_us):
    from uma_qmoe_amd.evidence import percentile

    s = sorted(per_call_us)
    mean = sum(s) / len(s)
    var = sum((v - mean) ** 2 for v in s) / max(1, len(s) - 1)
    cv = math.sqrt(var) / mean
    return {"samples": len(s), "p50_us": round(percentile(s, 0.50), 3), "p95_us": round(percentile(s, 0.95), 3),
            "p99_us": round(percentile(s, 0.99), 3), "mean_us": round(mean, 3), "cv": round(cv, 5),
            "cv_limit": CV_LIMIT, "cv_ok": cv <= CV_LIMIT}


def measure(torch, syn, ext, shape, tokens, steps, warmup, rotate_bytes):
    """Times one MoE block call on `tokens` tokens: R distinct layer instances
    whose per-call reads together exceed `rotate_bytes` (>= 1 GB, so the 256 MB
    MALL cannot serve the weights) are captured in one HIP graph (plus a graph
    of the first `steps mod R` calls), and each sample replays exactly `steps`
    calls between HIP events on torch's current stream (the stream the
    library launches on). Returns the per-call statistics and algorithmic
    GB/s (each distinct selected expert counted once, plus router and shared
    expert)."""
    dev = torch.device("cuda:0")
    x = syn.hidden_states(shape, tokens, device=dev)
    routed_only = shape.zipf_s is not None
    ws = ext._workspace(dev, tokens, shape.hidden, shape.intermediate, shape.shared_intermediate, shape.num_experts,
                        shape.top_k)
    probe = syn.build_experts(shape, device=dev, seed=syn.SEED)
    dense0 = syn.build_dense(shape, device=dev, seed=syn.SEED)
    fixed = zipf_routes(torch, syn, shape, x, dense0) if routed_only else None
    if routed_only:
        probe_idx = fixed[0]
        probe_bytes = syn.algorithmic_bytes(probe, None, int(torch.unique(probe_idx).numel()))
    else:
        probe_idx = ext.moe_layer(probe, dense0, x, shape.top_k, workspace=ws)[3]
        probe_bytes = syn.algorithmic_bytes(probe, dense0, int(torch.unique(probe_idx).numel()))
    r_inst = max(2, math.ceil(rotate_bytes / probe_bytes))
    progress(f"{shape.name} T={tokens}: building {r_inst} layer instances")
    layers, denses = [probe], [dense0]
    for i in range(r_inst - 1):
        layers.append(syn.build_experts(shape, device=dev, seed=syn.SEED + 100 + i))
        denses.append(syn.build_dense(shape, device=dev, seed=syn.SEED + 100 + i))
        torch.cuda.synchronize()
        progress(f"{shape.name} T={tokens}: instance {i + 2}/{r_inst} built")
    outs = [torch.empty((tokens, shape.hidden), dtype=torch.bfloat16, device=dev) for _ in range(r_inst)]

    def run_range(n):
        res = []
        for i in range(n):
            if routed_only:
                ext.moe_forward(layers[i], x, fixed[0], fixed[1], out=outs[i], workspace=ws)
                res.append((outs[i], None, fixed[1], fixed[0]))
            else:
                res.append(ext.moe_layer(layers[i], denses[i], x, shape.top_k, out=outs[i], workspace=ws))
        return res

    # eager warm-up; a fused launch that hit its wait budget (workgroups not
    # all resident) raises here instead of being timed
    results = run_range(r_inst)
    torch.cuda.synchronize()
    ext.workspace_status(ws)
    progress(f"{shape.name} T={tokens}: eager pass done")
    results = run_range(r_inst)
    torch.cuda.synchronize()
    distinct = [int(torch.unique(res[3]).numel()) for res in results]
    algo_bytes = [syn.algorithmic_bytes(layers[i], None if routed_only else denses[i], distinct[i])
                  for i in range(r_inst)]
    valid_routes = [int((res[3] >= 0).sum()) for res in results]
    flops = sum(layer_flops(shape, tokens, r) for r in valid_routes) / r_inst
    if routed_only:
        flops -= 2.0 * shape.hidden * shape.num_experts * tokens  # the router is not run
    graphs = {}
    for n in {r_inst, steps % r_inst, warmup % r_inst} - {0}:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run_range(n)
        graphs[n] = g
    torch.cuda.synchronize()
    progress(f"{shape.name} T={tokens}: graphs captured")

    def run_calls(n):
        for _ in range(n // r_inst):
            graphs[r_inst].replay()
        if n % r_inst:
            graphs[n % r_inst].replay()

    samples = sample_plan(steps)
    ms = timed_samples(torch, run_calls, steps, warmup, samples)
    ext.workspace_status(ws)
    per_call_us = [v * 1000.0 / steps for v in ms]
    stats = sample_stats(per_call_us)
    progress(f"{shape.name} T={tokens}: {samples} samples x {steps} calls, p50 {stats['p50_us']} us, "
             f"cv {stats['cv']}")
    # the first `steps mod R` instances are timed once more per sample than
    # the rest: weight the bytes the same way
    counts = [steps // r_inst + (1 if i < steps % r_inst else 0) for i in range(r_inst)]
    mean_bytes = sum(c * b for c, b in zip(counts, algo_bytes)) / steps
    us = stats["p50_us"]
    del graphs, layers, denses, outs, ws
    torch.cuda.empty_cache()
    return {"us_per_layer": us, "gbps": mean_bytes / (us * 1e-6) / 1e9, "bytes": mean_bytes, "instances": r_inst,
            "steps": steps, "warmup": warmup, "flops": flops, "tflops": flops / (us * 1e-6) / 1e12,
            "distinct_experts": sum(distinct) / len(distinct), "stats": stats,
            "per_call_ms": [v / 1000.0 for v in per_call_us]}


def measure_stack(torch, syn, ext, steps_per_rep: int, reps: int):
    """c3: the 24-layer Qwen stack, one token, ``steps_per_rep`` decode steps
    of x <- MoE_l(RMSNorm(x)) for l = 0..23 (routed BF16 in layers 0-15, Q8 in
    16-23, BF16 shared expert in every layer; RMSNorm eps 1e-6, weight ones).
    One step (24 pre-normalised blocks) is captured in a HIP graph that starts
    and ends in the same token buffer, so replays chain the steps. The ~22.6 GB
    of weights are read once per step (no MALL reuse). Returns the median over
    ``reps`` of the per-step time for: the fused single-token kernel with the
    norm folded in (the product path), the same kernel after a separate
    RMSNorm launch, and the multi-kernel path."""
    from uma_qmoe_amd import _native

    dev = torch.device("cuda:0")
    progress("c3: building 24 layers")
    shapes = [syn.c3_layer_shape(l) for l in range(syn.C3_LAYERS)]
    layers = [syn.build_experts(s, layer=l, device=dev) for l, s in enumerate(shapes)]
    denses = [syn.build_dense(s, layer=l, device=dev) for l, s in enumerate(shapes)]
    s0 = shapes[0]
    ws = ext._workspace(dev, 1, s0.hidden, s0.intermediate, s0.shared_intermediate, s0.num_experts, s0.top_k)
    x0 = syn.hidden_states(s0, 1, device=dev, tag="c3_x0")
    # layer l reads bufs[l % 2] and writes bufs[(l + 1) % 2]: an even layer
    # count ends every step in bufs[0], where the next step starts
    bufs = [x0.clone(), torch.empty_like(x0)]
    # one token routes to top_k distinct experts in every layer
    algo = sum(syn.algorithmic_bytes(layers[l], denses[l], s.top_k) for l, s in enumerate(shapes))

    def step_folded():
        for l, s in enumerate(shapes):
            ext.norm_moe_layer(layers[l], denses[l], bufs[l % 2], s.top_k, 1e-6, out=bufs[(l + 1) % 2], workspace=ws)

    def step_separate():
        for l, s in enumerate(shapes):
            normed = ext.rmsnorm(bufs[l % 2], 1e-6)
            ext.moe_layer(layers[l], denses[l], normed, s.top_k, out=bufs[(l + 1) % 2], workspace=ws)

    out = {}
    for mode, fused, step in (("fused", 1, step_folded), ("fused_separate_norm", 1, step_separate),
                              ("multi_kernel", 0, step_folded)):
        ext.set_option(_native.UQM_OPT_FUSED_DECODE, fused)
        bufs[0].copy_(x0)
        for _ in range(2):
            step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            step()
        torch.cuda.synchronize()
        for _ in range(2):
            graph.replay()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        samples = []
        for _ in range(reps):
            start.record()
            for _ in range(steps_per_rep):
                graph.replay()
            stop.record()
            torch.cuda.synchronize()
            samples.append(start.elapsed_time(stop) * 1000.0 / steps_per_rep)
        ext.workspace_status(ws)
        if not bool(torch.isfinite(bufs[0].float()).all()):
            raise RuntimeError(f"c3 stack ({mode}) produced non-finite values")
        out[mode] = sorted(samples)[len(samples) // 2]
        progress(f"c3 {mode}: {out[mode]:.1f} us per token")
        del graph
    ext.set_option(_native.UQM_OPT_FUSED_DECODE, 1)
    del layers, denses, ws
    torch.cuda.empty_cache()
    return {"us_per_token": out["fused"], "separate_norm_us_per_token": out["fused_separate_norm"],
            "multi_kernel_us_per_token": out["multi_kernel"], "bytes": algo, "steps": steps_per_rep * reps}


def cpu_baseline_stack(seconds: float):
    """The oracle on the host cores for c3, sampled: one BF16 layer (layer 0)
    and one Q8 layer (layer 16) are timed (median of repeated single-token
    block calls, ~``seconds`` in all) and the stack is 16 x the first + 8 x the
    second (the RMSNorms are < 0.1% and not counted)."""
    import torch

    from oracle import moe as om
    from uma_qmoe_amd import synthetic as syn

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    med = {}
    for layer in (0, 16):
        shape = syn.c3_layer_shape(layer)
        experts = syn.build_experts(shape, layer=layer)
        dense = syn.build_dense(shape, layer=layer)
        reader = syn.DeviceLayerReader({layer: experts})
        lay = {"router": dense.router, "top_k": shape.top_k, "num_experts": shape.num_experts,
               "shared_gate": dense.shared_gate, "shared_up": dense.shared_up, "shared_down": dense.shared_down,
               "shared_expert_gate": dense.shared_expert_gate}
        x = syn.hidden_states(shape, 1, tag="c3_x0")
        om.qwen_block(x, lay, reader, layer)
        times = []
        start = time.perf_counter()
        while time.perf_counter() - start < seconds / 2 or len(times) < 3:
            t0 = time.perf_counter_ns()
            om.qwen_block(x, lay, reader, layer)
            times.append((time.perf_counter_ns() - t0) / 1e3)
            if len(times) >= 100:
                break
        times.sort()
        med[layer] = (times[len(times) // 2], len(times))
        del experts, dense, reader
    value = 16 * med[0][0] + 8 * med[16][0]
    return {
        "value": round(value, 1),
        "unit": "us/token",
        "cores": cores,
        "kind": "port",
        "sample": (f"16 x median of {med[0][1]} BF16 layer-0 block calls + 8 x median of {med[16][1]} Q8 layer-16 "
                   "block calls (oracle, dequantize per call), single token"),
    }


def main_stack(args, torch, syn, ext) -> int:
    # the default --steps (240) keeps c3's own 32 steps per timing; a smaller
    # --steps is split over the 5 timings
    reps = 5
    steps_per_rep = syn.C3_STEPS if args.steps >= 240 else max(1, args.steps // reps)
    head = measure_stack(torch, syn, ext, steps_per_rep, reps)
    us = head["us_per_token"]
    gbps = head["bytes"] / (us * 1e-6) / 1e9
    line = {
        "metric": "24-layer Qwen MoE stack µs/token + achieved HBM GB/s (% peak), batch 1",
        "value": round(us, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": 4,
        "ms_per_step": round(us / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 / w8a16 (bf16 activations, fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) token)",
        "config": {
            "workload": ("c3_qwen_stack: 24 x (RMSNorm + MoE block: router + top-4 of 60 experts I=1408 + bf16 shared "
                         "expert 5632), routed BF16 in layers 0-15 and Q8 in 16-23, H=2048, one token, "
                         f"{steps_per_rep} chained decode steps per timing"),
            "tokens": 1,
            "parallelism": "single GPU",
        },
        "us_per_layer": round(us / syn.C3_LAYERS, 3),
        "separate_norm_us_per_token": round(head["separate_norm_us_per_token"], 3),
        "multi_kernel_us_per_token": round(head["multi_kernel_us_per_token"], 3),
        "algorithmic_bytes_per_token": int(head["bytes"]),
        "hbm_gbps": round(gbps, 1),
        "hbm_frac": round(gbps / HBM_PEAK_GBPS, 4),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_stack(args.cpu_seconds)
    print(json.dumps(line), flush=True)
    return 0


TRACE_FIXTURE = ROOT / "tests" / "golden" / "route_trace" / "olmoe_1b_7b_0125_128x32_greedy_v1.npz"


def qwen_config():
    """Transformers config of Qwen1.5-MoE-A2.7B (its config.json: 24 layers,
    hidden 2048, 16 heads, 60 routed experts of 1408, top-4, shared expert
    5632, vocabulary 151936)."""
    from transformers import Qwen2MoeConfig

    return Qwen2MoeConfig(vocab_size=151936, hidden_size=2048, intermediate_size=5632, moe_intermediate_size=1408,
                          shared_expert_intermediate_size=5632, num_hidden_layers=24, num_attention_heads=16,
                          num_key_value_heads=16, num_experts=60, num_experts_per_tok=4, norm_topk_prob=False,
                          max_position_embeddings=8192, rope_theta=1000000.0, rms_norm_eps=1e-6,
                          tie_word_embeddings=False, decoder_sparse_step=1, mlp_only_layers=[])


def main_qwen(args, torch, syn, ext) -> int:
    """Greedy decode of a Qwen1.5-MoE-A2.7B-shaped model with synthetic
    weights (dense BF16 tensors N(0, 0.02), norms 1; routed experts the
    synthetic Q4 layers of c2, one per layer) through the host integration:
    every MoE block one ``moe_block`` op over a registered pack, attention and
    head in torch, the whole step captured in one HIP graph per token over a
    static KV cache (uma_qmoe_amd.qwen_host). Times ``--steps`` tokens per
    sample after a 128-token prompt; the reference quotes 94.6 ms TPOT for
    its eager host on a gfx1151 APU with the real checkpoint,
    which is not this hardware nor these weights, so vs_baseline is null."""
    from uma_qmoe_amd.custom_op import register_expert_pack, register_moe_forward, unregister_expert_pack
    from uma_qmoe_amd.native_backend import install_packed_q4_backend
    from uma_qmoe_amd.qwen_host import DecodeGraph, replace_moe_blocks, restore_nonpersistent_buffers
    from transformers import Qwen2MoeForCausalLM

    dev = torch.device("cuda:0")
    config = qwen_config()
    layers = config.num_hidden_layers
    progress(f"qwen: building {layers} synthetic Q4 layers")
    reader = syn.DeviceLayerReader({l: syn.build_experts(syn.C2, layer=l, device=dev) for l in range(layers)},
                                   model={"num_experts": config.num_experts})
    register_moe_forward()
    install_packed_q4_backend()
    handle = register_expert_pack(reader)
    try:
        with torch.device("meta"):
            model = Qwen2MoeForCausalLM(config).to(torch.bfloat16)
        replace_moe_blocks(model, handle, performance_mode=True)
        model.to_empty(device=dev)
        gen = torch.Generator(device=dev).manual_seed(syn.SEED)
        with torch.no_grad():
            for name, p in model.named_parameters():
                if name.endswith("norm.weight") or "layernorm" in name:
                    p.fill_(1.0)
                else:
                    p.normal_(0.0, 0.02, generator=gen)
        restore_nonpersistent_buffers(model, config, dev)
        model.eval()
        # a 128-token prompt and a few hundred generated tokens: the static
        # cache (which attention reads whole every step) stays short
        prompt_len, samples = 128, 5
        per_sample = max(1, min(args.steps, 32))
        warmup = max(1, min(args.warmup, 8))
        dg = DecodeGraph(model, max_len=prompt_len + 8 + warmup + samples * per_sample + 2)
        ids = torch.randint(0, config.vocab_size, (1, prompt_len), generator=gen, device=dev)
        progress("qwen: prefill (stages every layer's experts)")
        dg.prefill(ids)
        torch.cuda.synchronize()
        # eager decode for comparison (same operations, launched one by one)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        for _ in range(2):
            dg.step_eager()
        torch.cuda.synchronize()
        e0.record()
        for _ in range(4):
            dg.step_eager()
        e1.record()
        torch.cuda.synchronize()
        eager_ms = e0.elapsed_time(e1) / 4
        progress(f"qwen: eager decode {eager_ms:.3f} ms/token; capturing")
        dg.capture()
        for _ in range(warmup):
            dg.replay()
        torch.cuda.synchronize()
        per_token = []
        for _ in range(samples):
            e0.record()
            for _ in range(per_sample):
                dg.replay()
            e1.record()
            torch.cuda.synchronize()
            per_token.append(e0.elapsed_time(e1) / per_sample)
        stats = sample_stats([v * 1000.0 for v in per_token])
        ms = stats["p50_us"] / 1000.0
        progress(f"qwen: graph decode {ms:.3f} ms/token, cv {stats['cv']}")
        line = {
            "metric": "Qwen1.5-MoE-A2.7B-shaped greedy decode TPOT (ms/token), synthetic weights, HIP graph per token",
            "value": round(ms, 4), "unit": "ms/token", "n_gpus": 1, "steps": samples * per_sample, "warmup": warmup,
            "ms_per_step": round(ms, 4), "higher_is_better": False, "scaling": "weak", "vs_baseline": None,
            "dtype": "w4a16 routed experts, bf16 dense", "data": "synthetic (random weights, random 128-token prompt)",
            "config": {"workload": "qwen: 24 x (attention + moe_block), vocab 151936, prompt 128, static KV cache",
                       "tokens": 1, "parallelism": "single GPU"},
            "tokens_per_s": round(1000.0 / ms, 2),
            "eager_ms_per_token": round(eager_ms, 4),
            "timing": {**stats, "steps_per_sample": per_sample},
            "reference_tpot_ms": {"value": 94.6, "hardware": "gfx1151 (the reference's eager host, real weights)"},
        }
        progress("done")
        print(json.dumps(line), flush=True)
        return 0
    finally:
        unregister_expert_pack(handle)


def main_pack(args, torch, syn, ext) -> int:
    """The pack reader (f1) on a Q4 TargetPack of four c2-shaped layers
    written to local disk: open + full validation (both SHA-256s over every
    byte, per-tensor hashes, payload scans) and staging of each layer to the
    device, in GB/s of pack bytes. The file is read from the page cache
    (written just before), so these are the reader's own rates, not the
    disk's."""
    import tempfile

    from uma_qmoe_amd.native_backend import stage_experts
    from uma_qmoe_amd.packfile import TargetPackReader, write_target_pack

    dev = torch.device("cuda:0")
    layers = 4
    with tempfile.TemporaryDirectory(dir=os.environ.get("TMPDIR", "/tmp")) as tmp:
        path = Path(tmp) / "c2_q4.uqtp"
        progress(f"pack: writing {layers} c2 layers")

        def tensors():
            for l in range(layers):
                built = syn.build_experts(syn.C2, layer=l, device=dev)
                for name, t in syn.pack_tensors({0: built}):
                    yield name.replace("layers.0.", f"layers.{l}."), t

        write_target_pack(path, tensors(), model_id="Qwen/Qwen1.5-MoE-A2.7B", model_revision="a" * 40,
                          model_manifest_sha256="b" * 64, policy_id="bench-q4",
                          layer_encodings={i: "q4_group128" for i in range(24)}, policy_evidence_sha256="e" * 64)
        size = path.stat().st_size
        opens, stages = [], []
        for rep in range(3):
            t0 = time.perf_counter()
            reader = TargetPackReader(path)
            opens.append(time.perf_counter() - t0)
            try:
                t0 = time.perf_counter()
                for l in range(layers):
                    staged = stage_experts(reader, l, dev)
                torch.cuda.synchronize()
                stages.append(time.perf_counter() - t0)
                del staged
            finally:
                reader.close()
            progress(f"pack: pass {rep + 1}: open {opens[-1]:.3f} s, stage {stages[-1]:.3f} s")
    o, st = sorted(opens)[1], sorted(stages)[1]
    line = {
        "metric": "pack reader: open + validate and stage to HBM, GB/s of pack bytes",
        "value": round(size / st / 1e9, 3), "unit": "GB/s (staging)", "n_gpus": 1, "steps": 3, "warmup": 0,
        "ms_per_step": round(st * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic (c2 Q4 layers written to a pack file on local disk, page cache warm)",
        "config": {"workload": f"pack: {layers} c2 Q4 layers, {size} bytes", "tokens": 0, "parallelism": "single GPU"},
        "open_validate_s": round(o, 4), "open_validate_gbps": round(size / o / 1e9, 3),
        "stage_s": round(st, 4), "host_threads": len(os.sched_getaffinity(0)),
    }
    print(json.dumps(line), flush=True)
    return 0


def main_trace(args, torch, syn, ext) -> int:
    """Replays the measured routes of the reference's RouteTrace (OLMoE,
    batch 1, 128 prompt tokens, 32 output tokens: one prefill event, 31
    decode events) through 16 synthetic c1-shaped Q4 layers: each (event,
    layer) is one routed-expert call with the trace's expert ids and routing
    weights. The prefill (16 calls of 128 tokens) and the decode steps (31 x
    16 single-token calls) are captured in two HIP graphs and timed apart;
    algorithmic bytes count each distinct expert of an (event, layer) once
    (16 x 64 experts x 3.34 MB = 3.4 GB of layers, no rotation needed)."""
    from uma_qmoe_amd.route_trace import distinct_experts, load_arrays

    arrays = load_arrays(TRACE_FIXTURE)
    dev = torch.device("cuda:0")
    shape = syn.C1
    n_layers = arrays["expert_indices"].shape[0]
    progress(f"trace: building {n_layers} c1 layers")
    layers = [syn.build_experts(shape, layer=l, device=dev) for l in range(n_layers)]
    counts = [int(c) for c in arrays["token_counts"]]
    bounds = [0]
    for c in counts:
        bounds.append(bounds[-1] + c)
    idx = torch.from_numpy(arrays["expert_indices"]).to(dev)
    wts = torch.from_numpy(arrays["routing_weights"]).to(torch.bfloat16).to(dev)
    xs = [syn.hidden_states(shape, c, device=dev, tag=f"trace{e}") for e, c in enumerate(counts)]
    outs = [torch.empty_like(x) for x in xs]
    ws = ext._workspace(dev, max(counts), shape.hidden, shape.intermediate, 0, shape.num_experts, shape.top_k)

    def run(events):
        for e in events:
            for l in range(n_layers):
                ext.moe_forward(layers[l], xs[e], idx[l, bounds[e]:bounds[e + 1]], wts[l, bounds[e]:bounds[e + 1]],
                                out=outs[e], workspace=ws)

    prefill, decode = [0], list(range(1, len(counts)))
    run(prefill + decode)
    torch.cuda.synchronize()
    graphs = {}
    for name, evs in (("prefill", prefill), ("decode", decode)):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            run(evs)
        graphs[name] = g
    torch.cuda.synchronize()
    progress("trace: graphs captured")
    per_expert = layers[0].bytes_per_expert()
    dist = distinct_experts(arrays)
    res = {}
    for name, evs in (("prefill", prefill), ("decode", decode)):
        # 20 timings of one whole replay each (the decode graph is 496 calls)
        ms = timed_samples(torch, lambda n, g=graphs[name]: [g.replay() for _ in range(n)], 1, 2, 20)
        stats = sample_stats([v * 1000.0 for v in ms])
        nbytes = int(sum(dist[e].sum() for e in evs) * per_expert)
        res[name] = {"us": stats["p50_us"], "bytes": nbytes, "stats": stats}
        progress(f"trace {name}: {stats['p50_us']} us ({len(evs)} events x {n_layers} layers)")
    dec = res["decode"]
    us_token = dec["us"] / len(decode)
    gbps = dec["bytes"] / (dec["us"] * 1e-6) / 1e9
    pre_gbps = res["prefill"]["bytes"] / (res["prefill"]["us"] * 1e-6) / 1e9
    line = {
        "metric": "RouteTrace replay: routed-expert µs per decode token over 16 OLMoE-shaped W4A16 MoE layers",
        "value": round(us_token, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": len(decode) * n_layers,
        "warmup": 2 * len(decode) * n_layers,
        "ms_per_step": round(dec["us"] / (len(decode) * n_layers) / 1000.0, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (q4 weights, bf16 activations, fp32 accumulate)",
        "data": "routes measured by the reference (benchmarks/traces/olmoe_1b_7b_0125_128x32_greedy_v1.json, "
                "stored as tests/golden/route_trace/*.npz); synthetic N(0,0.02) weights and N(0,1) hidden states",
        "config": {"workload": "trace: 16 c1-shaped Q4 layers (E 64, top-8, I 1024, H 2048), routed experts only, "
                               "one 128-token prefill event and 31 single-token decode events",
                   "parallelism": "single GPU"},
        "us_per_layer_call": round(dec["us"] / (len(decode) * n_layers), 3),
        "decode": {"us_all_steps": round(dec["us"], 3), "algorithmic_bytes": dec["bytes"],
                   "hbm_gbps": round(gbps, 1), "frac": round(gbps / HBM_PEAK_GBPS, 4), "timing": dec["stats"]},
        "prefill": {"us": round(res["prefill"]["us"], 3), "tokens": counts[0], "algorithmic_bytes": res["prefill"]["bytes"],
                    "hbm_gbps": round(pre_gbps, 1), "frac": round(pre_gbps / HBM_PEAK_GBPS, 4),
                    "distinct_experts_per_layer": [int(v) for v in dist[0]], "timing": res["prefill"]["stats"]},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
    }
    ext.workspace_status(ws)
    progress("done")
    print(json.dumps(line), flush=True)
    return 0


def workload_name(shape) -> str:
    enc = {"q4_group128": "Q4", "q8_group128": "Q8", "bf16_le": "BF16"}[shape.encoding]
    w = (f"{shape.name}: one MoE block (router + top-{shape.top_k} of {shape.num_experts} {enc} experts "
         f"I={shape.intermediate}")
    if shape.shared_intermediate:
        w += f" + bf16 shared expert {shape.shared_intermediate}"
    w += f"), H={shape.hidden}"
    if shape.zipf_s is not None:
        w = (f"{shape.name}: routed experts only, top-{shape.top_k} of {shape.num_experts} {enc} experts "
             f"I={shape.intermediate}, H={shape.hidden}, Zipf(s={shape.zipf_s}) routes")
    return w


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2
    if counter_collection_active() and not args.copy_probe:
        print("bench.py refuses to run under rocprofv3 counter collection (--pmc): a FETCH_SIZE run of it once "
              "stopped for 180 s while building its layer instances and the cause is not known. Take counters "
              "with the standalone programs (uma-qmoe_amd/lib/fused_timeline, uma-qmoe_amd/lib/grouped_counters) "
              "or calibrate with --copy-probe.", file=sys.stderr)
        return 3
    import torch

    if args.copy_probe:
        src = torch.empty(args.copy_probe, dtype=torch.uint8, device="cuda:0").fill_(1)
        dst = torch.empty_like(src)
        for _ in range(8):
            # an elementwise kernel (x ^ 0): a device-to-device copy_ may go to
            # a DMA engine, which the counters do not see
            torch.bitwise_xor(src, 0, out=dst)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": args.copy_probe, "copies": 8}), flush=True)
        return 0

    from uma_qmoe_amd import _native
    from uma_qmoe_amd import synthetic as syn
    from uma_qmoe_amd.native_backend import load_native_extension

    _platform, ext = load_native_extension()
    if args.config == "c3":
        return main_stack(args, torch, syn, ext)
    if args.config == "qwen":
        return main_qwen(args, torch, syn, ext)
    if args.config == "pack":
        return main_pack(args, torch, syn, ext)
    if args.config == "trace":
        return main_trace(args, torch, syn, ext)
    if args.multi_kernel:
        ext.set_option(_native.UQM_OPT_FUSED_DECODE, 0)
    shape = syn.CONFIGS[args.config]
    tokens = args.tokens if args.tokens > 0 else shape.tokens
    head = measure(torch, syn, ext, shape, tokens, args.steps, args.warmup, args.rotate_bytes)
    us_per_layer = head["us_per_layer"]
    achieved = head["gbps"]
    # the bound is whichever roofline leaves less time: HBM bytes or MFMA flops
    mfma_bound = head["flops"] / (MFMA_PEAK_TFLOPS * 1e12) > head["bytes"] / (HBM_PEAK_GBPS * 1e9)
    if mfma_bound:
        roofline = {"bound": "mfma", "achieved": round(head["tflops"], 1), "peak": MFMA_PEAK_TFLOPS,
                    "unit": "TFLOP/s", "frac": round(head["tflops"] / MFMA_PEAK_TFLOPS, 4), "traffic": None}
    else:
        roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                    "frac": round(achieved / HBM_PEAK_GBPS, 4),
                    "traffic": profiled_traffic(shape.name) if tokens == 1 and not args.multi_kernel else None}
    line = {
        "metric": BASELINE_METRIC,
        "value": round(us_per_layer / tokens, 3),
        "unit": "us/token",
        "n_gpus": 1,
        "steps": head["steps"],
        "warmup": head["warmup"],
        "ms_per_step": round(us_per_layer / 1000.0, 6),
        "us_per_layer_call": round(us_per_layer, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "w4a16 (q4 weights, bf16 activations, fp32 accumulate)",
        "data": "synthetic (seeded N(0,0.02) weights, N(0,1) token)",
        "config": {
            "workload": workload_name(shape),
            "tokens": tokens,
            "rotated_instances": head["instances"],
            "path": "multi-kernel" if args.multi_kernel or tokens > 2 else "fused",
            "parallelism": "single GPU",
        },
        "tokens_per_s": round(tokens / (us_per_layer * 1e-6), 1),
        "algorithmic_bytes_per_call": int(head["bytes"]),
        "hbm_gbps": round(achieved, 1),
        "hbm_frac": round(achieved / HBM_PEAK_GBPS, 4),
        "mfma_tflops": round(head["tflops"], 2),
        "mfma_frac": round(head["tflops"] / MFMA_PEAK_TFLOPS, 4),
        "distinct_experts": round(head["distinct_experts"], 2),
        "timing": {**head["stats"], "steps_per_sample": head["steps"]},
        "roofline": roofline,
        "evidence": evidence_performance(head, shape),
    }
    if not head["stats"]["cv_ok"]:
        progress(f"WARNING: sample CV {head['stats']['cv']} exceeds {CV_LIMIT}: timing.cv_ok is false")
    if args.batch32 and tokens == 1 and args.config == "c2":
        b32 = measure(torch, syn, ext, shape, 32, max(32, args.steps // 4), max(8, args.warmup // 4), args.rotate_bytes)
        line["batch32"] = {
            "us_per_layer": round(b32["us_per_layer"], 3),
            "us_per_token": round(b32["us_per_layer"] / 32, 3),
            "tokens_per_s": round(32 / (b32["us_per_layer"] * 1e-6), 1),
            "algorithmic_bytes_per_call": int(b32["bytes"]),
            "achieved_gbps": round(b32["gbps"], 1),
            "frac": round(b32["gbps"] / HBM_PEAK_GBPS, 4),
            "distinct_experts": round(b32["distinct_experts"], 2),
            "timing": {**b32["stats"], "steps_per_sample": b32["steps"]},
        }
    if not args.no_cpu_baseline and tokens == 1:
        line["cpu_baseline"], line["reference_oracle"] = cpu_baseline(shape, args.cpu_seconds, ext)
    progress("done")
    print(json.dumps(line), flush=True)
    return 0


def evidence_performance(head, shape) -> dict:
    """The performance block of a packed_q4_kernel_evidence record for this
    measurement: per-call milliseconds of every sample, median, nearest-rank
    p95, and one layer's compressed expert bytes (nothing dequantized)."""
    from uma_qmoe_amd.evidence import timing

    t = timing(head["per_call_ms"])
    per_expert = {"q4_group128": 0.5 + 4 / 128, "q8_group128": 1 + 4 / 128, "bf16_le": 2}[shape.encoding]
    expert_bytes = int(shape.num_experts * 3 * shape.hidden * shape.intermediate * per_expert)
    return {"scope": "single_moe_layer_microbenchmark", "samples_milliseconds": [round(v, 6) for v in t["samples_milliseconds"]],
            "median_milliseconds": round(t["median_milliseconds"], 6), "p95_milliseconds": round(t["p95_milliseconds"], 6),
            "compressed_cache_tensor_count": 3 * shape.num_experts, "compressed_cache_bytes": expert_bytes,
            "dequantized_weight_cache_bytes": 0, "formal_tps_claim": False}


if __name__ == "__main__":
    sys.exit(main())
