"""Benchmark of the MI355X routed-expert (MoE) path.

Headline workload: one MoE-layer decode step at batch 1 -- router softmax/top-8
over 128 expert logits, then the FP8 W8A8 routed experts (hidden 2048, expert
intermediate 768, per-output-channel E4M3 weight scales, bf16 activations) with
the slot-order weighted combine.  A step is one layer for one token; steps
rotate over LAYERS distinct layer banks (16 x 606 MB, far above the 256 MB
Infinity Cache) with fresh seeded logits per step, all inputs resident in HBM,
and are replayed from hipGraphs.

Reported: value = microseconds per layer decode step (lower is better).  The
step is one launch of the single-launch decode kernel (fp8_fused_decode_kernel),
so the roofline line is that kernel's: algorithmic bytes of the step (distinct
experts' FP8 rows and scales, activations, logits) over its average launch
duration from HIP events on the launch stream; traffic = its copy-calibrated
FETCH_SIZE + WRITE_SIZE from the committed counter summary.  Beside it: the
same steps through the three-launch decode, 4-, 8- and 16-token decode, the
whole MoE block (router GEMV, routed experts, shared expert, residual adds),
the 2048-token FP8 prefill, the packed-bank formats, and the reference's own CPU
expert executor (compiled from its sources into oracle/_ref) timed on this
host's cores on a bounded sample of the same layer shape.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "drama3-studio_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HIDDEN, INTER, EXPERTS, TOP_K = 2048, 768, 128, 8
LAYERS = 16
HBM_PEAK_GBS = 8000.0
SEED = 20261202  # 20261201 + config index 1


def log(*parts):
    print("[bench]", *parts, file=sys.stderr, flush=True)


def make_layer_bank(layer: int, device):
    """One layer of 128 experts: N(0, 0.02) weights, per-channel E4M3 scales."""
    import torch

    from drama_moe.formats import StagedExperts, quantize_fp8_weights

    g = torch.Generator(device=device).manual_seed(SEED * 100 + layer)
    parts = []
    for rows, cols in ((2 * INTER, HIDDEN), (HIDDEN, INTER)):
        w = torch.empty(EXPERTS, rows, cols, device=device)
        for e0 in range(0, EXPERTS, 32):
            w[e0:e0 + 32].normal_(0.0, 0.02, generator=g)
        q, s = quantize_fp8_weights(w, "channel")
        del w
        parts += [q, s]
    return StagedExperts(*parts)


def decode_graph_us(backend, xs, logits, banks, outs, stream, steps: int, warmup: int) -> tuple[float, float]:
    """Replays a hipGraph of one routed decode step per layer bank (all inputs
    resident) until `steps` steps ran; HIP events on the launch stream.
    Returns (microseconds per step, total milliseconds)."""
    import torch

    layers = len(banks)

    def step(i):
        backend.forward_routed(xs[i], logits[i], TOP_K, banks[i], out=outs[i])

    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the current stream
    with torch.cuda.stream(stream):  # workspace and descriptor caches, outside capture
        for i in range(layers):
            step(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(layers):
            step(i)
    remainder = steps % layers
    tail = None
    if remainder:
        tail = torch.cuda.CUDAGraph()
        with torch.cuda.graph(tail, stream=stream):
            for i in range(remainder):
                step(i)
    for _ in range(max(1, warmup // layers)):
        graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        torch.cuda.synchronize()
        start.record(stream)
        for _ in range(steps // layers):
            graph.replay()
        if tail is not None:
            tail.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    total_ms = start.elapsed_time(stop)
    return total_ms * 1e3 / steps, total_ms


def decode_inputs(tokens: int, device, seed: int):
    import torch

    g = torch.Generator(device=device).manual_seed(seed)
    xs = torch.randn(LAYERS, tokens, HIDDEN, device=device, generator=g).bfloat16()
    logits = torch.randn(LAYERS, tokens, EXPERTS, device=device, generator=g)
    return xs, logits, torch.empty_like(xs)


def step_bytes(logits, tokens: int) -> tuple[float, float]:
    """Algorithmic HBM bytes of one decode step, averaged over the layers:
    the distinct experts' FP8 rows and per-channel scales, the bf16 input and
    output rows, the fp32 logits.  Returns (bytes, mean distinct experts)."""
    import torch

    from drama_moe import router

    with torch.no_grad():
        ids = [router.route_topk(logits[i], TOP_K)[1].reshape(-1).tolist() for i in range(logits.shape[0])]
    uniq = [len(set(r)) for r in ids]
    return sum(u * EXPERT_BYTES + 2 * tokens * HIDDEN * 2 + tokens * EXPERTS * 4 for u in uniq) / len(uniq), \
        sum(uniq) / len(uniq)


# one expert's FP8 rows (w13 + w2) and per-output-channel fp32 scales
EXPERT_BYTES = 2 * INTER * HIDDEN + HIDDEN * INTER + (2 * INTER + HIDDEN) * 4


def run_gpu(steps: int, warmup: int):
    """The headline decode (1 token) through the single-launch kernel, the
    same steps through the three-launch decode, and multi-token decode."""
    import torch

    from drama_moe import _lib
    from drama_moe.offload import HipExpertBackend

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    log("device", torch.cuda.get_device_name(device))
    banks = [make_layer_bank(layer, device) for layer in range(LAYERS)]
    torch.cuda.synchronize()
    log("banks ready:", LAYERS, "layers x", round(banks[0].nbytes / 1e6, 1), "MB")
    backend = HipExpertBackend()
    stream = torch.cuda.Stream(device)
    lib = _lib.library()

    xs, logits, outs = decode_inputs(1, device, SEED)
    # The graph holds one fp8_fused_decode_kernel launch per step and nothing
    # else, so the per-step time is that kernel's average launch duration.
    us_per_step, total_ms = decode_graph_us(backend, xs, logits, banks, outs, stream, steps, warmup)
    # the status word of every timed step: a bounded wait that gave up
    # (SYNC_TIMEOUT) or a bad route would make the timing meaningless
    status = backend.status(device)
    if status:
        raise RuntimeError(f"decode steps raised device status bits {status:#x}")
    alg_bytes, uniq = step_bytes(logits, 1)
    fused_out = outs.clone()
    lib.dmoe_set_fused_decode(0)
    try:
        staged_us, _ = decode_graph_us(backend, xs, logits, banks, outs, stream, min(steps, 1024), warmup)
    finally:
        lib.dmoe_set_fused_decode(1)
    same = bool(torch.equal(outs, fused_out))
    multi = {}
    for tokens in (4, 8, 16):
        mx, ml, mo = decode_inputs(tokens, device, SEED + tokens)
        t_us, _ = decode_graph_us(backend, mx, ml, banks, mo, stream, min(steps, 1024), warmup)
        mbytes, muniq = step_bytes(ml, tokens)
        multi[f"tokens_{tokens}"] = {"us": round(t_us, 2), "unique_experts_mean": round(muniq, 2),
                                     "hbm_frac": round(mbytes / (t_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    status = backend.status(device)
    if status:
        raise RuntimeError(f"decode steps raised device status bits {status:#x}")
    return {
        "us_per_step": us_per_step, "total_ms": total_ms, "alg_bytes_step": alg_bytes,
        "step_gbs": alg_bytes / (us_per_step * 1e-6) / 1e9, "unique_experts_mean": uniq,
        "three_launch_us": staged_us, "three_launch_identical": same, "multi_token": multi,
        "device": torch.cuda.get_device_name(device),
    }


PMC_WORKLOADS = ("decode", "prefill", "w4a16", "decode_multi", "packed", "block")


def pmc_pass(workload: str = "decode", rounds: int = 8, copy_mib: int = 256):
    """Eager workload for hardware-counter runs, then a plain fp32 copy of
    `copy_mib` MiB (read once, written once) whose counter readings calibrate
    the bytes-per-count of the HBM counters.  Workloads (each `rounds` times):
      decode        the 1-token decode step over the LAYERS layer banks;
      prefill       a 2048-token FP8 prefill layer, per-token activation scales;
      w4a16         a 512-token asymmetric W4A16 prefill layer;
      decode_multi  the three-launch decode at 4, 8 and 16 tokens (one layer
                    bank per token count, rotating over the banks);
      packed        the 1-token decode layer of every packed format (modes 0-5),
                    router inside, LAYERS banks per mode;
      block         the MoE block kernels around the routed experts at 1 token
                    (block_pre / block_post, LAYERS layers)."""
    import torch

    from drama_moe.offload import HipExpertBackend

    device = torch.device("cuda", 0)
    calls = rounds
    if workload == "decode_multi":
        banks = [make_layer_bank(layer, device) for layer in range(LAYERS)]
        backend = HipExpertBackend()
        for tokens in (4, 8, 16):
            xs, logits, outs = decode_inputs(tokens, device, SEED + tokens)
            for _ in range(rounds):
                for i in range(LAYERS):
                    backend.forward_routed(xs[i], logits[i], TOP_K, banks[i], out=outs[i])
        calls = 3 * rounds * LAYERS
    elif workload == "packed":
        from drama_moe.formats import random_quantized_bank
        from drama_moe.quantized import QuantizedExpertBackend

        g = torch.Generator(device=device).manual_seed(SEED + 5)
        xs, logits, outs = decode_inputs(1, device, SEED)
        layers = 4  # 4 banks x 6 formats stay within HBM comfortably; rotation defeats the MALL
        for mode in range(6):
            banks = [random_quantized_bank(mode, EXPERTS, HIDDEN, INTER, asymmetric=mode == 0, device=device,
                                           generator=g) for _ in range(layers)]
            backend = QuantizedExpertBackend(mode)
            for _ in range(rounds):
                for i in range(LAYERS):
                    backend.forward_routed(xs[i], logits[i], TOP_K, banks[i % layers], out=outs[i])
            del banks
            torch.cuda.synchronize()
        calls = 6 * rounds * LAYERS
    elif workload == "block":
        from drama_moe import block

        g = torch.Generator(device=device).manual_seed(SEED + 77)

        def w(*shape):
            return (torch.randn(*shape, device=device, generator=g) * 0.02).bfloat16()

        blocks = [block.MoeBlock(w(EXPERTS, HIDDEN), w(1, HIDDEN), w(SHARED_INTER, HIDDEN), w(SHARED_INTER, HIDDEN),
                                 w(HIDDEN, SHARED_INTER), None, None, top_k=TOP_K) for _ in range(LAYERS)]
        xs = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()
        after = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()
        experts_out = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()
        outs = torch.empty_like(xs)
        for _ in range(rounds):
            for i in range(LAYERS):
                logits, sgate, act = blocks[i].pre(xs[i])
                blocks[i].post(act, sgate, experts_out[i], after[i], out=outs[i])
        calls = rounds * LAYERS
    elif workload == "w4a16":
        from drama_moe import router
        from drama_moe.formats import random_quantized_bank
        from drama_moe.quantized import QuantizedExpertBackend

        g = torch.Generator(device=device).manual_seed(SEED)
        bank = random_quantized_bank(0, EXPERTS, HIDDEN, INTER, asymmetric=True, device=device, generator=g)
        x = torch.randn(512, HIDDEN, device=device, generator=g).bfloat16()
        w, i = router.route_topk(torch.randn(512, EXPERTS, device=device, generator=g), TOP_K)
        out = torch.empty_like(x)
        backend = QuantizedExpertBackend(0)
        for _ in range(rounds):
            backend.forward(x, i, w, bank, out=out)
    elif workload == "prefill":
        bank = make_layer_bank(LAYERS, device)
        g = torch.Generator(device=device).manual_seed(PREFILL_SEED)
        x = torch.randn(PREFILL_TOKENS, HIDDEN, device=device, generator=g).bfloat16()
        logits = zipf_logits(PREFILL_TOKENS, EXPERTS, PREFILL_SEED).to(device)
        out = torch.empty_like(x)
        backend = HipExpertBackend(x_group="token")
        for _ in range(rounds):
            backend.forward_routed(x, logits, TOP_K, bank, out=out)
    else:
        banks = [make_layer_bank(layer, device) for layer in range(LAYERS)]
        xs, logits, outs = decode_inputs(1, device, SEED)
        backend = HipExpertBackend()
        for _ in range(rounds):
            for i in range(LAYERS):
                backend.forward_routed(xs[i], logits[i], TOP_K, banks[i], out=outs[i])
    src = torch.ones(copy_mib << 18, device=device)
    dst = torch.empty_like(src)
    for _ in range(4):
        torch.mul(src, 1.0, out=dst)
    torch.cuda.synchronize()
    if workload == "decode":
        calls = rounds * LAYERS
    print(json.dumps({"pmc_pass": {"workload": workload, "calls": calls,
                                   "copy_bytes_read": src.numel() * 4, "copy_bytes_written": dst.numel() * 4}}),
          flush=True)


FUSED_PHASES = ("entry", "routed", "loads_issued", "first_gateup_batch", "gateup_done", "hidden_ready", "down_done")


def phase_times(replays: int = 64):
    """Phase timeline of the 1-token single-launch decode: the graph of one
    routed decode step per rotating layer bank that the headline times, each
    step captured with its own phase buffer (dmoe_debug_set_phase_buffer: the
    kernel's timing instance stamps the 100 MHz real-time counter at 7 points
    in thread 0 of every workgroup), replayed `replays` times.  Per phase, over
    workgroups and steps, the 10th / 50th / 90th percentile of (stamp - the
    step's earliest entry stamp) in microseconds; beside it the same graph's
    HIP-event time per step with the ordinary kernel."""
    import numpy as np
    import torch

    from drama_moe import _lib
    from drama_moe.offload import HipExpertBackend

    device = torch.device("cuda", 0)
    torch.cuda.set_device(device)
    banks = [make_layer_bank(layer, device) for layer in range(LAYERS)]
    backend = HipExpertBackend()
    stream = torch.cuda.Stream(device)
    lib = _lib.library()
    xs, logits, outs = decode_inputs(1, device, SEED)
    us_plain, _ = decode_graph_us(backend, xs, logits, banks, outs, stream, 16 * replays, 64)
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    per_step = cus * len(FUSED_PHASES)
    buf = torch.zeros(LAYERS, per_step, dtype=torch.int64, device=device)

    def step(i):
        _lib.check(lib.dmoe_debug_set_phase_buffer(_lib.ptr(buf[i]), per_step))
        backend.forward_routed(xs[i], logits[i], TOP_K, banks[i], out=outs[i])

    try:
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            for i in range(LAYERS):
                step(i)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(LAYERS):
                step(i)
    finally:
        _lib.check(lib.dmoe_debug_set_phase_buffer(None, 0))
    for _ in range(4):
        graph.replay()
    torch.cuda.synchronize()
    rel = []
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    timed_ms = 0.0
    for _ in range(replays):
        buf.zero_()
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            start.record(stream)
            graph.replay()
            stop.record(stream)
        torch.cuda.synchronize()
        timed_ms += start.elapsed_time(stop)
        stamps = buf.view(LAYERS, cus, len(FUSED_PHASES)).cpu().numpy().astype(np.float64)
        for layer in range(LAYERS):
            st = stamps[layer]
            t0 = st[:, 0][st[:, 0] > 0].min()
            rel.append(np.where(st > 0, (st - t0) / 100.0, np.nan))  # 100 MHz ticks -> us
    status = backend.status(device)
    if status:
        raise RuntimeError(f"decode steps raised device status bits {status:#x}")
    rel = np.stack(rel)  # [steps, workgroups, phases]
    phases = {}
    for k, name in enumerate(FUSED_PHASES):
        v = rel[:, :, k]
        v = v[~np.isnan(v)]
        phases[name] = {"p10_us": round(float(np.percentile(v, 10)), 2), "median_us": round(float(np.median(v)), 2),
                        "p90_us": round(float(np.percentile(v, 90)), 2), "workgroups": int(v.size // rel.shape[0])}
    last = np.nanmax(rel[:, :, -1], axis=1)
    print(json.dumps({"phase_times": phases, "steps": int(rel.shape[0]), "workgroups_per_step": cus,
                      "last_down_done_median_us": round(float(np.median(last)), 2),
                      "timing_instance_us_per_step": round(timed_ms * 1e3 / (replays * LAYERS), 2),
                      "ordinary_kernel_us_per_step": round(us_plain, 2),
                      "clock": "s_memrealtime, 100 MHz"}), flush=True)


# MiB one 1-token decode call reads: 8 experts x 3 x 768 x 2048 FP8 bytes plus
# their per-channel scales (37.86 MB).
DECODE_MB = 36.1


def stream_sweep(total_mib: int = 2048, replays: int = 10):
    """Plain streaming-read rate of the device by size: for each size S,
    ceil(total / S) distinct buffers of S bytes (so the rotation exceeds the
    256 MB Infinity Cache), each read once per round by the library's read
    probe (dmoe_stream_read: 16-byte non-temporal loads, four per lane in
    flight, up to 8 workgroups of 512 per CU), one launch per buffer replayed
    from a hipGraph as the decode steps are; microseconds per launch from HIP
    events.  The attainable fraction of the 8 TB/s peak for one pass of a
    given size, to set the single-launch decode (DECODE_MB per call) against."""
    import math

    import torch

    from drama_moe import _lib

    lib = _lib.library()
    device = torch.device("cuda", 0)
    stream = torch.cuda.Stream(device)
    sink = torch.zeros(1, dtype=torch.int32, device=device)
    rows = []
    for mb in (4, 8, 16, 24, 32, DECODE_MB, 48, 64, 128, 256, 512):
        nbytes = int(mb * (1 << 20)) // 16 * 16
        count = max(2, math.ceil(total_mib / mb))
        bufs = [torch.ones(nbytes // 4, device=device) for _ in range(count)]

        def reads():
            handle = ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)
            for b in bufs:
                _lib.check(lib.dmoe_stream_read(_lib.ptr(b), nbytes, _lib.ptr(sink), handle))

        us = _graph_time_us(reads, count, replays, stream)
        gbs = nbytes / (us * 1e-6) / 1e9
        rows.append({"mib": mb, "buffers": count, "workgroups": min(2048, -(-nbytes // (512 * 4 * 16))),
                     "us_per_read": round(us, 2), "gbs": round(gbs, 1), "frac_of_8tbs": round(gbs / HBM_PEAK_GBS, 4)})
        del bufs
        torch.cuda.empty_cache()
    if int(sink.item()) != 0:
        raise RuntimeError("stream read probe wrote its sink")
    print(json.dumps({"stream_sweep": rows}), flush=True)


PREFILL_TOKENS = 2048
PREFILL_SEED = 20261203  # 20261201 + config index 2
FP8_PEAK_TFLOPS = 5000.0


def zipf_logits(tokens: int, experts: int, seed: int, exponent: float = 1.1):
    """log p_e + Gumbel(0, 1), p_e ~ rank_e^-exponent over a seeded rank
    permutation: the top-k of these logits samples experts without replacement."""
    import torch

    g = torch.Generator().manual_seed(seed)
    ranks = torch.randperm(experts, generator=g).double() + 1
    logp = -exponent * torch.log(ranks)
    logp -= torch.logsumexp(logp, 0)
    u = torch.rand(tokens, experts, generator=g, dtype=torch.float64).clamp_(1e-12, 1 - 1e-12)
    return (logp - torch.log(-torch.log(u))).float()


def run_prefill(reps: int = 10):
    """2048-token MoE layer: router + grouped FP8 experts, per-token activation
    scales (and the reference's per-128 groups), one 606 MB bank."""
    import torch

    from drama_moe.offload import HipExpertBackend

    device = torch.device("cuda", 0)
    bank = make_layer_bank(LAYERS, device)
    g = torch.Generator(device=device).manual_seed(PREFILL_SEED)
    x = torch.randn(PREFILL_TOKENS, HIDDEN, device=device, generator=g).bfloat16()
    logits = zipf_logits(PREFILL_TOKENS, EXPERTS, PREFILL_SEED).to(device)
    out = torch.empty_like(x)
    flops = 2.0 * PREFILL_TOKENS * TOP_K * 3 * INTER * HIDDEN
    nbytes = EXPERTS * (3 * INTER * HIDDEN + (2 * INTER + HIDDEN) * 4) + 2 * PREFILL_TOKENS * HIDDEN * 2 \
        + PREFILL_TOKENS * EXPERTS * 4
    result = {}
    for name, group in (("per_token", "token"), ("per_128", 128)):
        backend = HipExpertBackend(x_group=group)
        for _ in range(3):
            backend.forward_routed(x, logits, TOP_K, bank, out=out)
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(reps):
            backend.forward_routed(x, logits, TOP_K, bank, out=out)
        stop.record()
        torch.cuda.synchronize()
        status = backend.status(device)
        if status:
            raise RuntimeError(f"prefill calls raised device status bits {status:#x}")
        us = start.elapsed_time(stop) * 1e3 / reps
        tflops = flops / (us * 1e-6) / 1e12
        gbs = nbytes / (us * 1e-6) / 1e9
        result[name] = {"us": round(us, 2), "tflops": round(tflops, 1),
                        "mfma_frac": round(tflops / FP8_PEAK_TFLOPS, 4),
                        "hbm_frac": round(gbs / HBM_PEAK_GBS, 4),
                        "roofline_frac": round(max(tflops / FP8_PEAK_TFLOPS, gbs / HBM_PEAK_GBS), 4)}
    result.update({"tokens": PREFILL_TOKENS, "top_k": TOP_K, "experts": EXPERTS, "routing": "zipf1.1",
                   "alg_gflop": round(flops / 1e9, 2), "alg_mb": round(nbytes / 1e6, 1),
                   "mfma_frac_is": "algorithmic flops / measured time / FP8 dense peak",
                   "mfma_busy_counters": prefill_mfma_busy()})
    return result


def run_hybrid(calls: int = 128, threads: int = 8, layers: int = 2):
    """Cooperative decode: the lowest-ranked route slots of a 1-token FP8
    layer call on the host cores (the library's executor, `threads` workers),
    the others on the GPU, merged in slot order.  `layers` of the bench's
    banks attached from host memory; eager calls (the mode waits on the host
    for its partials), seeded inputs rotating over 16 tokens; wall-clock
    microseconds per layer call for 1, 2 and 4 host slots, beside the same
    calls on the GPU alone (eager, one host sync per call) and the executor
    alone on all 8 slots of a call."""
    import torch

    from drama_moe import fp8_moe, router
    from drama_moe.formats import EXPERT_BUFFER_NAMES, StagedExperts
    from drama_moe.hybrid import CpuExpertExecutor, silu_table
    from drama_moe.offload import HipExpertBackend, ResidentExpertManager

    device = torch.device("cuda", 0)

    class Experts(torch.nn.Module):
        fp8 = True

        def __init__(self, bank):
            super().__init__()
            for name in EXPERT_BUFFER_NAMES:
                self.register_buffer(name, getattr(bank, name))

    manager = ResidentExpertManager(backend=HipExpertBackend())
    modules = []
    for layer in range(layers):
        bank = make_layer_bank(layer, device)
        host = StagedExperts(*(getattr(bank, n).cpu() for n in EXPERT_BUFFER_NAMES))
        del bank
        module = Experts(host)
        manager.attach(str(layer), module)
        modules.append(module)
    g = torch.Generator(device=device).manual_seed(SEED + 91)
    xs = torch.randn(16, 1, HIDDEN, device=device, generator=g).bfloat16()
    routes = [router.route_topk(torch.randn(1, EXPERTS, device=device, generator=g), TOP_K)[::-1] for _ in range(16)]  # (ids, weights)

    def timed(n):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(n):
            ids, w = routes[i % 16]
            modules[i % layers](xs[i % 16], ids, w)
            torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e6 / n

    try:
        timed(16)  # device copies of the banks, first launches
        result = {"gpu_only_us": round(timed(calls), 1)}
        for jobs in (1, 2, 4):
            hybrid = manager.configure_hybrid_decode(jobs, threads=threads)
            with hybrid.decode():
                timed(8)
                us = timed(calls)
            stats = hybrid.report()
            result[f"cpu_jobs_{jobs}_us"] = round(us, 1)
            result[f"cpu_jobs_{jobs}_recomputed_pairs"] = stats["boundary_recomputed_pairs"]
        executor = CpuExpertExecutor(manager._bank_of(modules[0]), capacity=8, threads=threads,
                                     silu_table=silu_table(device))
        result["executor_isa"] = executor.implementation
        q, s = fp8_moe.quantize_groups(fp8_moe.quant_kernel, xs[0], HIDDEN)
        qh = q.view(torch.uint8).cpu().reshape(-1).contiguous()
        sh = s.cpu().reshape(-1).contiguous()
        ids, w = routes[0]
        ids_h, w_h = ids.cpu().reshape(-1), w.float().cpu().reshape(-1)
        store = manager._bank_of(modules[0])
        for _ in range(4):
            executor.forward_quantized_pairs(qh, sh, ids_h, w_h, store=store)
        t0 = time.perf_counter()
        reps = 32
        for _ in range(reps):
            executor.forward_quantized_pairs(qh, sh, ids_h, w_h, store=store)
        result["executor_8_slots_us"] = round((time.perf_counter() - t0) * 1e6 / reps, 1)
        executor.close()
        result.update({"threads": threads, "layers": layers, "calls": calls, "guard": True,
                       "timing": "wall clock per eager layer call"})
        return result
    finally:
        manager.close()


SHARED_INTER = 768  # the shared expert's intermediate size in the block leg


def run_block(steps: int, warmup: int):
    """Whole MoE block of one decoder layer at batch 1 (router GEMV, FP8
    routed experts, sigmoid-gated bf16 shared expert of SHARED_INTER, residual
    adds: three launches), over the same LAYERS rotating banks, hipGraph-
    replayed; beside it the two block launches alone."""
    import torch

    from drama_moe import block
    from drama_moe.offload import HipExpertBackend

    device = torch.device("cuda", 0)
    banks = [make_layer_bank(layer, device) for layer in range(LAYERS)]
    g = torch.Generator(device=device).manual_seed(SEED + 77)

    def w(*shape):
        return (torch.randn(*shape, device=device, generator=g) * 0.02).bfloat16()

    backend = HipExpertBackend()
    blocks = [block.MoeBlock(w(EXPERTS, HIDDEN), w(1, HIDDEN), w(SHARED_INTER, HIDDEN), w(SHARED_INTER, HIDDEN),
                             w(HIDDEN, SHARED_INTER), banks[i], backend, top_k=TOP_K) for i in range(LAYERS)]
    xs = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()
    after = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()
    outs = torch.empty_like(xs)
    stream = torch.cuda.Stream(device)
    steps = max(LAYERS, steps // LAYERS * LAYERS)
    replays = steps // LAYERS

    def whole():
        for i in range(LAYERS):
            blocks[i](xs[i], after[i], out=outs[i])

    pre_out = [blocks[i].pre(xs[i]) for i in range(LAYERS)]
    experts_out = torch.randn(LAYERS, 1, HIDDEN, device=device, generator=g).bfloat16()

    def pre_only():
        for i in range(LAYERS):
            blocks[i].pre(xs[i])

    def post_only():
        for i in range(LAYERS):
            blocks[i].post(pre_out[i][2], pre_out[i][1], experts_out[i], after[i], out=outs[i])

    del warmup  # _graph_time_us replays once before timing
    result = {"us": round(_graph_time_us(whole, LAYERS, replays, stream), 2),
              "pre_us": round(_graph_time_us(pre_only, LAYERS, replays, stream), 2),
              "post_us": round(_graph_time_us(post_only, LAYERS, replays, stream), 2)}
    status = backend.status(device)
    if status:
        raise RuntimeError(f"block steps raised device status bits {status:#x}")
    routed, uniq = step_bytes(torch.stack([pre_out[i][0] for i in range(LAYERS)]), 1)
    dense = (EXPERTS * HIDDEN + HIDDEN + 3 * SHARED_INTER * HIDDEN) * 2 + 3 * HIDDEN * 2
    nbytes = routed + dense
    result.update({"alg_mb": round(nbytes / 1e6, 2), "unique_experts_mean": round(uniq, 2),
                   "hbm_frac": round(nbytes / (result["us"] * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                   "shared_inter": SHARED_INTER, "launches": 3})
    return result


QUANT_NAMES = {0: "w4a16_asym_g128", 1: "int8_convrot", 2: "w6a8", 3: "w4a8_codebook", 4: "w4a8_g128_fp8",
               5: "w6a8_g128_fp8"}


def quant_expert_bytes(mode: int) -> int:
    """Packed bytes of one expert (w13 + w2 with their scales / aux / zeros)."""
    total = 0
    for n, k in ((2 * INTER, HIDDEN), (HIDDEN, INTER)):
        if mode == 0:
            total += n * k // 2 + n * (k // 128) * 2 + (k // 128) * (n // 8) * 4
        elif mode == 1:
            total += n * k + n * 4
        elif mode == 2:
            total += n * k * 3 // 4 + n * (k // 16 + 4)
        elif mode == 3:
            total += n * k // 2 + n * (k // 16 + 8)
        elif mode == 4:
            total += n * k // 2 + n * (k // 128) * 2
        else:
            total += n * k * 3 // 4 + n * (k // 128) * 2
    return total


def _graph_time_us(fn, steps_per_graph: int, replays: int, stream) -> float:
    import torch

    stream.wait_stream(torch.cuda.current_stream())  # inputs were made on the current stream
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        fn()
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(replays):
            graph.replay()
        stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) * 1e3 / (replays * steps_per_graph)


def run_quant(layers: int = 24, window: int = 16, replays: int = 16):
    """Packed-bank MoE layers (H 2048, 128 experts x I 768, top-8), all
    experts resident.  Per mode: a hipGraph of `window` decode steps through
    its layer banks (`layers` distinct banks for the 24-layer formats,
    LAYERS for the others), each (step, layer) a router + experts call on its
    own seeded logits (T=1), replayed so that `window * replays` steps run;
    plus the 512-token W4A16 prefill."""
    import torch

    from drama_moe.formats import random_quantized_bank
    from drama_moe.quantized import QuantizedExpertBackend

    device = torch.device("cuda", 0)
    stream = torch.cuda.Stream(device)
    result = {}
    for mode in (0, 2, 3, 4, 5, 1):
        step_layers = mode in (2, 3, 4, 5)
        n_layers = layers if step_layers else LAYERS
        banks = [random_quantized_bank(mode, EXPERTS, HIDDEN, INTER, asymmetric=mode == 0, device=device,
                                       generator=torch.Generator(device=device).manual_seed(SEED + 1000 * mode + l))
                 for l in range(n_layers)]
        backend = QuantizedExpertBackend(mode)
        g = torch.Generator(device=device).manual_seed(SEED + 7 * mode)
        xs = torch.randn(window, n_layers, 1, HIDDEN, device=device, generator=g).bfloat16()
        logits = torch.randn(window, n_layers, 1, EXPERTS, device=device, generator=g)
        outs = torch.empty_like(xs)

        def steps():
            for t in range(window):
                for l in range(n_layers):
                    backend.forward_routed(xs[t, l], logits[t, l], TOP_K, banks[l], out=outs[t, l])

        layer_us = _graph_time_us(steps, window * n_layers, replays, stream)
        status = backend.status(device)
        if status:
            raise RuntimeError(f"packed mode {mode} steps raised device status bits {status:#x}")
        _, step_uniq = step_bytes(logits.reshape(-1, 1, EXPERTS), 1)
        layer_bytes = step_uniq * quant_expert_bytes(mode) + 2 * HIDDEN * 2 + EXPERTS * 4
        entry = {"layer_us": round(layer_us, 2), "expert_bytes": quant_expert_bytes(mode),
                 "hbm_frac": round(layer_bytes / (layer_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                 "routing": "in the timed region"}
        if step_layers:
            entry.update({"layers": n_layers, "step_us": round(layer_us * n_layers, 1),
                          "steps_timed": window * replays})
        if mode == 0:  # 512-token prefill
            from drama_moe import router

            x = torch.randn(512, HIDDEN, device=device, generator=g).bfloat16()
            w, i = router.route_topk(torch.randn(512, EXPERTS, device=device, generator=g), TOP_K)
            out = torch.empty_like(x)
            prefill_us = _graph_time_us(lambda: backend.forward(x, i, w, banks[0], out=out), 1, 10, stream)
            flops = 2.0 * 512 * TOP_K * 3 * INTER * HIDDEN
            nbytes = EXPERTS * quant_expert_bytes(0) + 2 * 512 * HIDDEN * 2
            entry["prefill_512"] = {"us": round(prefill_us, 1), "tflops": round(flops / prefill_us / 1e6, 1),
                                    "hbm_frac": round(nbytes / (prefill_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
        result[QUANT_NAMES[mode]] = entry
        del banks
        torch.cuda.empty_cache()
    return result


def host_cpu() -> dict:
    """The host the CPU lanes run on: model string, vector ISA the reference
    executor selects (AVX-512 > AVX2 > scalar, as its cpuid dispatch), cores
    this process may use and physical cores."""
    model, flags, cores = "unknown", set(), set()
    try:
        phys = None
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            key, _, value = line.partition(":")
            key, value = key.strip(), value.strip()
            if key == "model name" and model == "unknown":
                model = value
            elif key == "flags" and not flags:
                flags = set(value.split())
            elif key == "physical id":
                phys = value
            elif key == "core id":
                cores.add((phys, value))
    except OSError:
        pass
    isa = "avx512" if {"avx512f", "avx512bw"} <= flags else "avx2" if "avx2" in flags else "scalar"
    return {"model": model, "isa": isa, "affinity_cpus": len(os.sched_getaffinity(0)),
            "physical_cores": len(cores) or os.cpu_count()}


def _timed(fn, budget_s: float, min_calls: int = 2):
    fn()
    calls, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s or calls < min_calls:
        fn()
        calls += 1
    return (time.perf_counter() - t0) * 1e6 / calls, calls


def cpu_baseline(budget_s: float = 8.0):
    """CPU lanes beside the GPU, on this host's cores.

    Headline (value): the reference's own CPU expert executor (compiled from
    its sources into oracle/_ref; scalar C oracle port without it), one token
    per call, its 8 route slots over 8 worker threads (the most it uses:
    it parallelises over route slots only), on a 128-expert bank of the
    decode layer's shape and weight distribution -- N(0, 0.02) weights, but
    with the 128x128 block scales the executor takes (the GPU leg uses
    per-channel scales) -- and 8 distinct random experts per call (the GPU
    leg routes N(0,1) logits).  Also: 1 thread; 4 tokens as 4 consecutive
    calls (the executor is batch-one); and the torch-CPU
    dequantize-then-matmul lanes (oracle/torch_cpu.py) of the FP8 and packed
    formats with torch's CPU threads."""
    import numpy as np
    import torch

    from drama_moe.formats import random_fp8_bank, random_quantized_bank
    from oracle import ref_native, torch_cpu

    device = torch.device("cuda", 0)
    rng = np.random.default_rng(SEED)
    gen = torch.Generator(device=device).manual_seed(SEED + 17)
    bank = random_fp8_bank(EXPERTS, HIDDEN, INTER, layout="block", generator=gen, device=device)
    host = {name: t.cpu() for name, t in bank.buffers().items()}
    w13, s13 = host["w13_weight"].view(torch.uint8).numpy(), host["w13_scale_inv"].numpy()
    w2, s2 = host["w2_weight"].view(torch.uint8).numpy(), host["w2_scale_inv"].numpy()
    xt = torch.randn(4, HIDDEN, generator=torch.Generator().manual_seed(SEED)).bfloat16()
    x = xt.view(torch.int16).numpy().view(np.uint16)
    weights = np.full(TOP_K, 1.0 / TOP_K, np.float32)
    lanes = {}
    info = host_cpu()

    def ids():
        return rng.choice(EXPERTS, TOP_K, replace=False).astype(np.int64)

    if ref_native.available():
        lib = ref_native.RefLibrary()
        kind = "reference"
        out = np.empty((TOP_K, HIDDEN), np.float32)
        for threads in (8, 1):
            with ref_native.RefExecutor(lib, HIDDEN, INTER, capacity=TOP_K, threads=threads) as ex:
                us, calls = _timed(lambda: ex.forward(w13, s13, w2, s2, x[0], ids(), weights, out),
                                   budget_s if threads == 8 else budget_s / 3)
                lanes[f"reference_executor_t1_threads{threads}"] = {"us_per_layer": round(us, 1), "calls": calls}
                if threads == 8:
                    def four():
                        for t in range(4):
                            ex.forward(w13, s13, w2, s2, x[t], ids(), weights, out)
                    us4, calls4 = _timed(four, budget_s / 4)
                    lanes["reference_executor_t4_threads8"] = {"us_per_layer": round(us4, 1), "calls": calls4}
        value, cores = lanes["reference_executor_t1_threads8"]["us_per_layer"], 8
        sample = (f"{lanes['reference_executor_t1_threads8']['calls']} one-token layer decodes on the reference's "
                  "drama_native executor, 8 threads over the 8 route slots")
    else:
        from oracle import oracle as orc

        kind, cores = "port", 1
        b13, b2 = orc.Fp8Bank(w13, s13), orc.Fp8Bank(w2, s2)
        xf = xt[0].float().numpy()
        value, calls = _timed(lambda: orc.fp8_expert_pairs(b13, b2, xf, ids(), weights), budget_s, 1)
        lanes["scalar_oracle_t1_threads1"] = {"us_per_layer": round(value, 1), "calls": calls}
        sample = f"{calls} one-token layer decodes on the scalar C oracle port, 1 thread"

    threads = torch.get_num_threads()
    torch.set_num_threads(info["affinity_cpus"])
    try:
        tids = torch.from_numpy(ids()[None])
        tw = torch.full((1, TOP_K), 1.0 / TOP_K)
        bank_cpu = type(bank)(**host)
        us, calls = _timed(lambda: torch_cpu.fp8_layer(bank_cpu, xt[:1], tids, tw), budget_s / 8)
        lanes["torch_cpu_fp8_o2_t1"] = {"us_per_layer": round(us, 1), "calls": calls}
        for mode in (0, 1, 2, 3, 4, 5):
            store = random_quantized_bank(mode, EXPERTS, HIDDEN, INTER, asymmetric=mode == 0, device=device,
                                          generator=torch.Generator(device=device).manual_seed(SEED + 31 * mode))
            store = type(store)(**{f: (getattr(store, f).cpu() if isinstance(getattr(store, f), torch.Tensor)
                                       else getattr(store, f)) for f in store.__dataclass_fields__})
            us, calls = _timed(lambda: torch_cpu.layer(store, xt[:1], tids, tw), budget_s / 8)
            lanes[f"torch_cpu_{QUANT_NAMES[mode]}_t1"] = {"us_per_layer": round(us, 1), "calls": calls}
    finally:
        torch.set_num_threads(threads)
    return {"value": round(value, 2), "unit": "us", "cores": cores, "kind": kind, "sample": sample,
            "host": info, "torch_threads": info["affinity_cpus"], "lanes": lanes,
            "inputs": "N(0,0.02) weights with 128x128 block scales (executor and O2 lanes; the GPU uses "
                      "per-channel scales), N(0,1) bf16 activations, 8 distinct random experts per token"}


TRAFFIC_SUMMARY = ROOT / "profiles" / "fp8_fused_decode_kernel_moe_layer_b1_hbm_traffic.txt"


PREFILL_COUNTERS = ROOT / "profiles" / "fp8_grouped_prefill_2048_counters.txt"


def prefill_mfma_busy():
    """SQ_VALU_MFMA_BUSY_CYCLES fractions of the grouped prefill GEMMs from the
    committed counter summary of the 2048-token layer, or None."""
    try:
        busy = {}
        for text in PREFILL_COUNTERS.read_text().splitlines():
            if text.startswith("mfma_busy_"):
                key, value = text.split(":", 1)
                busy[key[len("mfma_busy_"):]] = float(value)
        if busy:
            busy["source"] = str(PREFILL_COUNTERS.relative_to(ROOT))
            return busy
    except (OSError, ValueError):
        pass
    return None


def measured_traffic():
    """HBM bytes per launch of the fused decode kernel from the committed
    FETCH_SIZE / WRITE_SIZE counter summary (copy-calibrated), or None."""
    try:
        for text in TRAFFIC_SUMMARY.read_text().splitlines():
            if text.startswith("traffic_bytes_per_launch:"):
                return int(text.split(":", 1)[1])
    except (OSError, ValueError):
        pass
    return None


def main():
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=4096)
    parser.add_argument("--warmup", type=int, default=256)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-prefill", action="store_true")
    parser.add_argument("--no-quant", action="store_true")
    parser.add_argument("--no-block", action="store_true")
    parser.add_argument("--no-hybrid", action="store_true")
    parser.add_argument("--pmc-pass", nargs="?", const="decode", choices=PMC_WORKLOADS,
                        help="run an eager counter-collection workload (see pmc_pass) instead of the benchmark")
    parser.add_argument("--phase-times", action="store_true",
                        help="time the phases of the 1-token single-launch decode instead of the benchmark")
    parser.add_argument("--stream-sweep", action="store_true",
                        help="measure the plain streaming-read bandwidth by size instead of the benchmark")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the path is built and "
              "measured on a single MI355X, multi-GPU sharding is design-only.", file=sys.stderr)
        sys.exit(2)
    if int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py runs as a single process on one GPU", file=sys.stderr)
        sys.exit(2)
    if args.pmc_pass:
        pmc_pass(args.pmc_pass)
        return
    if args.stream_sweep:
        stream_sweep()
        return
    if args.phase_times:
        phase_times()
        return
    steps = max(1, args.steps)
    gpu = run_gpu(steps, args.warmup)
    log("gpu", json.dumps(gpu))
    moe_block = None if args.no_block else run_block(steps, args.warmup)
    log("block", json.dumps(moe_block))
    prefill = None if args.no_prefill else run_prefill()
    log("prefill", json.dumps(prefill))
    quant = None if args.no_quant else run_quant()
    log("quant", json.dumps(quant))
    hybrid = None if args.no_hybrid else run_hybrid()
    log("hybrid", json.dumps(hybrid))
    cpu = None if args.no_cpu_baseline else cpu_baseline()
    if cpu:
        log("cpu", json.dumps(cpu))
    frac = gpu["step_gbs"] / HBM_PEAK_GBS
    line = {
        "metric": "MoE-layer decode us + % peak HBM GB/s (B=1); FP8 prefill TFLOPS @2048 tok",
        "value": round(gpu["us_per_step"], 3),
        "unit": "us",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(gpu["us_per_step"] / 1e3, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 (W8A8, fp32 accumulate)",
        "data": "synthetic: N(0,0.02) weights -> per-channel E4M3, N(0,1) bf16 activations and fp32 logits, seeded",
        "config": {"workload": "MoE layer decode B=1: router top-8 of 128 + FP8 experts H2048 I768, "
                               f"{LAYERS} rotating layer banks, hipGraph",
                   "tokens": 1, "experts": EXPERTS, "hidden": HIDDEN, "intermediate": INTER,
                   "top_k": TOP_K, "layers_rotated": LAYERS},
        "hbm_gbs_step": round(gpu["step_gbs"], 1),
        "pct_peak_hbm_step": round(100 * frac, 2),
        "roofline": {"bound": "hbm", "achieved": round(gpu["step_gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(frac, 4), "traffic": measured_traffic(),
                     "kernel": "fp8_fused_decode_kernel", "kernel_us": round(gpu["us_per_step"], 3),
                     "alg_bytes_per_launch": round(gpu["alg_bytes_step"]),
                     "unique_experts_mean": round(gpu["unique_experts_mean"], 3)},
        "decode_three_launch_us": round(gpu["three_launch_us"], 3),
        "decode_three_launch_identical": gpu["three_launch_identical"],
        "decode_multi_token": gpu["multi_token"],
        "moe_block_decode": moe_block,
        "cpu_baseline": cpu,
        "prefill_fp8": prefill,
        "packed_banks": quant,
        "cooperative_decode": hybrid,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
