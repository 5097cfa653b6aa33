#!/usr/bin/env python
"""Benchmark of the fused IQ3_S x MXFP8 projection on one MI355X.

Default workload: the Llama-3-70B-shaped sweep - 80 layers x 7 projections (q 8192x8192,
k/v 1024x8192, o 8192x8192, gate/up 28672x8192, down 8192x28672), 560 distinct IQ3_S
weights (~29.4 GB resident in HBM) generated on the GPU from the counter-based
generator, streamed once per step at M tokens (default M=1, decode). One step = the
560 projections in 320 launches (projections that read the same input - q/k/v, gate/up -
share a grouped launch; --no-group launches each alone), replayed from a captured HIP
graph; MXFP8 activations are quantized once before timing (the reference times the
matmul alone, iq3_s_fp8.py:402-465). --workload llama8b runs the same sweep over the
32 layers of Llama-3-8B (3.0 GB of weights). --tp G sweeps one GPU's shard of a
G-way tensor-parallel layer (N/G rows of the column-parallel projections, K/G columns of
the row-parallel ones).

value = algorithmic bytes per step / step time, with
  bytes per projection = N*K*110/256 (IQ3_S weights) + M*K*33/32 (E4M3 + E8M0 activations)
                         + 4*M*N (f32 output)
roofline: HBM (8 TB/s) for the weight stream; for M >= 128 (prefill, MFMA-bound) the
line reports TFLOP/s (2*M*N*K per projection) against the 5.0 PFLOP/s dense MX-FP8 MFMA
peak instead. cpu_baseline: the oracle's restatement of the reference CPU path
(ggml_reference.cpp:495-523: IQ3_S to_float + float64 dot) on its CPU case, one IQ3_S
linear N=K=4096 with M=8, timed on this host.

    python bench.py [--steps K] [--warmup W] [--m M]
                    [--workload llama70b|llama8b|quant|copy|read|readsweep|mfma]
                    [--model llama70b|llama8b] [--layers L] [--tp G] [--no-group] [--no-graph] [--with-quant none|separate|fused]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
MXFP8_PEAK_TFLOPS = 5000.0  # dense MX-FP8 MFMA peak of MI355X
PREFILL_M = 128  # from this many tokens the projections are MFMA-bound: report TFLOP/s

from mambo_amd.utils.sweep import (build_launches, build_weights, capture, launch_shape, layer_shapes,  # noqa: E402
                                   make_step, time_replays)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def proj_bytes(m: int, n: int, k: int, act_bytes_per_value: float = 33 / 32) -> int:
    return n * k * 110 // 256 + int(m * k * act_bytes_per_value) + 4 * m * n


def run_gemm(args, weights=None):
    import torch
    from mambo_amd.kernels.iq3_s_fp8 import select_config

    if weights is None:
        weights = build_weights(args.workload, args.layers, args.tp)
    launches = build_launches(weights, args.m, args.no_group)
    projections = [p for (_, projs, _) in launches for p in projs]
    configs = [select_config(args.m, *launch_shape(projs)) for (_, projs, _) in launches]
    weight_bytes = sum(f.packed.numel() for (_, _, f, _) in projections)
    # with quantization in the step the activations come in as bf16 rows
    act_bytes = 2 if args.with_quant != "none" else 33 / 32
    step_bytes = sum(proj_bytes(args.m, n, k, act_bytes) for (n, k, _, _) in projections)
    step_flops = sum(2 * args.m * n * k for (n, k, _, _) in projections)
    log(f"{len(projections)} projections in {len(launches)} launches, {weight_bytes / 1e9:.2f} GB of IQ3_S "
        "weights resident")

    step = make_step(launches, configs, args.with_quant, chain=args.chain, chain_waves=args.chain_waves,
                     chain_tpw=args.chain_tpw)
    outputs = list({id(o): o for (_, _, _, o) in projections}.values())
    step()
    torch.cuda.synchronize()
    if args.chain:
        from mambo_amd.kernels.iq3_s_fp8 import chain_status
        chain_status(step.sync)  # a dependency wait that timed out stops the run here
    replay = step
    if not args.no_graph:
        # Capture one step on a side stream, then check one replay against eager results.
        ref = [o.clone() for o in outputs]
        graph = capture(step)
        for o in outputs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outputs, ref):
            # K-split launches add partial sums with f32 atomics, whose order varies from
            # run to run: allow last-bit differences relative to the output's scale
            if not torch.allclose(o, r, rtol=1e-4, atol=1e-5 * float(r.abs().max())):
                diff = (o - r).abs().max().item()
                raise RuntimeError(f"graph replay differs from eager launch (output {tuple(o.shape)}: max diff "
                                   f"{diff}, nan {int(torch.isnan(o).sum())}, ref nan {int(torch.isnan(r).sum())})")
        replay = graph.replay
        log("captured the step in a HIP graph; replay matches eager")

    ms, wall = time_replays(replay, args.steps, args.warmup)
    if args.chain:
        from mambo_amd.kernels.iq3_s_fp8 import chain_status
        chain_status(step.sync)  # raises if any dependency wait of the timed replays timed out
    gbs = step_bytes / (ms * 1e-3) / 1e9
    tflops = step_flops / (ms * 1e-3) / 1e12
    log(f"{ms:.3f} ms/step (wall {wall * 1e3 / args.steps:.3f}), {gbs:.1f} GB/s, {tflops:.2f} TFLOP/s")
    return {
        "ms": ms, "value": gbs, "tflops": tflops, "step_bytes": step_bytes, "step_flops": step_flops,
        "weight_bytes": weight_bytes, "projections": len(projections), "launches": len(launches),
        "per_launch_bytes": step_bytes / len(launches), "per_launch_us": ms * 1e3 / len(launches),
    }


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(seconds: float, unit: str = "GB/s") -> dict:
    """Oracle restatement of the reference CPU path on its CPU case: one IQ3_S linear
    N=K=4096 (seed-0 counter-based blocks), M=8 bf16 ~N(0,1) activations quantized to
    MXFP8, IQ3_S to_float + float64-accumulated dot per output. Timed on all host cores
    this process may use (OpenMP), then on one thread. Reported in the unit of the GPU
    line (GB/s of algorithmic bytes, or TFLOP/s)."""
    from oracle import oracle
    n = k = 4096
    m = 8
    raw = oracle.gen_iq3s(0, n, k // 256)
    xv, xs = oracle.quantize_mxfp8(oracle.gen_bf16(1, m * k).reshape(m, k))

    def timed(threads: int, budget: float):
        iters, t0 = 0, time.perf_counter()
        while True:
            oracle.iq3s_fp8_matmul(xv, xs, raw, threads=threads)
            iters += 1
            if time.perf_counter() - t0 >= budget:
                break
        return iters, (time.perf_counter() - t0) / iters

    def rate(per: float) -> float:
        return 2 * m * n * k / per / 1e12 if unit == "TFLOP/s" else proj_bytes(m, n, k) / per / 1e9

    threads = len(os.sched_getaffinity(0))
    iters, per = timed(threads, seconds)
    iters1, per1 = timed(1, seconds / 2)
    return {"value": round(rate(per), 6), "unit": unit, "cores": threads, "kind": "port",
            "cpu_model": cpu_model(),
            "single_thread": {"value": round(rate(per1), 6), "unit": unit, "cores": 1,
                              "ms_per_run": round(per1 * 1e3, 2), "runs": iters1},
            "sample": f"one IQ3_S linear N=K=4096, M=8 (the reference CPU case): {iters} runs in {per * iters:.1f} s "
                      f"({per * 1e3:.1f} ms each) on {threads} threads, {iters1} runs ({per1 * 1e3:.1f} ms each) on "
                      f"1 thread, of the oracle's to_float + f64-dot restatement of ggml_reference.cpp:495-523"}


def run_quant(args):
    import torch
    from mambo_amd import _native
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    m = k = 4096
    copies = 8  # rotate 8 x 32 MiB inputs so the 256 MB MALL does not hold them
    xs = []
    for c in range(copies):
        bits = torch.empty(m * k, dtype=torch.int16, device="cuda")
        _native.check(_native.lib().mambo_synth_bf16(1 + c, 2, 0.001, 0, m * k, bits.data_ptr(),
                                                     _native.stream_handle(None)))
        xs.append(bits.view(torch.bfloat16).view(m, k))
    outs = [(torch.empty((m, k), dtype=torch.uint8, device="cuda"),
             torch.empty((m, k // 32), dtype=torch.uint8, device="cuda")) for _ in range(copies)]
    for i in range(copies):  # eager first pass (checks the launch), then capture
        launch_quantize_fp8(xs[i], out=outs[i])
    torch.cuda.synchronize()
    rounds = 1 if args.no_graph else 8
    replay = lambda: [launch_quantize_fp8(xs[i], out=outs[i]) for _ in range(rounds) for i in range(copies)]  # noqa: E731
    if not args.no_graph:
        # one HIP graph of 8 rounds over the 8 inputs: a 10 us kernel launched from Python one
        # at a time would time the host's launch rate instead, and a graph of 8 launches
        # pays the ~20 us between graph replays once per 8 kernels
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=side):
            replay()
        torch.cuda.current_stream().wait_stream(side)
        replay = graph.replay
    for _ in range(args.warmup):
        replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        replay()
    stop.record()
    torch.cuda.synchronize()
    n = args.steps * copies * rounds
    ms = start.elapsed_time(stop) / n
    nbytes = m * k * (2 + 1) + m * (k // 32)
    return {"ms": ms, "value": nbytes / (ms * 1e-3) / 1e9, "step_bytes": nbytes, "launches": 1,
            "per_launch_bytes": nbytes, "per_launch_us": ms * 1e3}


COPY_BYTES = 1 << 30


def run_copy(args):
    """Plain copy of COPY_BYTES with mambo_copy_bytes: the calibration workload for the
    HBM byte counters (every byte read once and written once)."""
    import torch
    from mambo_amd import _native
    src = torch.empty(COPY_BYTES, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    src.fill_(1)

    def launch():
        _native.check(_native.lib().mambo_copy_bytes(src.data_ptr(), dst.data_ptr(), COPY_BYTES,
                                                     _native.stream_handle(None)), "copy")

    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        launch()
    stop.record()
    torch.cuda.synchronize()
    if not bool((dst == 1).all()):
        raise RuntimeError("copy kernel produced wrong bytes")
    ms = start.elapsed_time(stop) / args.steps
    nbytes = 2 * COPY_BYTES
    return {"ms": ms, "value": nbytes / (ms * 1e-3) / 1e9, "step_bytes": nbytes, "launches": 1,
            "per_launch_bytes": nbytes, "per_launch_us": ms * 1e3}


def run_read(args):
    """Plain read of COPY_BYTES with mambo_read_bytes: the read ceiling of this device for
    a stream of 16-byte loads (checked against the XOR of the input)."""
    import torch
    from mambo_amd import _native
    src = torch.empty(COPY_BYTES // 4, dtype=torch.int32, device="cuda")
    src.copy_(torch.arange(COPY_BYTES // 4, dtype=torch.int32, device="cuda") * 2654435761)
    sink = torch.empty(_native.READ_SINK_WORDS, dtype=torch.int32, device="cuda")

    def launch():
        _native.check(_native.lib().mambo_read_bytes(src.data_ptr(), COPY_BYTES, sink.data_ptr(),
                                                     _native.stream_handle(None)), "read")

    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        launch()
    stop.record()
    torch.cuda.synchronize()
    import numpy as np
    if int(np.bitwise_xor.reduce(sink.cpu().numpy())) != int(np.bitwise_xor.reduce(src.cpu().numpy())):
        raise RuntimeError("read kernel returned a wrong checksum")
    ms = start.elapsed_time(stop) / args.steps
    return {"ms": ms, "value": COPY_BYTES / (ms * 1e-3) / 1e9, "step_bytes": COPY_BYTES, "launches": 1,
            "per_launch_bytes": COPY_BYTES, "per_launch_us": ms * 1e3}


def sweep_launch_bytes(args) -> list:
    """Packed IQ3_S bytes each launch of the projection sweep reads (the grouping of
    mambo_amd.utils.sweep.build_launches: q/k/v and gate/up share a launch unless args.no_group)."""
    shapes = layer_shapes(args.model, args.tp)
    sizes = []
    for _ in range(args.layers):
        prev = None
        for _, n, k, slot in shapes:
            nbytes = n * (k // 256) * 110
            if not args.no_group and prev == slot and len(sizes[-1]) < 4:
                sizes[-1].append(nbytes)
            else:
                sizes.append([nbytes])
            prev = slot
    return [sum(s) for s in sizes]


def run_readsweep(args):
    """Plain read (mambo_read_bytes) of one buffer per launch of the --model sweep, each
    the size of the packed weights that launch streams, replayed from a HIP graph: the
    ceiling a weight stream with this launch structure can reach on this device (per-launch
    ramp-up and drain included). The last buffer's read is checked against its XOR."""
    import numpy as np
    import torch
    from mambo_amd import _native
    sizes = sweep_launch_bytes(args)
    bufs = [torch.empty(s, dtype=torch.uint8, device="cuda") for s in sizes]
    sink = torch.empty(_native.READ_SINK_WORDS, dtype=torch.int32, device="cuda")
    log(f"{len(sizes)} launches, {sum(sizes) / 1e9:.2f} GB resident")

    def step():
        for b, s in zip(bufs, sizes):
            _native.check(_native.lib().mambo_read_bytes(b.data_ptr(), s, sink.data_ptr(),
                                                         _native.stream_handle(None)), "read")

    step()
    torch.cuda.synchronize()
    words = bufs[-1].view(torch.int32).cpu().numpy()
    if int(np.bitwise_xor.reduce(sink.cpu().numpy())) != int(np.bitwise_xor.reduce(words)):
        raise RuntimeError("read kernel returned a wrong checksum")
    replay = step
    if not args.no_graph:
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.graph(graph, stream=side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        replay = graph.replay
    for _ in range(args.warmup):
        replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        replay()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    total = sum(sizes)
    log(f"{ms:.3f} ms/step, {total / (ms * 1e-3) / 1e9:.1f} GB/s")
    return {"ms": ms, "value": total / (ms * 1e-3) / 1e9, "step_bytes": total, "launches": len(sizes),
            "per_launch_bytes": total / len(sizes), "per_launch_us": ms * 1e3 / len(sizes)}


MFMA_WORKGROUPS = 1024  # x 4 waves: 4 waves per SIMD on 256 CUs
MFMA_ITERS = 20000


def run_mfma(args):
    """Scaled-MFMA (f8f6f4 16x16x128) throughput with mambo_mfma_peak: the on-device
    check of the 5.0 PFLOP/s dense MX-FP8 figure (checked against the known sums)."""
    import torch
    from mambo_amd import _native
    out = torch.empty(MFMA_WORKGROUPS * 256, dtype=torch.float32, device="cuda")

    def launch():
        _native.check(_native.lib().mambo_mfma_peak(MFMA_WORKGROUPS, MFMA_ITERS, out.data_ptr(),
                                                    _native.stream_handle(None)), "mfma_peak")

    for _ in range(args.warmup):
        launch()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        launch()
    stop.record()
    torch.cuda.synchronize()
    if not bool((out == 4096.0 * MFMA_ITERS).all()):
        raise RuntimeError("MFMA throughput kernel returned wrong sums")
    ms = start.elapsed_time(stop) / args.steps
    flops = MFMA_WORKGROUPS * 4 * MFMA_ITERS * 8 * 2 * 16 * 16 * 128
    return {"ms": ms, "value": flops / (ms * 1e-3) / 1e12, "tflops": flops / (ms * 1e-3) / 1e12,
            "step_flops": flops, "launches": 1, "per_launch_us": ms * 1e3}


def measured_traffic(workload: str):
    """HBM bytes per launch of the dominant kernel for `workload`, from the committed
    counter summaries (profiles/traffic_*.json), or None when none matches."""
    for path in sorted((REPO / "profiles").glob("traffic_*.json")):
        rec = json.loads(path.read_text())
        if rec.get("workload") == workload:
            return round(rec["traffic_bytes_per_launch"])
    return None


def gemm_workload_name(args) -> str:
    grouping = "one launch per projection" if args.no_group else "q/k/v and gate/up grouped per launch"
    if args.with_quant != "none":
        grouping += {"separate": ", a quantizer launch before each GEMM launch",
                     "fused": ", quantization inside the GEMM launch where it fits (M <= 4)"}[args.with_quant]
    if getattr(args, "chain", 0):
        grouping += (f", runs of up to {args.chain} consecutive launches of one K per chained launch (each "
                     "launch's activation reads wait for the one before it)")
    model = "llama3-70b" if args.workload == "llama70b" else "llama3-8b"
    shard = f" (one GPU's shard at tensor parallelism {args.tp})" if args.tp > 1 else ""
    return f"{model} projection sweep{shard}: {args.layers} layers x 7 IQ3_S linears, M={args.m}, {grouping}"


def roofline_of(r: dict, mfma_bound: bool, workload: str) -> dict:
    """roofline object of one measurement: achieved = algorithmic work per launch / the
    average launch time over the timed region (HIP events on the launch stream)."""
    if mfma_bound:
        value = r["tflops"]
        roof = {"bound": "mfma", "achieved": round(value, 2), "peak": MXFP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(value / MXFP8_PEAK_TFLOPS, 4), "traffic": measured_traffic(workload),
                "algorithmic_flops_per_launch": round(r["step_flops"] / r["launches"]),
                "avg_launch_us": round(r["per_launch_us"], 3)}
        if "per_launch_bytes" in r:  # the projections' operand bytes (not for the MFMA-rate check)
            roof["algorithmic_operand_bytes_per_launch"] = round(r["per_launch_bytes"])
        return roof
    value = r["value"]
    return {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4), "traffic": measured_traffic(workload),
            "algorithmic_bytes_per_launch": round(r["per_launch_bytes"]),
            "avg_launch_us": round(r["per_launch_us"], 3)}


# Further points of the M = 1..8192 metric timed by the default run, after the headline:
# the Llama-3-70B sweep at 16, 32 and 512 tokens (same weights), and at 1 token with one
# launch per projection (":nogroup", the way a caller of the reference's
# launch_iq3_s_fp8_matmul runs a layer, iq3_s_fp8.py:364-399); then the Llama-3-8B sweep
# at the decode sizes 1, 4 and 16 (1 also one launch per projection) and the prefill sizes
# 2048 and 8192 (32 layers, 3.0 GB of weights built beside the 70B ones).
DEFAULT_POINTS = ("llama70b:16,llama70b:32,llama70b:512,llama70b:1:nogroup,llama8b:1,llama8b:4,llama8b:16,"
                  "llama8b:1:nogroup,llama8b:2048,llama8b:8192")


def sweep_points(args, held: dict) -> list:
    """Time the --points list (workload:m, ...) with the same steps, warmup and
    grouping as the headline. held maps (workload, layers, tp) to built weights (the
    headline's at first); weights stay allocated until the end of the run: after a
    large free (the 70B sweep's 29 GB) the 8B decode sweeps measured 4% slower on the
    same, still allocated, 8B weights, and both models together take 32 GB of the
    device's 288."""
    import argparse as _ap
    spec = args.points
    if spec == "auto":
        headline = (args.workload == "llama70b" and args.m == 1 and args.layers == 80 and args.with_quant == "none"
                    and args.tp == 1)
        spec = DEFAULT_POINTS if headline else "none"
    if spec == "none":
        return []
    out = []
    for item in spec.split(","):
        wl, m, *flags = item.split(":")
        sub = _ap.Namespace(**vars(args))
        sub.workload, sub.m = wl, int(m)
        if flags:
            if flags != ["nogroup"]:
                raise ValueError(f"point {item}: the only flag is nogroup")
            sub.no_group = True
        sub.layers = 80 if wl == "llama70b" else 32
        key = (sub.workload, sub.layers, sub.tp)
        if key not in held:
            held[key] = build_weights(sub.workload, sub.layers, sub.tp)
        log(f"point {item}")
        r = run_gemm(sub, held[key])
        mfma_bound = sub.m >= PREFILL_M
        name = gemm_workload_name(sub)
        out.append({"workload": name, "m": sub.m, "value": round(r["tflops"] if mfma_bound else r["value"], 2),
                    "unit": "TFLOP/s" if mfma_bound else "GB/s", "ms_per_step": round(r["ms"], 4),
                    "launches_per_step": r["launches"],
                    "gbs": round(r["value"], 2), "tflops": round(r["tflops"], 3),
                    "roofline": roofline_of(r, mfma_bound, name)})
    return out


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--m", type=int, default=1, help="tokens per projection")
    p.add_argument("--workload", choices=["llama70b", "llama8b", "quant", "copy", "read", "readsweep", "mfma"],
                   default="llama70b")
    p.add_argument("--layers", type=int, default=None, help="layers in the sweep (default 80 for llama70b, 32 for llama8b)")
    p.add_argument("--model", choices=["llama70b", "llama8b"], default=None,
                   help="the sweep whose launch sizes --workload readsweep reads (default llama70b; the GEMM "
                        "workloads name their model themselves)")
    p.add_argument("--no-graph", action="store_true", help="launch eagerly instead of replaying a HIP graph")
    p.add_argument("--with-quant", choices=["none", "separate", "fused"], default="none",
                   help="time the activation quantization in the step: a quantizer launch before each GEMM "
                        "(separate) or inside it (fused, launch_iq3_s_matmul_quantize); default: activations "
                        "quantized once before timing, as the reference times the matmul alone")
    p.add_argument("--no-group", action="store_true",
                   help="one launch per projection (default: q/k/v and gate/up share a launch)")
    p.add_argument("--chain", type=int, default=0,
                   help="1..4 tokens: run each run of this many consecutive launches (at most 16) as one "
                        "persistent chained launch, each launch waiting for the one before it")
    p.add_argument("--chain-waves", type=int, default=0, help="waves per workgroup of the chained launches")
    p.add_argument("--chain-tpw", type=int, default=0, help="16-row tiles per workgroup of the chained launches")
    p.add_argument("--points", default="auto",
                   help="further workload:m[:nogroup] points timed after the headline, comma-separated, or 'none' "
                        f"(auto: {DEFAULT_POINTS} when the headline is the default 70B M=1 sweep)")
    p.add_argument("--tp", type=int, default=1,
                   help="sweep one GPU's shard of a tensor-parallel layer: N/tp rows of q/k/v and gate/up, "
                        "K/tp columns of o and down (the collectives are not part of this single-GPU build)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    args = p.parse_args(argv)
    if args.model is None:
        args.model = args.workload if args.workload in ("llama70b", "llama8b") else "llama70b"
    if args.layers is None:
        args.layers = 32 if args.model == "llama8b" else 80
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus})",
              file=sys.stderr)
        return 2
    rank = int(os.environ.get("RANK", "0"))
    points = []

    import torch
    from mambo_amd import _native
    _native.lib()
    log(f"device {torch.cuda.get_device_name(0)} ({_native.device_arch()})")

    dtype = "fp8-e4m3 x iq3_s, f32 accumulate"
    data = "synthetic (counter-based IQ3_S blocks, bf16 ~N(0,1) activations)"
    if args.workload == "copy":
        r = run_copy(args)
        metric = "plain device copy GB/s (HBM counter calibration)"
        workload = f"copy {COPY_BYTES} bytes"
        config = {"workload": workload}
        dtype, data = "u8", "synthetic bytes"
    elif args.workload == "read":
        r = run_read(args)
        metric = "plain device read GB/s (16-byte loads, read ceiling)"
        workload = f"read {COPY_BYTES} bytes"
        config = {"workload": workload}
        dtype, data = "u8", "synthetic bytes"
    elif args.workload == "readsweep":
        r = run_readsweep(args)
        model = "llama3-8b" if args.model == "llama8b" else "llama3-70b"
        metric = f"plain device read GB/s over the {model} sweep's launch sizes (weight-stream ceiling)"
        grouping = "one launch per projection" if args.no_group else "q/k/v and gate/up grouped per launch"
        shard = f" (one GPU's shard at tensor parallelism {args.tp})" if args.tp > 1 else ""
        workload = (f"read the packed IQ3_S bytes of {model}'s {args.layers} layers x 7 linears{shard}, one "
                    f"buffer per launch, {grouping}")
        config = {"workload": workload, "launches_per_step": r["launches"],
                  "bytes_gb": round(r["step_bytes"] / 1e9, 3), "graph": not args.no_graph}
        dtype, data = "u8", "uninitialised device bytes"
    elif args.workload == "mfma":
        r = run_mfma(args)
        metric = "scaled MFMA f8f6f4 16x16x128 TFLOP/s (device check of the MX-FP8 peak)"
        workload = f"mfma_scale_f32_16x16x128_f8f6f4: {MFMA_WORKGROUPS} workgroups x 4 waves x {MFMA_ITERS} x 8 MFMAs"
        config = {"workload": workload}
        dtype, data = "fp8-e4m3 x fp8-e4m3, f32 accumulate", "constant operands"
    elif args.workload == "quant":
        r = run_quant(args)
        metric = "MXFP8 activation quantizer GB/s (bf16 [4096,4096] -> E4M3 + E8M0)"
        workload = "mxfp8 quantize bf16 [4096,4096], 0.1% x100 outliers, 8 rotated inputs"
        config = {"workload": workload, "m": 4096, "k": 4096}
        dtype, data = "bf16 -> fp8-e4m3 + e8m0", "synthetic (bf16 ~N(0,1), 0.1% x100 outliers)"
    else:
        weights = build_weights(args.workload, args.layers, args.tp)
        r = run_gemm(args, weights)
        metric = ("fused IQ3_S x MXFP8 GEMM TFLOP/s vs MX-FP8 MFMA roofline" if args.m >= PREFILL_M else
                  "fused IQ3_S x MXFP8 GEMM weight-stream GB/s vs HBM roofline")
        if args.with_quant != "none":
            metric += " (bf16 activations quantized in the step)"
        workload = gemm_workload_name(args)
        config = {"workload": workload, "m": args.m, "tp_shard": args.tp, "projections_per_step": r["projections"],
                  "launches_per_step": r["launches"], "weight_gb": round(r["weight_bytes"] / 1e9, 3),
                  "tflops": round(r["tflops"], 3), "graph": not args.no_graph}
        points = sweep_points(args, {(args.workload, args.layers, args.tp): weights})
    mfma_bound = (args.workload in ("llama70b", "llama8b") and args.m >= PREFILL_M) or args.workload == "mfma"
    value = r["tflops"] if mfma_bound else r["value"]
    unit = "TFLOP/s" if mfma_bound else "GB/s"
    roofline = roofline_of(r, mfma_bound, workload)
    line = {
        "metric": metric,
        "value": round(value, 2),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": data,
        "config": config,
        "roofline": roofline,
    }
    if points:
        line["points"] = points
    if rank == 0 and not args.no_cpu_baseline:
        log("timing the CPU baseline")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds, unit)
    if rank == 0:
        print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
