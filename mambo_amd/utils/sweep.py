"""A model's projection sweep on the GPU: the seven IQ3_S linears of each decoder layer of
Llama-3 8B or 70B (optionally one GPU's tensor-parallel shard), with synthetic weights
and activations, launched as a decode or prefill step launches them (q/k/v and gate/up,
which read the same input, share a grouped launch) and replayed from a HIP graph.

bench.py times this step; the autotuner's in-sweep mode (kernel_benchmark --sweep)
times each launch shape's candidate configurations inside it, since a launch timed
alone differs from the same launch between its neighbours (the ramp and drain of one
launch overlap the cache and clock state the previous one leaves).
"""

from __future__ import annotations

import sys
import time
from typing import Callable, Sequence

LLAMA70B_LAYER = [("q", 8192, 8192, 0), ("k", 1024, 8192, 0), ("v", 1024, 8192, 0), ("o", 8192, 8192, 1),
                  ("gate", 28672, 8192, 2), ("up", 28672, 8192, 2), ("down", 8192, 28672, 3)]
LLAMA8B_LAYER = [("q", 4096, 4096, 0), ("k", 1024, 4096, 0), ("v", 1024, 4096, 0), ("o", 4096, 4096, 1),
                 ("gate", 14336, 4096, 2), ("up", 14336, 4096, 2), ("down", 4096, 14336, 3)]
MODELS = {"llama70b": (LLAMA70B_LAYER, 80), "llama8b": (LLAMA8B_LAYER, 32)}


def log(msg: str) -> None:
    print(f"[sweep] {msg}", file=sys.stderr, flush=True)


def layer_shapes(model: str, tp: int = 1) -> list:
    """(name, N, K, input slot) of one layer's linears; with tp > 1, one GPU's shard of a
    tensor-parallel layer: the column-parallel projections (q/k/v, gate/up: slots 0 and 2)
    keep N/tp rows, the row-parallel ones (o, down: slots 1 and 3) K/tp columns, whole
    256-weight blocks (their partial outputs would be summed across GPUs)."""
    shapes = MODELS[model][0]
    if tp == 1:
        return shapes
    out = []
    for name, n, k, slot in shapes:
        if slot in (0, 2):
            if n % (16 * tp):
                raise ValueError(f"{name}: N={n} does not split into {tp} shards of whole 16-row tiles")
            out.append((name, n // tp, k, slot))
        else:
            if k % (256 * tp):
                raise ValueError(f"{name}: K={k} does not split into {tp} shards of whole 256-weight blocks")
            out.append((name, n, k // tp, slot))
    return out


def synth_weight(n: int, k: int, seed: int):
    """Packed IQ3_S fields of an [n, k] weight of counter-based synthetic blocks."""
    import torch
    from mambo_amd import _native
    from mambo_amd.utils.iq3_s_weight import prepare_iq3_s_fields
    raw = torch.empty((n, k // 256, 110), dtype=torch.uint8, device="cuda")
    _native.check(_native.lib().mambo_synth_iq3s(seed, k // 256, 0, n, raw.data_ptr(), _native.stream_handle(None)))
    fields = prepare_iq3_s_fields(raw, fields=False)
    del raw
    return fields


def synth_activation(m: int, k: int, seed: int):
    """(E4M3 values, E8M0 scales, bf16 rows) of synthetic ~N(0,1) activations."""
    import torch
    from mambo_amd import _native
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8
    bits = torch.empty(m * k, dtype=torch.int16, device="cuda")
    _native.check(_native.lib().mambo_synth_bf16(seed, 2, 0.0, 0, m * k, bits.data_ptr(), _native.stream_handle(None)))
    rows = bits.view(torch.bfloat16).view(m, k)
    return (*launch_quantize_fp8(rows), rows)


def build_weights(model: str, layers: int, tp: int = 1):
    """The sweep's distinct IQ3_S weights (packed form only), generated on the GPU:
    [(layer, name, n, k, slot, fields)], seed 1000*layer + index in the layer."""
    import torch
    shapes = layer_shapes(model, tp)
    weights = []
    t0 = time.time()
    for layer in range(layers):
        for j, (name, n, k, slot) in enumerate(shapes):
            weights.append((layer, name, n, k, slot, synth_weight(n, k, seed=1000 * layer + j)))
        if layer % 10 == 9:
            log(f"prepared {layer + 1}/{layers} layers ({time.time() - t0:.1f} s)")
    torch.cuda.synchronize()
    return weights


def build_launches(weights, m: int, no_group: bool = False):
    """Activations, outputs and the launch list of one step at m tokens. Each launch is
    (names, [(n, k, fields, out)], (x_values, x_scales, bf16 rows)); projections of one
    layer that read the same input (q/k/v, gate/up) share a launch unless no_group."""
    import torch
    acts, outs, launches = {}, {}, []
    for layer, name, n, k, slot, fields in weights:
        if slot not in acts:
            acts[slot] = synth_activation(m, k, seed=1 + slot)
        key = (name, n, k)
        if key not in outs:
            outs[key] = torch.empty((m, n), dtype=torch.float32, device="cuda")
        proj = (n, k, fields, outs[key])
        if not no_group and launches and launches[-1][3] == (layer, slot) and len(launches[-1][1]) < 4:
            launches[-1][0].append(name)
            launches[-1][1].append(proj)
        else:
            launches.append(([name], [proj], acts[slot], (layer, slot)))
    torch.cuda.synchronize()
    return [(names, projs, act) for names, projs, act, _ in launches]


def launch_shape(projs) -> tuple[int, int]:
    """(N summed over the launch's projections, K): the shape a launch configuration is
    chosen for (launch_iq3_s_fp8_matmul_grouped passes the summed N)."""
    return sum(n for n, _, _, _ in projs), projs[0][1]


def make_step(launches, configs: Sequence[dict], with_quant: str = "none", chain: int = 0,
              chain_waves: int = 0, chain_tpw: int = 0) -> Callable[[], None]:
    """One step: every launch with its configuration. with_quant: "none" (MXFP8 rows
    prepared beforehand), "separate" (a quantizer launch before each GEMM) or "fused"
    (the rows quantized inside the GEMM). chain > 0 (1..4 tokens): consecutive runs of
    `chain` launches go to launch_iq3_s_fp8_matmul_chain as one persistent launch each,
    every launch still reading its activations only after the one before it has stored
    all its outputs (configs are then unused; chain_waves: 4, 8 or 16, chain_tpw: tiles per
    workgroup, 0 = the library's);
    "fused" hands the chain the bf16 rows, which it quantizes in the kernel."""
    from mambo_amd.kernels.iq3_s_fp8 import (ChainLaunch, launch_iq3_s_fp8_matmul, launch_iq3_s_fp8_matmul_chain,
                                             launch_iq3_s_fp8_matmul_grouped, launch_iq3_s_matmul_quantize,
                                             new_chain_sync)
    from mambo_amd.kernels.quantize_fp8 import launch_quantize_fp8

    if chain:
        if with_quant == "separate":
            raise ValueError("a chain quantizes inside the kernel (with_quant fused) or takes MXFP8 rows (none)")
        descs = []
        for _, projs, (xv, xs, rows) in launches:
            if with_quant == "fused":
                descs.append(ChainLaunch(rows, [p[2] for p in projs], outs=[p[3] for p in projs]))
            else:
                descs.append(ChainLaunch(xv, [p[2] for p in projs], x_scales=xs, outs=[p[3] for p in projs]))
        # runs of consecutive launches with the same K, at most `chain` each: the chained
        # kernel's LDS holds the rows of its longest K for every workgroup, so a long-K launch
        # (the down projection) would cut the residency of all the others; it runs alone
        chunks, i = [], 0
        while i < len(descs):
            j = i + 1
            k = launches[i][1][0][1]
            while j < len(descs) and j - i < chain and launches[j][1][0][1] == k:
                j += 1
            chunks.append((i, j))
            i = j
        sync = new_chain_sync()  # the chained calls are ordered on one stream: one set of words

        def chained():
            for i, j in chunks:
                if j - i == 1:
                    single_launch(i)
                else:
                    launch_iq3_s_fp8_matmul_chain(descs[i:j], waves=chain_waves, tiles_per_workgroup=chain_tpw,
                                                  sync=sync)

        def single_launch(i):
            (_, projs, (xv, xs, rows)), cfg = launches[i], configs[i]
            if with_quant == "fused":
                launch_iq3_s_matmul_quantize(rows, [p[2] for p in projs], config=cfg, outs=[p[3] for p in projs])
            elif len(projs) == 1:
                launch_iq3_s_fp8_matmul(xv, xs, projs[0][2], config=cfg, out=projs[0][3])
            else:
                launch_iq3_s_fp8_matmul_grouped(xv, xs, [p[2] for p in projs], config=cfg,
                                                outs=[p[3] for p in projs])

        chained.sync = sync
        return chained

    def step():
        for (_, projs, (xv, xs, rows)), cfg in zip(launches, configs):
            if with_quant == "fused":
                launch_iq3_s_matmul_quantize(rows, [p[2] for p in projs], config=cfg, outs=[p[3] for p in projs])
                continue
            if with_quant == "separate":
                launch_quantize_fp8(rows, out=(xv, xs))
            if len(projs) == 1:
                launch_iq3_s_fp8_matmul(xv, xs, projs[0][2], config=cfg, out=projs[0][3])
            else:
                launch_iq3_s_fp8_matmul_grouped(xv, xs, [p[2] for p in projs], config=cfg,
                                                outs=[p[3] for p in projs])

    return step


def capture(step: Callable[[], None]):
    """A HIP graph of one step, captured on a side stream."""
    import torch
    stream = torch.cuda.current_stream()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            step()
    stream.wait_stream(side)
    return graph


def time_replays(replay: Callable[[], None], steps: int, warmup: int) -> tuple[float, float]:
    """(ms per step from HIP events, wall-clock s of the timed loop) over `steps` replays
    after `warmup` untimed ones, on the current stream."""
    import torch
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        replay()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps, time.perf_counter() - t0
