"""Autotuning and benchmark command for the gfx950 projection kernels.

Mirror of src/python/mambo/utils/kernel_benchmark.py: each kernel module supplies
benchmark cases; this module searches each case's launch configurations, re-times the
winner with the reference's three timers (mean_us with a sync per launch, batched_us,
event_us; 5 warm-up and 20 iterations, kernel_benchmark.py:56-94) and reports it.

Candidates are timed as the projections run in a decode step: each case rotates over
enough copies of its weight that every launch streams the weight from HBM (the
reference re-launches on one weight, which the 256 MB memory-side cache then holds for
the smaller projections), and the launches are replayed from a captured HIP graph, so
that a 5 us kernel is not timed as the host's launch rate. The library default is one
of the candidates; a tuned entry replaces it only when it is faster by ``min_gain``.

    python -m mambo_amd.utils.kernel_benchmark iq3_s_fp8 --model M.gguf --weight-name NAME
    python -m mambo_amd.utils.kernel_benchmark iq3_s_fp8 --synthetic 4096 4096 [--write-table]
    python -m mambo_amd.utils.kernel_benchmark iq3_s_fp8 --sweep llama70b --tokens 1 16 [--no-group] [--write-table]

``--sweep`` tunes every launch shape of a Llama-3 projection sweep inside the sweep
itself, replayed from a HIP graph, where the step time decides (sweep_tune).

The reference copies winners into BEST_CONFIGS by hand (kernels/AGENTS.md:27); here
``--write-table`` stores them per shape in mambo_amd/kernels/tuned_gfx950.json, which
launch_iq3_s_fp8_matmul consults first.
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from time import perf_counter
from typing import Any, Callable, Sequence

import torch

from mambo_amd.utils.gguf import read_block_matrix

Config = dict[str, Any]


@dataclass(frozen=True)
class BenchmarkCase:
    name: str
    stream: Any
    launch: Callable[[Config], None]
    search_space: Sequence[Config]
    summary_keys: tuple[str, ...] = ()
    # Per-invocation state reset, included in reported timings after tuning.
    before_launch_fn: Callable[[Config], None] | None = None
    key: str = ""
    # launches per timed graph: `launch` cycles over this many weight copies
    rotation: int = 1
    # the library's own configuration for the shape (a member of search_space), if any
    default: Config | None = None


@dataclass
class TuneResult:
    case: str
    key: str
    best: Config
    mean_us: float
    batched_us: float
    event_us: float
    tuner_us: float
    successes: list = field(default_factory=list)
    failures: list = field(default_factory=list)
    default_us: float | None = None  # the library default's time (None: not a candidate)
    default_of: Config | None = None

    @property
    def is_default(self) -> bool:
        """The library default won (or no candidate beat it by the required margin)."""
        return self.default_us is not None and self.best == self.default_of


def _graph_time(stream, fn, launches: int, target_us: float = 2000.0, max_reps: int = 20) -> float:
    """Average time of `fn` over `launches` calls captured in one HIP graph, replayed
    until about `target_us` has been timed."""
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(launches):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    one = _time_events(stream, graph.replay, 1)
    reps = max(1, min(max_reps, math.ceil(target_us / max(one, 1e-3))))
    us = _time_events(stream, graph.replay, reps) / launches
    del graph
    return us


def _time_events(stream, fn, iters: int) -> float:
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(iters):
        fn()
    stop.record(stream)
    stop.synchronize()
    return start.elapsed_time(stop) * 1000.0 / iters


def _host_time(stream, fn, *, drain_each: bool, warmup: int = 5, iters: int = 20) -> float:
    """Host wall-clock microseconds per call of `fn` over `iters` calls after `warmup`
    untimed ones. drain_each: the stream is synchronized after every call (the
    reference's mean_us, launch + completion latency); otherwise once after the batch
    (batched_us, throughput with queued launches)."""
    def batch(calls: int) -> None:
        for _ in range(calls):
            fn()
            if drain_each:
                stream.synchronize()
        stream.synchronize()

    batch(warmup)
    t0 = perf_counter()
    batch(iters)
    return (perf_counter() - t0) * 1e6 / iters


def _time_config(case: BenchmarkCase, config: Config, *, warmup: int, iters: int, graph: bool) -> float:
    def once() -> None:
        if case.before_launch_fn is not None:
            case.before_launch_fn(config)
        case.launch(config)
    for _ in range(max(warmup, 1)):
        once()
    torch.cuda.synchronize()
    if graph:
        return _graph_time(case.stream, once, max(case.rotation, 1))
    return _time_events(case.stream, once, iters)


def exhaustive_search(case: BenchmarkCase, *, warmup: int = 2, iters: int = 10, graph: bool = True):
    """Time every configuration of the case; failures (invalid configs) are recorded.
    Warm-up launches run eagerly (an invalid configuration raises there, before any
    capture); with `graph` the timed launches are `case.rotation` launches replayed
    from a HIP graph, else `iters` eager launches."""
    successes, failures = [], []
    for config in case.search_space:
        try:
            successes.append((config, _time_config(case, config, warmup=warmup, iters=iters, graph=graph)))
        except (ValueError, RuntimeError) as exc:
            failures.append((config, str(exc)))
    if not successes:
        raise RuntimeError(f"{case.name}: no configuration ran ({failures[:3]})")
    return successes, failures


def _versus_default(case: BenchmarkCase, best: Config, *, graph: bool, rounds: int = 2) -> tuple[float, float]:
    """Best-of-`rounds` times of the library default and `best`, timed alternately, so
    that neither is favoured by its place in the search (clock ramp, cache state)."""
    d_us, b_us = float("inf"), float("inf")
    for _ in range(rounds):
        d_us = min(d_us, _time_config(case, case.default, warmup=2, iters=10, graph=graph))
        b_us = min(b_us, _time_config(case, best, warmup=2, iters=10, graph=graph))
    return d_us, b_us


def mini_benchmark(cases: Sequence[BenchmarkCase], *, quiet: bool = False, graph: bool = True,
                   min_gain: float = 0.03) -> list[TuneResult]:
    """Tune each case, then time the winner with any per-launch reset (kernel_benchmark.py:41-100).
    The case's library default stays the answer unless the search's winner, re-timed
    alternately with it, is at least `min_gain` (a fraction) faster."""
    results = []
    for case in cases:
        successes, failures = exhaustive_search(case, graph=graph)
        best, tuner_us = min(successes, key=lambda item: item[1])
        default_us = next((us for config, us in successes if config == case.default), None)
        if default_us is not None:
            if best != case.default:
                default_us, tuner_us = _versus_default(case, best, graph=graph)
            if tuner_us > default_us * (1.0 - min_gain):
                best, tuner_us = case.default, default_us

        def launch_once() -> None:
            if case.before_launch_fn is not None:
                case.before_launch_fn(best)
            case.launch(best)

        mean_us = _host_time(case.stream, launch_once, drain_each=True)
        batched_us = _host_time(case.stream, launch_once, drain_each=False)
        event_us = _time_events(case.stream, launch_once, 20)
        result = TuneResult(case.name, case.key, dict(best), mean_us, batched_us, event_us, tuner_us,
                            successes, failures, default_us,
                            dict(case.default) if case.default is not None else None)
        results.append(result)
        if not quiet:
            versus = "" if default_us is None else (
                " (library default)" if result.is_default else f" (library default {default_us:.3f})")
            print(f"{case.name}: best_config={best}, "
                  f"mean_us={mean_us:.3f}, batched_us={batched_us:.3f}, "
                  f"event_us={event_us:.3f}, "
                  f"tuner_us={tuner_us:.3f}{versus} (warmup=5, iterations=20), "
                  f"candidates={len(successes)} passed/{len(failures)} failed", flush=True)
            if case.summary_keys:
                by_group: dict[tuple[Any, ...], float] = {}
                for config, us in successes:
                    group = tuple(config.get(key, 0) for key in case.summary_keys)
                    by_group[group] = min(by_group.get(group, float("inf")), us)
                print(f"  best latency by {case.summary_keys} (us): {by_group}")
    return results


def write_tuned_table(results: Sequence[TuneResult], path: Path, arch: str) -> None:
    """Merge the winners into the table; a shape whose library default won loses any
    entry it had."""
    table = json.loads(path.read_text()) if path.exists() else {}
    entries = table.setdefault(arch, {})
    for r in results:
        if not r.key:
            continue
        if r.is_default:
            entries.pop(r.key, None)
        else:
            entries[r.key] = r.best
    path.write_text(json.dumps(table, indent=1, sort_keys=True) + "\n")


# Sweeps smaller than this are partly held by the 256 MB memory-side cache from one
# replay to the next (the 8B sweep on 4 layers rated a q/k/v entry 10% slow that the
# full 32-layer sweep runs 1% faster with).
SWEEP_MIN_BYTES = 1 << 30


def _rel_l2(out: torch.Tensor, ref: torch.Tensor) -> float:
    return float(torch.linalg.vector_norm(out - ref) / torch.linalg.vector_norm(ref).clamp_min(1e-30))


def sweep_tune(model: str, tokens: Sequence[int], *, layers: int | None = None, tp: int = 1, steps: int = 10,
               warmup: int = 2, min_gain: float = 0.01, rounds: int = 2, rtol: float = 1e-4,
               quiet: bool = False, progress: int = 10, no_group: bool = False) -> list[TuneResult]:
    """Tune each launch shape of a model's projection sweep inside the sweep.

    For each token count, the sweep's launches (mambo_amd.utils.sweep) are replayed from
    a HIP graph with one launch shape's configuration set to each of its candidates and
    every other shape at its current choice (the tuned table's, then the winners of the
    shapes tuned before it), and the step time is what decides: a launch between its
    neighbours differs from one timed alone, whose clocks and caches no earlier launch
    has touched. A candidate whose outputs differ from the library default's by more than
    `rtol` (relative L2) counts as a failure. The winner, re-timed alternately with the
    library default for `rounds` rounds, replaces it only if the step is at least
    `min_gain` (a fraction of the step time) faster. tuner_us and default_us are step
    times; mean_us, batched_us and event_us time one launch of the shape alone with the
    reference's three timers. Unless quiet, a progress line (candidates done, failures,
    the best so far) is printed every `progress` candidates of a shape (0: none).
    no_group: one launch per projection, as a caller of launch_iq3_s_fp8_matmul runs a
    layer (the shapes of k, v, gate and up alone), instead of q/k/v and gate/up grouped."""
    from mambo_amd.kernels.iq3_s_fp8 import default_config, gemm_search_space, select_config, tuned_key
    from mambo_amd.utils.sweep import MODELS, build_launches, build_weights, capture, launch_shape, make_step, \
        time_replays

    layers = MODELS[model][1] if layers is None else layers
    weights = build_weights(model, layers, tp)
    weight_bytes = sum(f.packed.numel() for *_, f in weights)
    if weight_bytes < SWEEP_MIN_BYTES and not quiet:
        print(f"note: the sweep's weights take {weight_bytes / 1e6:.0f} MB; below "
              f"{SWEEP_MIN_BYTES / 1e9:.0f} GB the 256 MB memory-side cache holds part of them between "
              "replays and the timings favour configurations that re-read weights", flush=True)
    stream = torch.cuda.current_stream()
    results = []
    for m in tokens:
        launches = build_launches(weights, m, no_group)
        shapes = [launch_shape(projs) for _, projs, _ in launches]
        keys = list(dict.fromkeys(shapes))
        chosen = {key: select_config(m, *key) for key in keys}
        default = default_config(m)
        make_step(launches, [default] * len(launches))()
        torch.cuda.synchronize()
        outputs = {key: list({id(p[3]): p[3] for (_, projs, _), s in zip(launches, shapes) if s == key
                              for p in projs}.values()) for key in keys}
        refs = {key: [o.clone() for o in outs] for key, outs in outputs.items()}

        def step_us(key, config) -> float:
            configs = [config if s == key else chosen[s] for s in shapes]
            step = make_step(launches, configs)
            step()  # eager first: an invalid configuration raises here, before capture
            torch.cuda.synchronize()
            for out, ref in zip(outputs[key], refs[key]):
                err = _rel_l2(out, ref)
                if not err <= rtol:
                    raise RuntimeError(f"output differs from the library default's (rel-L2 {err:.3g})")
            graph = capture(step)
            ms, _ = time_replays(graph.replay, steps, warmup)
            del graph
            return ms * 1e3

        for key in keys:
            successes, failures = [], []
            space = gemm_search_space(m, *key)
            for i, config in enumerate(space):
                try:
                    successes.append((config, step_us(key, config)))
                except (ValueError, RuntimeError) as exc:
                    failures.append((config, str(exc)))
                # one line per `progress` candidates (each is an eager step, a capture and
                # the replays), so a long search over a large sweep keeps reporting
                if not quiet and progress and ((i + 1) % progress == 0 or i + 1 == len(space)):
                    lead = min(successes, key=lambda item: item[1]) if successes else None
                    best_text = f"best so far {lead[0]} at {lead[1]:.1f} us" if lead else "none ran yet"
                    print(f"[tune] M={m} N={key[0]} K={key[1]}: candidate {i + 1}/{len(space)}, "
                          f"{len(failures)} failed, {best_text}", flush=True)
            if not successes:
                raise RuntimeError(f"M={m} {key}: no configuration ran ({failures[:3]})")
            best, tuner_us = min(successes, key=lambda item: item[1])
            default_us = next((us for config, us in successes if config == default), None)
            if default_us is not None:
                if best != default:
                    default_us = tuner_us = float("inf")
                    for _ in range(rounds):
                        default_us = min(default_us, step_us(key, default))
                        tuner_us = min(tuner_us, step_us(key, best))
                if tuner_us > default_us * (1.0 - min_gain):
                    best, tuner_us = default, default_us
            chosen[key] = best
            one = make_step([launches[shapes.index(key)]], [best])
            mean_us = _host_time(stream, one, drain_each=True)
            batched_us = _host_time(stream, one, drain_each=False)
            event_us = _time_events(stream, one, 20)
            where = f"the {model} sweep{', one launch per projection' if no_group else ''}"
            result = TuneResult(f"M={m} N={key[0]} K={key[1]} in {where}", tuned_key(*key, m), dict(best),
                                mean_us, batched_us, event_us, tuner_us, successes, failures, default_us,
                                dict(default))
            results.append(result)
            if not quiet:
                versus = "" if default_us is None else (
                    " (library default)" if result.is_default else f" (library default {default_us:.1f})")
                print(f"{result.case}: best_config={best}, step_us={tuner_us:.1f}{versus}, one launch alone: "
                      f"mean_us={mean_us:.3f}, batched_us={batched_us:.3f}, event_us={event_us:.3f}, "
                      f"candidates={len(successes)} passed/{len(failures)} failed", flush=True)
        del launches, outputs, refs
        torch.cuda.empty_cache()
    return results


def load_gguf_weight(model: Path, weight_name: str, expected_type: str) -> torch.Tensor:
    """The named 2-D block-quantized GGUF tensor as u8 [N, K/block_elements, block_bytes]
    on the current GPU (the reference's load_gguf_weight, kernel_benchmark.py:103-122;
    same ValueErrors). The bytes are read on the host by gguf.read_block_matrix."""
    return torch.from_numpy(read_block_matrix(model, weight_name, expected_type)).to("cuda")


def synthetic_weight(n: int, k: int, seed: int = 0) -> torch.Tensor:
    """Random IQ3_S blocks u8 [N, K/256, 110] generated on the GPU (counter-based)."""
    from mambo_amd import _native
    raw = torch.empty((n, k // 256, 110), dtype=torch.uint8, device="cuda")
    _native.check(_native.lib().mambo_synth_iq3s(seed, k // 256, 0, n, raw.data_ptr(),
                                                 _native.stream_handle(None)), "synth_iq3s")
    return raw


# Add a kernel module and an entry here for each new benchmark.
_BENCHMARKS = {
    "iq3_s_fp8": ("iq3_s", "mambo_amd.kernels.iq3_s_fp8", "make_benchmark_cases"),
}


def benchmark_main(argv: Sequence[str] | None = None) -> list[TuneResult]:
    parser = argparse.ArgumentParser(description="Autotune a gfx950 projection kernel")
    parser.add_argument("kernel", choices=sorted(_BENCHMARKS))
    parser.add_argument("--model", type=Path, help="GGUF model path")
    parser.add_argument("--weight-name", help="tensor name in the GGUF model")
    parser.add_argument("--synthetic", nargs=2, type=int, metavar=("N", "K"), action="append",
                        help="use a random IQ3_S weight of this shape instead of a GGUF tensor (repeatable)")
    parser.add_argument("--sweep", choices=["llama70b", "llama8b"],
                        help="tune every launch shape of this model's projection sweep inside the replayed sweep "
                             "(iq3_s_fp8 only) instead of one weight at a time")
    parser.add_argument("--layers", type=int, help="layers of the --sweep (default: all of the model's)")
    parser.add_argument("--tp", type=int, default=1, help="--sweep one GPU's shard at this tensor parallelism")
    parser.add_argument("--steps", type=int, default=10, help="timed sweep replays per --sweep candidate")
    parser.add_argument("--no-group", action="store_true",
                        help="--sweep with one launch per projection (as launch_iq3_s_fp8_matmul callers run a layer)")
    parser.add_argument("--tokens", type=int, nargs="+", default=[4, 128], help="token counts M to tune")
    parser.add_argument("--write-table", action="store_true", help="store winners in the tuned table")
    parser.add_argument("--table", type=Path, help="tuned table to write (default: the one the launcher reads)")
    parser.add_argument("--rotate-mib", type=int, default=512,
                        help="weight copies per case to at least this many MiB (at most 64 copies)")
    parser.add_argument("--min-gain", type=float, default=None,
                        help="fraction by which a candidate must beat the library default (default 0.03 of the "
                             "launch time; with --sweep 0.01 of the step time)")
    parser.add_argument("--no-graph", action="store_true", help="time candidates by eager launches")
    args = parser.parse_args(argv)

    expected_type, kernel_module, factory = _BENCHMARKS[args.kernel]
    if args.sweep:
        if args.kernel != "iq3_s_fp8" or args.no_graph or args.synthetic or args.model:
            parser.error("--sweep tunes iq3_s_fp8 from replayed graphs of its own synthetic weights")
        module = importlib.import_module(kernel_module)
        results = sweep_tune(args.sweep, args.tokens, layers=args.layers, tp=args.tp, steps=args.steps,
                             min_gain=0.01 if args.min_gain is None else args.min_gain, no_group=args.no_group)
        if args.write_table:
            from mambo_amd import _native
            write_tuned_table(results, args.table or module.TUNED_PATH, _native.device_arch())
        return results
    if args.min_gain is None:
        args.min_gain = 0.03
    if args.synthetic:
        sources = [lambda shape=shape: synthetic_weight(*shape) for shape in args.synthetic]
    elif args.model and args.weight_name:
        sources = [lambda: load_gguf_weight(args.model, args.weight_name, expected_type)]
    else:
        parser.error("give --model and --weight-name, or --synthetic N K")
    module = importlib.import_module(kernel_module)
    results = []
    for source in sources:
        cases = getattr(module, factory)(source(), tuple(args.tokens), rotate_bytes=args.rotate_mib << 20)
        results += mini_benchmark(cases, graph=not args.no_graph, min_gain=args.min_gain)
        del cases
        torch.cuda.empty_cache()
    if args.write_table:
        from mambo_amd import _native
        write_tuned_table(results, args.table or module.TUNED_PATH, _native.device_arch())
    return results


if __name__ == "__main__":
    benchmark_main()
