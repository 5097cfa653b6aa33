"""Summaries of rocprofv3 CSV output for the kernels of this package.

Two reports, both plain text meant to be committed next to the numbers they back:

* ``stats``: the per-kernel duration table of a ``rocprofv3 --kernel-trace --stats
  --output-format csv`` run (``*_kernel_stats.csv``), plus a combined row for every
  kernel whose name contains ``--family`` (template instantiations of one kernel).
* ``window``: from the per-dispatch ``*_kernel_trace.csv`` of the same kind of run,
  the last ``--last`` dispatches whose kernel name contains ``--family`` (the timed
  replays of a benchmark, which come after its eager, check and warm-up launches): their
  average duration, their span from first start to last end, and the rate that the
  algorithmic work per launch gives over each.
* ``mfma``: MFMA counters per dispatch of a ``--pmc`` run (``SQ_VALU_MFMA_BUSY_CYCLES``,
  ``SQ_INSTS_VALU_MFMA_MOPS_F8``, ``GRBM_GUI_ACTIVE``) and optionally of a second run of
  rocprofiler's derived ``MfmaUtil``: MFMA busy fraction over all SIMDs and executed F8
  MFMA flops against the algorithmic ones. The CSV's ``GRBM_GUI_ACTIVE`` is the sum over
  the XCDs (MfmaUtil's formula takes the maximum), so the busy fraction divides by the
  per-XCD mean.
* ``points``: the same three figures for every point of one ``bench.py`` run (the headline
  and its ``points`` list, read from the JSON line the run printed): the kernel trace, the
  ``FETCH_SIZE`` / ``WRITE_SIZE`` runs and the MFMA counter run of the bench command are
  each cut into the points' steps (see ``segment_points``), and one Markdown table plus one
  traffic record per point (read by ``bench.py`` for ``roofline.traffic``) are written.
* ``traffic``: HBM bytes per dispatch from two ``--pmc`` runs (``FETCH_SIZE``, then
  ``WRITE_SIZE``) of a workload, each scaled by what the same counter reads for the plain
  copy kernel (``mambo_copy_bytes``) over a known number of bytes in two more runs. The
  counters are read per dispatch and averaged over the dispatches whose kernel name
  contains ``--family``. Writes a Markdown report and a small JSON record that the bench
  reads for ``roofline.traffic``.

    python -m mambo_amd.utils.rocprof_summary stats DIR --family gemm_stream_kernel \\
        --command "..." --out profiles/x.md
    python -m mambo_amd.utils.rocprof_summary traffic --fetch DIR --write DIR \\
        --calib-fetch DIR --calib-write DIR --copy-bytes N --family gemm_stream_kernel \\
        --algorithmic-bytes B --workload NAME --command "..." --out profiles/x
"""

from __future__ import annotations

import argparse
import csv
import json
from pathlib import Path


def _one(directory: str, suffix: str) -> Path:
    found = sorted(Path(directory).rglob(f"*{suffix}"))
    if not found:
        raise FileNotFoundError(f"no *{suffix} under {directory}")
    if len(found) > 1:
        raise ValueError(f"several *{suffix} under {directory}: {[str(p) for p in found]}")
    return found[0]


def kernel_stats(directory: str) -> list[dict]:
    """Rows of the kernel_stats CSV: name, calls, total/avg/min/max ns."""
    rows = []
    with open(_one(directory, "_kernel_stats.csv"), newline="") as f:
        for r in csv.DictReader(f):
            rows.append({"name": r["Name"], "calls": int(r["Calls"]), "total_ns": float(r["TotalDurationNs"]),
                         "avg_ns": float(r["AverageNs"]), "min_ns": float(r["MinNs"]),
                         "max_ns": float(r["MaxNs"]), "pct": float(r["Percentage"])})
    return rows


def counter_per_dispatch(directory: str, counter: str, family: str) -> list[float]:
    """Values of `counter` for every dispatch whose kernel name contains `family`."""
    values = []
    with open(_one(directory, "_counter_collection.csv"), newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter and family in r["Kernel_Name"]:
                values.append(float(r["Counter_Value"]))
    if not values:
        raise ValueError(f"no {counter} records for kernels matching {family!r} under {directory}")
    return values


def _short(name: str, width: int = 96) -> str:
    return name if len(name) <= width else name[:width - 3] + "..."


def stats_report(args) -> None:
    rows = kernel_stats(args.dir)
    lines = [f"# rocprofv3 kernel statistics: {args.title}", "", "Command:", "", "```", args.command, "```", ""]
    lines += ["| kernel | calls | total ms | avg us | min us | max us | % |", "|---|---|---|---|---|---|---|"]
    for r in rows[:args.top]:
        lines.append(f"| `{_short(r['name'])}` | {r['calls']} | {r['total_ns'] / 1e6:.3f} | {r['avg_ns'] / 1e3:.3f} | "
                     f"{r['min_ns'] / 1e3:.3f} | {r['max_ns'] / 1e3:.3f} | {r['pct']:.2f} |")
    if args.family:
        fam = [r for r in rows if args.family in r["name"]]
        calls = sum(r["calls"] for r in fam)
        total = sum(r["total_ns"] for r in fam)
        if calls:
            lines += ["", f"All `{args.family}` instantiations: {calls} calls, {total / 1e6:.3f} ms, "
                          f"average {total / calls / 1e3:.3f} us per launch."]
    Path(args.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def traffic_report(args) -> None:
    def mean(v):
        return sum(v) / len(v)

    fetch = counter_per_dispatch(args.fetch, "FETCH_SIZE", args.family)
    write = counter_per_dispatch(args.write, "WRITE_SIZE", args.family)
    cal_fetch = mean(counter_per_dispatch(args.calib_fetch, "FETCH_SIZE", args.calib_family))
    cal_write = mean(counter_per_dispatch(args.calib_write, "WRITE_SIZE", args.calib_family))
    f_factor = args.copy_bytes / cal_fetch  # bytes per counter unit
    w_factor = args.copy_bytes / cal_write
    fetch_b = mean(fetch) * f_factor
    write_b = mean(write) * w_factor
    traffic = fetch_b + write_b
    rec = {
        "workload": args.workload, "kernel_family": args.family, "dispatches": len(fetch),
        "fetch_size_avg": mean(fetch), "write_size_avg": mean(write),
        "calibration": {"copy_bytes": args.copy_bytes, "fetch_size": cal_fetch, "write_size": cal_write,
                        "fetch_bytes_per_unit": f_factor, "write_bytes_per_unit": w_factor},
        "fetch_bytes_per_launch": fetch_b, "write_bytes_per_launch": write_b,
        "traffic_bytes_per_launch": traffic,
        "algorithmic_bytes_per_launch": args.algorithmic_bytes,
        "traffic_over_algorithmic": traffic / args.algorithmic_bytes if args.algorithmic_bytes else None,
        "command": args.command,
    }
    out = Path(args.out)
    out.with_suffix(".json").write_text(json.dumps(rec, indent=1) + "\n")
    lines = [f"# HBM traffic per dispatch: {args.workload}", "", "Commands:", "", "```", args.command, "```", "",
             f"Kernel family `{args.family}`, {len(fetch)} dispatches per counter run.", "",
             "| | counter avg | bytes per counter unit (copy calibration) | bytes per launch |", "|---|---|---|---|",
             f"| FETCH_SIZE | {mean(fetch):.1f} | {f_factor:.1f} | {fetch_b:,.0f} |",
             f"| WRITE_SIZE | {mean(write):.1f} | {w_factor:.1f} | {write_b:,.0f} |", "",
             f"Calibration: `mambo_copy_bytes` over {args.copy_bytes:,} bytes reads FETCH_SIZE {cal_fetch:.1f} "
             f"and WRITE_SIZE {cal_write:.1f}.", "",
             f"Traffic {traffic:,.0f} B per launch against {args.algorithmic_bytes:,} algorithmic bytes "
             f"(ratio {rec['traffic_over_algorithmic']:.3f})."]
    out.with_suffix(".md").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def kernel_trace(directory: str) -> list[dict]:
    """Dispatch rows of the kernel_trace CSV in start order: name, start_ns, end_ns."""
    rows = []
    with open(_one(directory, "_kernel_trace.csv"), newline="") as f:
        for r in csv.DictReader(f):
            rows.append({"name": r["Kernel_Name"], "start": int(r["Start_Timestamp"]), "end": int(r["End_Timestamp"])})
    rows.sort(key=lambda r: r["start"])
    return rows


def window_report(args) -> None:
    rows = [r for r in kernel_trace(args.dir) if args.family in r["name"]]
    if len(rows) < args.last:
        raise ValueError(f"only {len(rows)} {args.family} dispatches, asked for the last {args.last}")
    win = rows[-args.last:]
    durs = [r["end"] - r["start"] for r in win]
    avg_ns = sum(durs) / len(durs)
    span_ns = win[-1]["end"] - win[0]["start"]
    per_launch_ns = span_ns / args.last
    unit, scale = ("TFLOP/s", 1e-3) if args.unit == "flops" else ("GB/s", 1.0)
    work = args.work_per_launch
    by_name: dict[str, list[int]] = {}
    for r, d in zip(win, durs):
        by_name.setdefault(r["name"], []).append(d)
    lines = [f"# rocprofv3 kernel trace, timed window: {args.title}", "", "Command:", "", "```", args.command, "```",
             "", f"All dispatches of `{args.family}` in the trace: {len(rows)}; the window is the last {args.last} "
             f"({args.note}).", "",
             "| kernel | dispatches in window | avg us | min us | max us |", "|---|---|---|---|---|"]
    for name, d in sorted(by_name.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{_short(name)}` | {len(d)} | {sum(d) / len(d) / 1e3:.3f} | {min(d) / 1e3:.3f} | "
                     f"{max(d) / 1e3:.3f} |")
    try:
        stats = kernel_stats(args.dir)
    except FileNotFoundError:
        stats = []
    if stats:
        lines += ["", "Whole run (`--stats`, every dispatch including set-up, eager and warm-up launches):", "",
                  "| kernel | calls | total ms | avg us |", "|---|---|---|---|"]
        for r in stats[:8]:
            lines.append(f"| `{_short(r['name'])}` | {r['calls']} | {r['total_ns'] / 1e6:.3f} | {r['avg_ns'] / 1e3:.3f} |")
    lines += ["", f"Window: average kernel duration {avg_ns / 1e3:.3f} us; span {span_ns / 1e6:.3f} ms = "
                  f"{per_launch_ns / 1e3:.3f} us per launch (kernel plus the gap to the next one).", "",
              f"Algorithmic work per launch {work:,.0f} {'flop' if args.unit == 'flops' else 'B'}: "
              f"{work / avg_ns * scale:.1f} {unit} over the average kernel duration, "
              f"{work / per_launch_ns * scale:.1f} {unit} over the span."]
    Path(args.out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


# Kernels a projection step dispatches: the GEMM families and the K split's output fill.
STEP_KERNELS = ("gemm_", "zero_rows_kernel")


def _is_step(name: str) -> bool:
    return any(k in name for k in STEP_KERNELS)


def bench_points(bench_json: str) -> tuple[list[dict], int, int]:
    """(points, steps, warmup) of a bench.py JSON line: the headline and its points in
    the order the run timed them (workload, m, launches per step, ms per step, roofline
    object, value and unit each), and the run's timed and warm-up steps."""
    line = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
    out = [{"workload": line["config"]["workload"], "m": line["config"]["m"],
            "launches": line["config"]["launches_per_step"], "ms_per_step": line["ms_per_step"],
            "roofline": line["roofline"], "value": line["value"], "unit": line["unit"]}]
    for p in line.get("points", []):
        out.append({"workload": p["workload"], "m": p["m"], "launches": p["launches_per_step"],
                    "ms_per_step": p["ms_per_step"], "roofline": p["roofline"], "value": p["value"],
                    "unit": p["unit"]})
    return out, line["steps"], line["warmup"]


def step_runs(names: list[str]) -> list[tuple[int, int]]:
    """[start, end) index ranges of the maximal runs of consecutive step dispatches."""
    runs, i = [], 0
    while i < len(names):
        if _is_step(names[i]):
            j = i
            while j < len(names) and _is_step(names[j]):
                j += 1
            runs.append((i, j))
            i = j
        else:
            i += 1
    return runs


def segment_points(names: list[str], points: list[dict], steps_per_run: int, window_steps: int) -> list[range]:
    """Per point, the dispatch indices of its last `window_steps` steps. A point's steps end
    in a run of step dispatches that nothing else interrupts, of a length that is
    `steps_per_run` times the point's dispatches per step (its launches plus any K-split
    fills: between 1x and 2x its launches). The points take such runs in order. In
    bench.py's graph mode the run is the warm-up and timed replays (W + K steps: the eager
    step and the check replay are each followed by other kernels); in its eager mode at
    --steps 1 --warmup 0 it is the eager step and the timed one (2 steps)."""
    runs = step_runs(names)
    out, r = [], 0
    for p in points:
        while r < len(runs):
            a, b = runs[r]
            r += 1
            n = b - a
            if n % steps_per_run == 0 and p["launches"] <= n // steps_per_run <= 2 * p["launches"]:
                d = n // steps_per_run
                out.append(range(b - window_steps * d, b))
                break
        else:
            raise ValueError(f"no run of steps for point {p['workload']}")
    return out


def _work_per_step(p: dict) -> tuple[float, str]:
    roof = p["roofline"]
    if roof["unit"] == "TFLOP/s":
        return roof["algorithmic_flops_per_launch"] * p["launches"], "flops"
    return roof["algorithmic_bytes_per_launch"] * p["launches"], "bytes"


def points_report(args) -> None:
    points, steps, warmup = bench_points(args.bench_json)
    lines = [f"# Every point of one bench run: kernel trace, HBM traffic, MFMA counters", "",
             "Bench line: `" + args.bench_command + "` (its JSON line is the source of the points, their steps "
             "and launches).", "", "Points, in the order the run times them, and their workload strings:", ""]
    lines += [f"* {_label(p)}: `{p['workload']}`" for p in points] + [""]
    rec_out = []
    trace = kernel_trace(args.trace) if args.trace else None
    plain = bench_points(args.plain_json)[0] if args.plain_json else None
    if plain is not None and [q["workload"] for q in plain] != [p["workload"] for p in points]:
        raise ValueError("the plain run's points differ from the traced run's")
    if trace is not None:
        names = [r["name"] for r in trace]
        windows = segment_points(names, points, warmup + steps, steps)
        lines += ["## Kernel trace (timed replays of each point)", "", "Commands (the plain run first, then the "
                  "traced one, on one box):", "", "```", args.plain_command, args.trace_command, "```", "",
                  "Per point, the last `steps` replays of its run of graph replays in the trace. GEMM us per "
                  "launch = the step's `gemm_*` kernel durations over its launches; kernel ms per step = every "
                  "dispatch of the step (GEMMs and K-split output fills) summed; frac (kernel) = the step's "
                  "algorithmic work over that kernel time, against the peak. Bench figures are HIP events around "
                  "the same replays: in the traced run (the tracer adds ~2 us between short graph kernels) and "
                  "in the plain run before it. The trace backs the plain line when its kernel time per step is "
                  "at most the plain ms per step. Under the tracer a K-split output fill (and even an empty "
                  "kernel) shows ~4.5 us, against ~1.8 us per fill in an untraced graph replay, so at the points "
                  "with fills the GEMM time per step is the figure to hold against the plain line.", "",
                  "| point | dispatches/step | GEMM us/launch | bench us/launch (traced) | bench us/launch (plain) "
                  "| GEMM ms/step | kernel ms/step | bench ms/step (plain) | frac (kernel) | frac (plain) |",
                  "|---|---|---|---|---|---|---|---|---|---|"]
        for k, (p, win) in enumerate(zip(points, windows)):
            rows = [trace[i] for i in win]
            kernel_ns = sum(r["end"] - r["start"] for r in rows)
            gemm = [r["end"] - r["start"] for r in rows if "gemm_" in r["name"]]
            work, unit = _work_per_step(p)
            kern_ms = kernel_ns / steps / 1e6
            peak = 5000.0 if unit == "flops" else 8000.0
            scale = 1e12 if unit == "flops" else 1e9
            frac_kernel = work / (kern_ms * 1e-3) / scale / peak
            q = plain[k] if plain is not None else None
            lines.append(f"| {_label(p)} | {len(rows) // steps} | {sum(gemm) / len(gemm) / 1e3:.3f} | "
                         f"{p['roofline']['avg_launch_us']:.3f} | "
                         f"{'-' if q is None else format(q['roofline']['avg_launch_us'], '.3f')} | "
                         f"{sum(gemm) / steps / 1e6:.4f} | {kern_ms:.4f} | "
                         f"{'-' if q is None else format(q['ms_per_step'], '.4f')} | {frac_kernel:.4f} | "
                         f"{'-' if q is None else format(q['roofline']['frac'], '.4f')} |")
            rec_out.append({"workload": p["workload"], "dispatches_per_step": len(rows) // steps,
                            "gemm_us_per_launch": sum(gemm) / len(gemm) / 1e3,
                            "gemm_ms_per_step": sum(gemm) / steps / 1e6, "kernel_ms_per_step": kern_ms,
                            "frac_kernel": frac_kernel, "traced_bench_ms_per_step": p["ms_per_step"],
                            "plain_bench_ms_per_step": None if q is None else q["ms_per_step"],
                            "plain_frac": None if q is None else q["roofline"]["frac"]})
    if args.fetch and args.write:
        cal_fetch = sum(counter_per_dispatch(args.calib_fetch, "FETCH_SIZE", args.calib_family)) / \
            len(counter_per_dispatch(args.calib_fetch, "FETCH_SIZE", args.calib_family))
        cal_write = sum(counter_per_dispatch(args.calib_write, "WRITE_SIZE", args.calib_family)) / \
            len(counter_per_dispatch(args.calib_write, "WRITE_SIZE", args.calib_family))
        f_factor, w_factor = args.copy_bytes / cal_fetch, args.copy_bytes / cal_write
        fetch = counter_rows(args.fetch, "FETCH_SIZE")
        write = counter_rows(args.write, "WRITE_SIZE")
        fw = segment_points([r[0] for r in fetch], points, 2, 1)
        ww = segment_points([r[0] for r in write], points, 2, 1)
        lines += ["", "## HBM traffic (one eager step of each point, every dispatch of the step)", "", "Commands:", "",
                  "```", args.traffic_command, "```", "",
                  f"Counters scaled by the copy calibration: FETCH_SIZE {f_factor:.1f} and WRITE_SIZE "
                  f"{w_factor:.1f} bytes per unit (`mambo_copy_bytes` over {args.copy_bytes:,} bytes).", "",
                  "| point | dispatches | traffic per launch | algorithmic per launch | ratio |", "|---|---|---|---|---|"]
        for p, fr, wr in zip(points, fw, ww):
            fb = sum(fetch[i][1] for i in fr) * f_factor
            wb = sum(write[i][1] for i in wr) * w_factor
            per_launch = (fb + wb) / p["launches"]
            roof = p["roofline"]
            algo = roof.get("algorithmic_bytes_per_launch")
            if algo is None:  # MFMA-bound points: bytes of the projections' operands
                algo = roof.get("algorithmic_operand_bytes_per_launch")
            ratio = per_launch / algo if algo else None
            lines.append(f"| {_label(p)} | {len(fr)} | {per_launch:,.0f} | "
                         f"{'-' if algo is None else f'{algo:,.0f}'} | {'-' if ratio is None else f'{ratio:.3f}'} |")
            rec = {"workload": p["workload"], "kernel_family": "gemm_ + zero_rows_kernel (whole step)",
                   "dispatches": len(fr), "calibration": {"copy_bytes": args.copy_bytes, "fetch_size": cal_fetch,
                                                          "write_size": cal_write, "fetch_bytes_per_unit": f_factor,
                                                          "write_bytes_per_unit": w_factor},
                   "fetch_bytes_per_launch": fb / p["launches"], "write_bytes_per_launch": wb / p["launches"],
                   "traffic_bytes_per_launch": per_launch, "algorithmic_bytes_per_launch": algo,
                   "traffic_over_algorithmic": ratio, "command": args.traffic_command}
            slug = _slug(p)
            Path(args.out_dir, f"traffic_{slug}.json").write_text(json.dumps(rec, indent=1) + "\n")
    if args.mfma:
        busy = counter_rows(args.mfma, "SQ_VALU_MFMA_BUSY_CYCLES")
        mops = counter_rows(args.mfma, "SQ_INSTS_VALU_MFMA_MOPS_F8")
        gui = counter_rows(args.mfma, "GRBM_GUI_ACTIVE")
        bw = segment_points([r[0] for r in busy], points, 2, 1)
        lines += ["", "## MFMA counters (one eager step of each MFMA-bound point)", "", "Command:", "", "```",
                  args.mfma_command, "```", "",
                  f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {args.xcds} XCDs x "
                  f"{args.cus * SIMD_PER_CU} SIMDs), over the step's tiled-kernel dispatches weighted by their "
                  "active cycles; executed F8 flops = SQ_INSTS_VALU_MFMA_MOPS_F8 x 512.", "",
                  "| point | MFMA busy | executed / algorithmic F8 flops |", "|---|---|---|"]
        simds = args.cus * SIMD_PER_CU
        for p, win in zip(points, bw):
            if p["roofline"]["unit"] != "TFLOP/s":
                continue
            b = sum(busy[i][1] for i in win)
            g = sum(gui[i][1] for i in win)
            m = sum(mops[i][1] for i in win)
            work, _ = _work_per_step(p)
            lines.append(f"| {_label(p)} | {100 * b / (g / args.xcds * simds):.1f}% | {m * 512 / work:.3f} |")
    Path(args.out).write_text("\n".join(lines) + "\n")
    if rec_out:
        Path(args.out).with_suffix(".json").write_text(json.dumps(rec_out, indent=1) + "\n")
    print("\n".join(lines))


def _label(p: dict) -> str:
    return (f"{'70B' if '70b' in p['workload'] else '8B'} M={p['m']}"
            f"{' (one launch per projection)' if 'one launch per' in p['workload'] else ''}")


def _slug(p: dict) -> str:
    model = "llama70b" if "70b" in p["workload"] else "llama8b"
    tail = "_nogroup" if "one launch per projection" in p["workload"] else ""
    return f"{model}_m{p['m']}{tail}"


def counter_rows(directory: str, counter: str) -> list[tuple[str, float]]:
    """(kernel name, value) of `counter` for every dispatch of a --pmc run, in dispatch order."""
    rows = []
    with open(_one(directory, "_counter_collection.csv"), newline="") as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"])))
    rows.sort()
    return [(n, v) for _, n, v in rows]


SIMD_PER_CU = 4


def mfma_report(args) -> None:
    busy = counter_per_dispatch(args.dir, "SQ_VALU_MFMA_BUSY_CYCLES", args.family)
    mops = counter_per_dispatch(args.dir, "SQ_INSTS_VALU_MFMA_MOPS_F8", args.family)
    gui = counter_per_dispatch(args.dir, "GRBM_GUI_ACTIVE", args.family)
    if not len(busy) == len(mops) == len(gui):
        raise ValueError("counter records do not pair up per dispatch")
    simds = args.cus * SIMD_PER_CU
    util = [b / (g / args.xcds * simds) for b, g in zip(busy, gui)]
    derived = counter_per_dispatch(args.util_dir, "MfmaUtil", args.family) if args.util_dir else []
    executed = [m_ * 512 for m_ in mops]
    mean = lambda v: sum(v) / len(v)  # noqa: E731
    rec = {"workload": args.workload, "kernel_family": args.family, "dispatches": len(busy), "cus": args.cus,
           "mfma_busy": mean(util), "mfma_busy_min": min(util), "mfma_busy_max": max(util),
           "mfma_util_rocprof": mean(derived) / 100 if derived else None,
           "executed_f8_flops_per_dispatch": mean(executed),
           "algorithmic_flops_per_dispatch": args.algorithmic_flops,
           "executed_over_algorithmic": mean(executed) / args.algorithmic_flops if args.algorithmic_flops else None,
           "command": args.command}
    out = Path(args.out)
    out.with_suffix(".json").write_text(json.dumps(rec, indent=1) + "\n")
    lines = [f"# MFMA counters per dispatch: {args.workload}", "", "Command:", "", "```", args.command, "```", "",
             f"Kernel family `{args.family}`, {len(busy)} dispatches.", "",
             "| counter (per dispatch, mean) | value |", "|---|---|",
             f"| SQ_VALU_MFMA_BUSY_CYCLES (sum over SIMDs) | {mean(busy):,.0f} |",
             f"| GRBM_GUI_ACTIVE | {mean(gui):,.0f} |",
             f"| SQ_INSTS_VALU_MFMA_MOPS_F8 (x512 = F8 flops) | {mean(mops):,.0f} |", "",
             f"MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / {args.xcds} XCDs x {simds} SIMDs): mean "
             f"{100 * rec['mfma_busy']:.1f}% (min {100 * min(util):.1f}%, max {100 * max(util):.1f}%)."
             + (f" rocprofv3's derived MfmaUtil in a run of its own: mean {mean(derived):.1f}%." if derived else ""),
             "",
             f"Executed F8 MFMA flops {mean(executed):,.0f} per dispatch against {args.algorithmic_flops:,} "
             f"algorithmic (ratio {rec['executed_over_algorithmic']:.3f})."]
    out.with_suffix(".md").write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = p.add_subparsers(dest="cmd", required=True)
    s = sub.add_parser("stats")
    s.add_argument("dir")
    s.add_argument("--family", default="")
    s.add_argument("--title", default="")
    s.add_argument("--command", required=True)
    s.add_argument("--top", type=int, default=12)
    s.add_argument("--out", required=True)
    t = sub.add_parser("traffic")
    for name in ("--fetch", "--write", "--calib-fetch", "--calib-write", "--workload", "--command", "--out"):
        t.add_argument(name, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--algorithmic-bytes", type=int, required=True)
    t.add_argument("--family", default="gemm_stream_kernel")
    t.add_argument("--calib-family", default="copy_bytes_kernel")
    w = sub.add_parser("window")
    w.add_argument("dir")
    w.add_argument("--family", required=True)
    w.add_argument("--last", type=int, required=True)
    w.add_argument("--work-per-launch", type=float, required=True)
    w.add_argument("--unit", choices=["bytes", "flops"], default="bytes")
    w.add_argument("--title", default="")
    w.add_argument("--note", default="the timed replays")
    w.add_argument("--command", required=True)
    w.add_argument("--out", required=True)
    q = sub.add_parser("points")
    q.add_argument("--bench-json", required=True)
    q.add_argument("--bench-command", required=True)
    q.add_argument("--plain-json", default="")
    q.add_argument("--plain-command", default="")
    q.add_argument("--trace", default="")
    q.add_argument("--trace-command", default="")
    q.add_argument("--fetch", default="")
    q.add_argument("--write", default="")
    q.add_argument("--calib-fetch", default="")
    q.add_argument("--calib-write", default="")
    q.add_argument("--calib-family", default="copy_bytes_kernel")
    q.add_argument("--copy-bytes", type=int, default=1 << 30)
    q.add_argument("--traffic-command", default="")
    q.add_argument("--mfma", default="")
    q.add_argument("--mfma-command", default="")
    q.add_argument("--cus", type=int, default=256)
    q.add_argument("--xcds", type=int, default=8)
    q.add_argument("--out", required=True)
    q.add_argument("--out-dir", default="profiles")
    m = sub.add_parser("mfma")
    m.add_argument("dir")
    m.add_argument("--family", required=True)
    m.add_argument("--cus", type=int, default=256)
    m.add_argument("--xcds", type=int, default=8)
    m.add_argument("--util-dir", default="")
    m.add_argument("--algorithmic-flops", type=int, required=True)
    for name in ("--workload", "--command", "--out"):
        m.add_argument(name, required=True)
    args = p.parse_args(argv)
    {"stats": stats_report, "traffic": traffic_report, "window": window_report, "mfma": mfma_report,
     "points": points_report}[args.cmd](args)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
