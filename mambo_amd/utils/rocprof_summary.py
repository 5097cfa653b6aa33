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
    {"stats": stats_report, "traffic": traffic_report, "window": window_report, "mfma": mfma_report}[args.cmd](args)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
