"""Summaries of rocprofv3 CSV output for the kernels of this package.

Two reports, both plain text meant to be committed next to the numbers they back:

* ``stats``: the per-kernel duration table of a ``rocprofv3 --kernel-trace --stats
  --output-format csv`` run (``*_kernel_stats.csv``), plus a combined row for every
  kernel whose name contains ``--family`` (template instantiations of one kernel).
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
    args = p.parse_args(argv)
    (stats_report if args.cmd == "stats" else traffic_report)(args)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
