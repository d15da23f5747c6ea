"""Per-frame kernel breakdown from a rocprofv3 kernel trace.

    python -m mockbird_amd.profile_frames TRACE.csv --delimiter k_frame_emit [--skip 3]
    python -m mockbird_amd.profile_frames TRACE.csv --delimiter k_codec_head --last 24
    python -m mockbird_amd.profile_frames TRACE.csv --grids k_ring_write

TRACE.csv is the `*_kernel_trace.csv` of `rocprofv3 --kernel-trace
--output-format csv`.  Dispatches are split into runs wherever the GPU sat
idle for more than `--gap-ms` (set-up between two benchmark runs), and each
run into frames at the delimiting kernel (the last launch of a frame: the
decode frame's `k_frame_emit`, the codec frame's `k_codec_head`).  For each
run the tool prints one markdown table: launches per frame, per-kernel
launches, mean duration and time per frame, over the frames kept (`--skip`
drops the first frames as warm-up, `--last` keeps only the last n).  The
"span" is the time from one delimiter's end to the next one's, the frame's
wall time on the GPU; under the tracer it includes the tracer's per-launch
overhead, the kernel time does not.

`--nth KERNEL` adds, per run, the mean duration of the i-th launch of the
kernels whose name contains KERNEL within a frame (i = 1, 2, ...: a frame's
layers or stages in launch order).

`--grids KERNEL` instead lists the dispatches of the kernels whose name
contains KERNEL grouped by kernel and grid size (one launch shape each):
dispatches, mean, min and max duration; with `--by-run` each unbroken run
of one shape's dispatches (in dispatch order) is a line of its own, which
tells apart two projections that share a grid.  Given the `*_counter_collection.csv`
of a `rocprofv3 --pmc` run instead, it lists each counter's median value per
dispatch for each launch shape.
"""
from __future__ import annotations

import argparse
import collections
import csv
import re
import sys


def load(path: str) -> list[dict]:
    with open(path, newline="") as fh:
        rows = list(csv.DictReader(fh))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    return rows


def split_runs(rows: list[dict], gap_ns: float) -> list[list[dict]]:
    runs, cur, last_end = [], [], None
    for r in rows:
        s, e = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        if last_end is not None and s - last_end > gap_ns and cur:
            runs.append(cur)
            cur = []
        cur.append(r)
        last_end = e if last_end is None else max(last_end, e)
    if cur:
        runs.append(cur)
    return runs


def short_name(name: str) -> str:
    """Kernel name without its argument list (template arguments kept)."""
    name = name.replace("(anonymous namespace)::", "")
    depth = 0
    for i, ch in enumerate(name):
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0:
            name = name[:i]
            break
    return re.sub(r"^void ", "", name).strip()


def frames_of(run: list[dict], delimiter: str, skip: int, last: int | None):
    """[(first index, last index)] of each kept frame: the launches after one
    delimiter up to and including the next."""
    ends = [i for i, r in enumerate(run) if delimiter in r["Kernel_Name"]]
    fr = list(zip(ends[:-1], ends[1:]))
    fr = fr[skip:]
    if last is not None:
        fr = fr[-last:]
    return fr


def breakdown(run: list[dict], frames) -> dict:
    agg = collections.defaultdict(lambda: [0, 0.0])
    span = 0.0
    for a, b in frames:
        span += (int(run[b]["End_Timestamp"]) - int(run[a]["End_Timestamp"])) / 1e3
        for r in run[a + 1:b + 1]:
            k = short_name(r["Kernel_Name"])
            agg[k][0] += 1
            agg[k][1] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
    n = len(frames)
    kernels = sorted(((k, c / n, t / c, t / n) for k, (c, t) in agg.items()), key=lambda x: -x[3])
    total = sum(x[3] for x in kernels)
    return {"frames": n, "launches": sum(x[1] for x in kernels), "kernel_us": total,
            "span_us": span / n, "kernels": kernels}


def nth_launches(run: list[dict], frames, kernel: str):
    """{name: [mean us of the i-th launch of that kernel in a frame]} over the
    frames (a, b]."""
    agg = collections.defaultdict(lambda: collections.defaultdict(list))
    for a, b in frames:
        seen = collections.Counter()
        for r in run[a + 1:b + 1]:
            if kernel in r["Kernel_Name"]:
                k = short_name(r["Kernel_Name"])
                agg[k][seen[k]].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                seen[k] += 1
    return {k: [sum(v[i]) / len(v[i]) for i in sorted(v)] for k, v in sorted(agg.items())}


def grid_of(run: list[dict], kernel: str) -> str:
    for r in run:
        if kernel in r["Kernel_Name"]:
            return r.get("Grid_Size_X", r.get("Grid_Size", "?"))
    return "?"


def by_grid(rows: list[dict], kernel: str, by_run: bool = False):
    """[(kernel, grid, workgroup, n, mean us, min us, max us)] per (kernel, grid,
    workgroup), or with by_run per unbroken run of such dispatches among the
    matching ones (in start order), runs listed in order."""
    agg = collections.defaultdict(list)
    run, last = 0, None
    for r in rows:
        if kernel in r["Kernel_Name"]:
            key = (short_name(r["Kernel_Name"]), int(r.get("Grid_Size_X", r.get("Grid_Size", 0))),
                   int(r.get("Workgroup_Size_X", r.get("Workgroup_Size", 0))))
            if by_run and key != last:
                run += 1
                last = key
            agg[(run, key) if by_run else key].append(
                (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    items = sorted(agg.items())
    if by_run:
        items = [(k, d) for (_, k), d in items]
    return [(k, g, w, len(d), sum(d) / len(d), min(d), max(d)) for (k, g, w), d in items]


def counters_by_grid(path: str, kernel: str, by_run: bool = False):
    """[(kernel, grid, counter, dispatches, median value)] from a counter
    collection CSV (one row per dispatch and counter); with by_run, per
    unbroken run of one shape's dispatches in dispatch order."""
    with open(path, newline="") as fh:
        rows = [r for r in csv.DictReader(fh) if kernel in r["Kernel_Name"]]
    rows.sort(key=lambda r: int(r.get("Dispatch_Id", 0)))
    agg = collections.defaultdict(list)
    run, last, last_id = 0, None, None
    for r in rows:
        shape = (short_name(r["Kernel_Name"]), int(r["Grid_Size"]))
        if by_run and shape != last and r.get("Dispatch_Id") != last_id:
            run += 1
            last = shape
        last_id = r.get("Dispatch_Id")
        agg[(run, shape[0], shape[1], r["Counter_Name"])].append(float(r["Counter_Value"]))
    out = []
    for (_, k, g, c), vals in sorted(agg.items()):
        vals.sort()
        n = len(vals)
        med = vals[n // 2] if n % 2 else 0.5 * (vals[n // 2 - 1] + vals[n // 2])
        out.append((k, g, c, n, med))
    return out


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("trace")
    ap.add_argument("--delimiter", help="name of a frame's last kernel")
    ap.add_argument("--nth", default=None, metavar="KERNEL",
                    help="also list the mean duration of each launch of KERNEL by its order in a frame")
    ap.add_argument("--grids", default=None, metavar="KERNEL",
                    help="list KERNEL's dispatches by grid size instead of frames")
    ap.add_argument("--by-run", action="store_true",
                    help="with --grids: one line per unbroken run of a shape's dispatches")
    ap.add_argument("--skip", type=int, default=0, help="frames dropped at the start of each run")
    ap.add_argument("--last", type=int, default=None, help="keep only the last n frames of a run")
    ap.add_argument("--gap-ms", type=float, default=5.0, help="idle time that separates runs")
    ap.add_argument("--top", type=int, default=14, help="kernels listed per run")
    ap.add_argument("--grid-of", default=None,
                    help="kernel whose grid size is printed per run (to tell runs apart)")
    a = ap.parse_args(argv)
    if a.grids:
        with open(a.trace, newline="") as fh:
            header = next(csv.reader(fh))
        if "Counter_Value" in header:
            print("| kernel | grid (threads) | counter | dispatches | median per dispatch |")
            print("|---|---:|---|---:|---:|")
            for k, g, c, n, med in counters_by_grid(a.trace, a.grids, a.by_run):
                print(f"| `{k}` | {g} | {c} | {n} | {med:.1f} |")
            return 0
        print("| kernel | grid (threads) | workgroup | dispatches | avg us | min us | max us |")
        print("|---|---:|---:|---:|---:|---:|---:|")
        for k, g, w, n, avg, lo, hi in by_grid(load(a.trace), a.grids, a.by_run):
            print(f"| `{k}` | {g} | {w} | {n} | {avg:.2f} | {lo:.2f} | {hi:.2f} |")
        return 0
    if not a.delimiter:
        ap.error("--delimiter or --grids is required")
    for run in split_runs(load(a.trace), a.gap_ms * 1e6):
        fr = frames_of(run, a.delimiter, a.skip, a.last)
        if not fr:
            continue
        b = breakdown(run, fr)
        grid = f", {a.grid_of} grid {grid_of(run, a.grid_of)}" if a.grid_of else ""
        print(f"\n{b['frames']} frames{grid}: {b['launches']:.0f} launches/frame, kernel time "
              f"{b['kernel_us']:.1f} us/frame, span {b['span_us']:.1f} us/frame\n")
        print("| kernel | per frame | avg us | us per frame | share |")
        print("|---|---:|---:|---:|---:|")
        for k, c, avg, per in b["kernels"][:a.top]:
            print(f"| `{k}` | {c:.0f} | {avg:.2f} | {per:.1f} | {100 * per / b['kernel_us']:.1f} % |")
        if a.nth:
            for k, means in nth_launches(run, fr, a.nth).items():
                print(f"\n`{k}` by launch order in the frame (us): " +
                      ", ".join(f"{m:.2f}" for m in means))
    return 0


if __name__ == "__main__":
    sys.exit(main())
