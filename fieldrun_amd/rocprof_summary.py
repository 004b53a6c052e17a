"""Summarise rocprofv3 CSV output as short markdown.

  python3 -m fieldrun_amd.rocprof_summary stats KERNEL_STATS_CSV [--command CMD]
      per-kernel call count and durations from `rocprofv3 --kernel-trace
      --stats --output-format csv` (the *_kernel_stats.csv file).

  python3 -m fieldrun_amd.rocprof_summary trace KERNEL_TRACE_CSV [--command CMD]
      the same per (kernel, workgroup count) from *_kernel_trace.csv, with
      register / LDS / scratch use.

  python3 -m fieldrun_amd.rocprof_summary steps KERNEL_TRACE_CSV --marker SUBSTR
          [--exclude SUBSTR ...] [--by-prev] [--command CMD]
      per-step time of each (kernel, workgroup count) over a run of decode
      steps: the trace (in start order) is cut at each launch of the kernel
      whose name contains the marker (one a step, e.g. the head), intervals
      holding a kernel whose name contains an --exclude string (a prefill's)
      are dropped, and each kernel's time is averaged over the kept steps
      (--by-prev: each (kernel, grid) split by the kernel launched before it).

  python3 -m fieldrun_amd.rocprof_summary pmc --fetch CSV --write CSV
          --kernel NAME --copy-bytes N --algo-bytes B [--command-fetch CMD]
          [--command-write CMD]
      HBM traffic per launch of kernel NAME from two `rocprofv3 --pmc` runs
      (FETCH_SIZE, then WRITE_SIZE; *_counter_collection.csv).  Each counter
      (KiB per dispatch) is scaled by the factor that makes the same counter
      read N bytes on the device-to-device copy of N bytes in the same run.

  python3 -m fieldrun_amd.rocprof_summary pmc-layer --fetch CSV --write CSV
          --kernel PREFIX --per-shape R --shapes S --copy-bytes N
          --algo-bytes B [--command-fetch CMD] [--command-write CMD]
      The same for a workload that launches S shapes of kernels named
      PREFIX... R times each, in order: the dispatches are split into S runs
      of R by dispatch order, each run's mean taken, and the S means summed
      (one launch of each shape, e.g. one model layer's linears).
"""
from __future__ import annotations

import argparse
import csv
import re
import sys
from collections import defaultdict


def short_name(name: str) -> str:
    """Kernel name without namespaces and parameter list, template args kept."""
    depth, cut = 0, len(name)
    for i, ch in enumerate(name):  # drop the trailing "(args)"
        if ch == "<":
            depth += 1
        elif ch == ">":
            depth -= 1
        elif ch == "(" and depth == 0 and not name.startswith("(", i + 1):
            if name[i:i + 21] == "(anonymous namespace)":
                continue
            cut = i
            break
    s = name[:cut].replace("(anonymous namespace)::", "")
    s = re.sub(r"^(void\s+)", "", s)
    s = re.sub(r"\bfrq::", "", s)
    return s.replace(" ", "")


def _rows(path: str):
    with open(path, newline="") as f:
        yield from csv.DictReader(f)


def stats(args) -> str:
    rows = list(_rows(args.csv))
    out = []
    if args.command:
        out += ["Command:", "", "    " + args.command, ""]
    out += ["| kernel | calls | avg us | min us | max us | % time |", "|---|---:|---:|---:|---:|---:|"]
    rows.sort(key=lambda r: -float(r.get("TotalDurationNs", 0) or 0))
    for r in rows[: args.top]:
        out.append("| `%s` | %s | %.2f | %.2f | %.2f | %.1f |" % (
            short_name(r["Name"]), r["Calls"], float(r["AverageNs"]) / 1e3,
            float(r["MinNs"]) / 1e3, float(r["MaxNs"]) / 1e3, float(r["Percentage"])))
    return "\n".join(out) + "\n"


def trace(args) -> str:
    """Per (kernel, grid) durations from *_kernel_trace.csv: launches of one
    kernel at different shapes have different grids."""
    acc = defaultdict(list)
    meta = {}
    for r in _rows(args.csv):
        key = (short_name(r["Kernel_Name"]), int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])))
        acc[key].append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        meta[key] = (r["VGPR_Count"], r["Accum_VGPR_Count"], r["SGPR_Count"], r["LDS_Block_Size"],
                     r["Scratch_Size"])
    out = []
    if args.command:
        out += ["Command:", "", "    " + args.command, ""]
    out += ["| kernel | workgroups | calls | avg us | min us | max us | VGPR | AGPR | SGPR | LDS B | scratch B |",
            "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    keys = sorted(acc, key=lambda k: -sum(acc[k]))[: args.top]
    for k in keys:
        v = acc[k]
        out.append("| `%s` | %d | %d | %.2f | %.2f | %.2f | %s | %s | %s | %s | %s |" % (
            k[0], k[1], len(v), sum(v) / len(v), min(v), max(v), *meta[k]))
    return "\n".join(out) + "\n"


def steps(args) -> str:
    """Per-step kernel times between consecutive marker launches."""
    rows = sorted(_rows(args.csv), key=lambda r: int(r["Start_Timestamp"]))
    marks = [i for i, r in enumerate(rows) if args.marker in r["Kernel_Name"]]
    acc = defaultdict(float)
    cnt = defaultdict(int)
    kept, span = 0, 0.0
    for a, b in zip(marks, marks[1:]):
        seg = rows[a + 1:b + 1]  # a step ends with its head launch
        if any(x in r["Kernel_Name"] for r in seg for x in args.exclude):
            continue
        kept += 1
        span += (int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"])) / 1e3
        prev = short_name(rows[a]["Kernel_Name"])
        for r in seg:
            name = short_name(r["Kernel_Name"])
            # --by-prev: launches of one kernel and grid told apart by the
            # kernel launched before them (e.g. two linears of a layer)
            key = (name if not args.by_prev else f"{name} after {prev.split('<')[0]}",
                   int(r["Grid_Size_X"]) // max(1, int(r["Workgroup_Size_X"])))
            acc[key] += (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            cnt[key] += 1
            prev = name
    out = []
    if args.command:
        out += ["Command:", "", "    " + args.command, ""]
    if not kept:
        return "\n".join(out + ["no complete step between markers"]) + "\n"
    busy = sum(acc.values()) / kept
    out += [f"{kept} steps: {busy:.1f} us of kernel time a step ({span / kept:.1f} us first start to last end)", "",
            "| kernel | workgroups | launches a step | us a step | avg us | share |",
            "|---|---:|---:|---:|---:|---:|"]
    for k in sorted(acc, key=lambda k: -acc[k])[: args.top]:
        out.append("| `%s` | %d | %.1f | %.1f | %.2f | %.1f%% |" % (
            k[0], k[1], cnt[k] / kept, acc[k] / kept, acc[k] / cnt[k], 100 * acc[k] / kept / busy))
    return "\n".join(out) + "\n"


def _per_kernel(path: str, counter: str, largest_grid=()):
    """Mean counter value per dispatch, by short kernel name.  For kernels
    whose short name contains one of `largest_grid`, only the dispatches with
    the largest grid count (the runtime's copy kernel also serves small
    host<->device copies, which must not dilute the calibration)."""
    acc = defaultdict(list)
    for r in _rows(path):
        if r.get("Counter_Name", "").strip() != counter:
            continue
        acc[short_name(r["Kernel_Name"])].append((int(r.get("Grid_Size", 0) or 0),
                                                  float(r["Counter_Value"])))
    out = {}
    for k, v in acc.items():
        if any(p in k for p in largest_grid):
            g = max(x[0] for x in v)
            v = [x for x in v if x[0] == g]
        vals = [x[1] for x in v]
        out[k] = (sum(vals) / len(vals), len(vals))
    return out


def _pick(table, pattern: str, what: str):
    key = pattern.replace(" ", "")
    hits = [k for k in table if key in k]
    if len(hits) != 1:
        sys.exit(f"{what}: {len(hits)} kernels match {pattern!r}: {sorted(table)}")
    return hits[0], table[hits[0]]


def pmc(args) -> str:
    lines = []
    total = 0.0
    for counter, path, cmd in (("FETCH_SIZE", args.fetch, args.command_fetch),
                               ("WRITE_SIZE", args.write, args.command_write)):
        table = _per_kernel(path, counter, largest_grid=(args.copy_kernel,))
        cname, (cval, cn) = _pick(table, args.copy_kernel, counter + " copy")
        kname, (kval, kn) = _pick(table, args.kernel, counter + " kernel")
        factor = args.copy_bytes / (cval * 1024.0)
        bytes_ = kval * 1024.0 * factor
        total += bytes_
        if cmd:
            lines += [f"{counter} run:", "", "    " + cmd, ""]
        lines += [f"- `{cname}` ({cn} dispatches of {args.copy_bytes} bytes): {counter} = {cval:.0f} KiB"
                  f" per dispatch, scale factor {factor:.4f}",
                  f"- `{kname}` ({kn} dispatches): {counter} = {kval:.0f} KiB per dispatch"
                  f" -> {bytes_:.0f} bytes", ""]
    lines += [f"Algorithmic bytes per launch: {args.algo_bytes}",
              f"Measured HBM traffic / algorithmic: {total / args.algo_bytes:.3f}", "",
              f"traffic_bytes_per_launch: {int(round(total))}"]
    return "\n".join(lines) + "\n"


def _dispatches(path: str, counter: str, prefix: str):
    """(dispatch id, counter value) of the kernels whose short name starts
    with `prefix`, in dispatch order."""
    out = []
    for r in _rows(path):
        if r.get("Counter_Name", "").strip() != counter:
            continue
        if short_name(r["Kernel_Name"]).startswith(prefix):
            out.append((int(r.get("Dispatch_Id", 0) or 0), float(r["Counter_Value"]), short_name(r["Kernel_Name"])))
    out.sort()
    return out


def pmc_layer(args) -> str:
    lines = []
    total = 0.0
    for counter, path, cmd in (("FETCH_SIZE", args.fetch, args.command_fetch),
                               ("WRITE_SIZE", args.write, args.command_write)):
        table = _per_kernel(path, counter, largest_grid=(args.copy_kernel,))
        cname, (cval, cn) = _pick(table, args.copy_kernel, counter + " copy")
        factor = args.copy_bytes / (cval * 1024.0)
        ds = _dispatches(path, counter, args.kernel)
        if len(ds) != args.per_shape * args.shapes:
            sys.exit(f"{counter}: {len(ds)} dispatches of {args.kernel}..., expected {args.per_shape * args.shapes}")
        if cmd:
            lines += [f"{counter} run:", "", "    " + cmd, ""]
        lines.append(f"- `{cname}` ({cn} dispatches of {args.copy_bytes} bytes): {counter} = {cval:.0f} KiB"
                     f" per dispatch, scale factor {factor:.4f}")
        sub = 0.0
        for i in range(args.shapes):
            run = ds[i * args.per_shape:(i + 1) * args.per_shape]
            kv = sum(x[1] for x in run) / len(run)
            b = kv * 1024.0 * factor
            sub += b
            lines.append(f"- shape {i} `{run[0][2]}` ({len(run)} dispatches): {counter} = {kv:.0f} KiB per dispatch"
                         f" -> {b:.0f} bytes")
        lines += [f"- {counter} over one launch of each shape: {sub:.0f} bytes", ""]
        total += sub
    lines += [f"Algorithmic bytes (one launch of each shape): {args.algo_bytes}",
              f"Measured HBM traffic / algorithmic: {total / args.algo_bytes:.3f}", "",
              f"traffic_bytes_per_launch: {int(round(total))}"]
    return "\n".join(lines) + "\n"


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    sub = ap.add_subparsers(dest="mode", required=True)
    s = sub.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--command", default="")
    s.add_argument("--top", type=int, default=25)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--command", default="")
    t.add_argument("--top", type=int, default=40)
    st = sub.add_parser("steps")
    st.add_argument("csv")
    st.add_argument("--marker", required=True)
    st.add_argument("--exclude", action="append", default=[])
    st.add_argument("--top", type=int, default=25)
    st.add_argument("--command", default="")
    st.add_argument("--by-prev", action="store_true")
    p = sub.add_parser("pmc")
    p.add_argument("--fetch", required=True)
    p.add_argument("--write", required=True)
    p.add_argument("--kernel", required=True)
    p.add_argument("--copy-kernel", default="copyBuffer")
    p.add_argument("--copy-bytes", type=int, required=True)
    p.add_argument("--algo-bytes", type=int, required=True)
    p.add_argument("--command-fetch", default="")
    p.add_argument("--command-write", default="")
    pl = sub.add_parser("pmc-layer")
    pl.add_argument("--fetch", required=True)
    pl.add_argument("--write", required=True)
    pl.add_argument("--kernel", required=True)
    pl.add_argument("--per-shape", type=int, required=True)
    pl.add_argument("--shapes", type=int, required=True)
    pl.add_argument("--copy-kernel", default="copyBuffer")
    pl.add_argument("--copy-bytes", type=int, required=True)
    pl.add_argument("--algo-bytes", type=int, required=True)
    pl.add_argument("--command-fetch", default="")
    pl.add_argument("--command-write", default="")
    a = ap.parse_args(argv)
    sys.stdout.write({"stats": stats, "trace": trace, "steps": steps, "pmc": pmc, "pmc-layer": pmc_layer}[a.mode](a))


if __name__ == "__main__":
    main()
