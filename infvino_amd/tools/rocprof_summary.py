"""Summaries of rocprofv3 output for this backend's kernels.

  python -m infvino_amd.tools.rocprof_summary trace <run_kernel_trace.csv> [--top N] [--grid-min G]
      per (kernel, grid size): dispatches, mean / min / max duration (us), total (ms)
  python -m infvino_amd.tools.rocprof_summary pmc <run_counter_collection.csv> [--kernel SUBSTR]
      per (kernel, grid size): mean value of each counter per dispatch

The same kernel template runs at many shapes (one launch per plan node), and a bench run
mixes batch 64 and batch 1 steps, so statistics are grouped by launch grid as well as name.
"""
import argparse
import csv
import sys
from collections import defaultdict


def short(name: str) -> str:
    name = name.replace("ivh::", "")
    for cut in ("(ivh", "(Conv", "(Small", "(const"):
        i = name.find(cut)
        if i > 0:
            name = name[:i]
    return name.strip()


def trace(path, top, grid_min):
    rows = defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            if g < grid_min:
                continue
            d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
            key = (short(r["Kernel_Name"]), f'{r["Grid_Size_X"]}x{r["Grid_Size_Y"]}x{r["Grid_Size_Z"]}')
            rows[key].append(d)
    total = sum(sum(v) for v in rows.values())
    print(f"| kernel | grid | dispatches | mean us | min us | max us | total ms | % |")
    print("|---|---|---:|---:|---:|---:|---:|---:|")
    for (k, g), v in sorted(rows.items(), key=lambda kv: -sum(kv[1]))[:top]:
        print(f"| {k} | {g} | {len(v)} | {sum(v) / len(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
              f"{sum(v) / 1e3:.3f} | {100 * sum(v) / total:.1f} |")
    print(f"\ntotal kernel time {total / 1e3:.3f} ms over {sum(len(v) for v in rows.values())} dispatches")


def pmc(path, kernel):
    acc = defaultdict(lambda: defaultdict(list))
    with open(path) as f:
        rdr = csv.DictReader(f)
        for r in rdr:
            name = short(r.get("Kernel_Name", ""))
            if kernel and kernel not in name:
                continue
            g = "x".join(r.get(k, "?") for k in ("Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z")) \
                if "Grid_Size_X" in r else r.get("Grid_Size", "?")
            cname = r.get("Counter_Name")
            val = float(r.get("Counter_Value", "nan"))
            disp = r.get("Dispatch_Id", "")
            acc[(name, g, cname)][disp].append(val)
    print("| kernel | grid | counter | dispatches | mean per dispatch |")
    print("|---|---|---|---:|---:|")
    for (k, g, c), d in sorted(acc.items()):
        per = [sum(v) for v in d.values()]
        print(f"| {k} | {g} | {c} | {len(per)} | {sum(per) / len(per):.1f} |")


def main(argv=None):
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--top", type=int, default=30)
    t.add_argument("--grid-min", type=int, default=0)
    p = sub.add_parser("pmc")
    p.add_argument("csv")
    p.add_argument("--kernel", default="")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        trace(a.csv, a.top, a.grid_min)
    else:
        pmc(a.csv, a.kernel)


if __name__ == "__main__":
    sys.exit(main())
