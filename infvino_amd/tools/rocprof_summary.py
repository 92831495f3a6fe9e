"""Summaries of rocprofv3 output for this backend's kernels.

  python -m infvino_amd.tools.rocprof_summary trace <run_kernel_trace.csv> [--top N] [--grid-min G]
      per (kernel, grid size): dispatches, mean / min / max duration (us), total (ms)
  python -m infvino_amd.tools.rocprof_summary pmc <run_counter_collection.csv> [--kernel SUBSTR]
      per (kernel, grid size): mean value of each counter per dispatch
  python -m infvino_amd.tools.rocprof_summary counters <prefix> --kernel SUBSTR [--calib <prefix>]
      one layer's derived figures from the runs <prefix>_trace (kernel trace) and <prefix>_A,
      _B, _F, _W (counter passes, see COUNTER_PASSES): MFMA busy, LDS busy, bank conflicts,
      VALU work, HBM bytes (FETCH_SIZE / WRITE_SIZE scaled by the calibration runs
      <calib>_F / <calib>_W of a known-size streaming kernel)

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


# The counter passes of `counters` (each within one pass's hardware limits: 8 SQ, 2 GRBM,
# 4 TCC counters).
COUNTER_PASSES = {
    "A": "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F16 "
         "SQ_LDS_IDX_ACTIVE SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_INSTS_VALU",
    "B": "SQ_WAIT_INST_LDS SQ_ACTIVE_INST_VALU SQ_ACTIVE_INST_LDS SQ_WAIT_ANY SQ_WAVE_CYCLES "
         "SQ_INSTS_SALU SQ_ACTIVE_INST_ANY SQ_INSTS_VMEM_RD",
    "F": "FETCH_SIZE",
    "W": "WRITE_SIZE",
}
CLOCK_GHZ = 2.4      # MI355X peak engine clock
SIMDS, CUS = 1024, 256


def _csv(d, name):
    import glob
    import os
    f = glob.glob(os.path.join(d, "**", name), recursive=True)
    return f[0] if f else None


def _pass_means(d, kernel):
    """Mean per dispatch of every counter of the kernels whose name contains `kernel`."""
    path = _csv(d, "*counter_collection.csv")
    if not path:
        return None
    acc = defaultdict(lambda: defaultdict(float))
    with open(path) as f:
        for r in csv.DictReader(f):
            if kernel in r["Kernel_Name"]:
                acc[r["Dispatch_Id"]][r["Counter_Name"]] += float(r["Counter_Value"])
    if not acc:
        return None
    n = len(acc)
    names = set().union(*(d.keys() for d in acc.values()))
    return {c: sum(d.get(c, 0.0) for d in acc.values()) / n for c in names}


def _trace_mean_us(d, kernel):
    path = _csv(d, "*kernel_trace.csv")
    if not path:
        return None, None
    v, name = [], None
    with open(path) as f:
        for r in csv.DictReader(f):
            if kernel in r["Kernel_Name"]:
                v.append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
                name = short(r["Kernel_Name"])
    return (sum(v) / len(v) if v else None), name


def counters(prefix, kernel, calib):
    us, name = _trace_mean_us(prefix + "_trace", kernel)
    a = _pass_means(prefix + "_A", kernel) or {}
    b = _pass_means(prefix + "_B", kernel) or {}
    fe = (_pass_means(prefix + "_F", kernel) or {}).get("FETCH_SIZE")
    wr = (_pass_means(prefix + "_W", kernel) or {}).get("WRITE_SIZE")
    kf = kw = None
    if calib:
        cf = (_pass_means(calib + "_F", "ew_") or {}).get("FETCH_SIZE")
        cw = (_pass_means(calib + "_W", "ew_") or {}).get("WRITE_SIZE")
        kf = 131072.0 / cf if cf else None  # the calibration pass reads and writes 128 MiB
        kw = 131072.0 / cw if cw else None
    print(f"kernel: {name}")
    if us:
        print(f"mean duration (kernel trace): {us:.2f} us")
    if a and us:
        cyc = us * 1e3 * CLOCK_GHZ
        mf = a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0)
        print(f"MFMA busy: {mf:.0f} SIMD-cycles = {100 * mf / (cyc * SIMDS):.1f} % of {SIMDS} SIMDs x duration "
              f"at {CLOCK_GHZ} GHz; fp16 MFMA work {a.get('SQ_INSTS_VALU_MFMA_MOPS_F16', 0) * 512 / 1e9:.2f} GFLOP")
        lds, bc = a.get("SQ_LDS_IDX_ACTIVE", 0.0), a.get("SQ_LDS_BANK_CONFLICT", 0.0)
        print(f"LDS indexed-active: {100 * lds / (cyc * CUS):.1f} % of {CUS} CUs x duration; bank-conflict cycles "
              f"{bc:.0f} ({100 * bc / lds if lds else 0:.1f} % of LDS-active); LDS instructions {a.get('SQ_INSTS_LDS', 0):.0f}")
        print(f"VALU instructions {a.get('SQ_INSTS_VALU', 0):.0f} (MFMA included)")
    if b:
        wc = b.get("SQ_WAVE_CYCLES", 0.0)
        if wc:
            print(f"wave time: waiting {100 * b.get('SQ_WAIT_ANY', 0) / wc:.1f} %, issuing any instruction "
                  f"{100 * b.get('SQ_ACTIVE_INST_ANY', 0) / wc:.1f} %, waiting on LDS issue "
                  f"{100 * b.get('SQ_WAIT_INST_LDS', 0) / wc:.1f} % (quad-cycle counters)")
    if fe is not None and wr is not None:
        if kf and kw:
            rb, wb = fe * kf * 1024, wr * kw * 1024
            line = f"HBM: read {rb / 1e6:.2f} MB, written {wb / 1e6:.2f} MB per launch"
            if us:
                line += f"; {(rb + wb) / (us * 1e-6) / 1e9:.0f} GB/s"
            print(line + f" (FETCH_SIZE x {kf:.4f}, WRITE_SIZE x {kw:.4f})")
        else:
            print(f"FETCH_SIZE {fe:.1f} KiB, WRITE_SIZE {wr:.1f} KiB per dispatch (unscaled)")


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
    c = sub.add_parser("counters")
    c.add_argument("prefix")
    c.add_argument("--kernel", required=True)
    c.add_argument("--calib", default="")
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        trace(a.csv, a.top, a.grid_min)
    elif a.cmd == "pmc":
        pmc(a.csv, a.kernel)
    else:
        counters(a.prefix, a.kernel, a.calib)


if __name__ == "__main__":
    sys.exit(main())
