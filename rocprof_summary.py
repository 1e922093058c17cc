"""Summarise rocprofv3 runs of bench.py into profiles/.

    python rocprof_summary.py --workload C3 --trace T --fetch F --write W [--sq S ...]

T is the output directory of
    rocprofv3 --kernel-trace --stats -d T -o trace --output-format csv -- \
        python3 bench.py --no-cpu --no-d64 --no-features
F and W are the output directories of the two counter runs
    rocprofv3 --pmc FETCH_SIZE -d F -o fetch --output-format csv -- \
        python3 bench.py --no-cpu --no-d64 --no-features --steps 3 --warmup 1 --copy-calibration 256
    rocprofv3 --pmc WRITE_SIZE -d W -o write --output-format csv -- (same bench command)
and each optional S a counter run with up to 8 SQ counters (the two sets the
summaries list). --no-d64 and --no-features keep the traces to the headline
shape's plain kernels.

FETCH_SIZE / WRITE_SIZE are reported in KiB per dispatch. The 256 MiB device
copy that --copy-calibration runs first must read and write 256 MiB; the ratio
of that to what the counters report for it is the scale applied to the
attention kernels' readings. Writes profiles/<kernel>_<workload>.md and
profiles/traffic_bwd_main_<workload>.json (read by bench.py's roofline).
"""
import argparse
import csv
import glob
import json
import os
from collections import defaultdict

ROOT = os.path.dirname(os.path.abspath(__file__))
KERNELS = {"fwd_kernel": "fwd", "bwd_kernel": "bwd_main", "bwd_pre_kernel": "bwd_preprocess"}


def short(name):
    # Only this library's kernels (namespace fa): bench.py also runs torch's
    # SDPA, whose kernels have names such as bwd_kernel_dq.
    if "_ZN2fa" not in name:
        return None
    for k, v in KERNELS.items():
        if k in name:
            return v
    return None


def read_counters(d):
    """{kernel: {counter: [values per dispatch]}} plus raw rows."""
    out = defaultdict(lambda: defaultdict(list))
    rows = []
    for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            rows.append(r)
            k = short(r["Kernel_Name"])
            if k:
                out[k][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return out, rows


def copy_reading(rows, counter):
    # The calibration copy is a device-to-device hipMemcpy, which the runtime
    # runs as its copyBuffer kernel; it is the largest such dispatch.
    vals = [float(r["Counter_Value"]) for r in rows
            if r["Counter_Name"] == counter and "copyBuffer" in r["Kernel_Name"]]
    return max(vals) if vals else None


def read_stats(d):
    stats = {}
    for f in glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            k = short(r["Name"])
            if k:
                stats[k] = {"calls": int(r["Calls"]), "avg_us": float(r["AverageNs"]) / 1e3,
                            "min_us": float(r["MinNs"]) / 1e3, "max_us": float(r["MaxNs"]) / 1e3,
                            "pct": float(r["Percentage"])}
    return stats


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workload", default="C3")
    ap.add_argument("--trace", required=True)
    ap.add_argument("--fetch", required=True)
    ap.add_argument("--write", required=True)
    ap.add_argument("--sq", nargs="*", default=[])
    ap.add_argument("--copy-mib", type=int, default=256)
    ap.add_argument("--out", default=os.path.join(ROOT, "profiles"))
    a = ap.parse_args()

    stats = read_stats(a.trace)
    fetch, frows = read_counters(a.fetch)
    write, wrows = read_counters(a.write)
    kib = a.copy_mib * 1024
    f_cal, w_cal = copy_reading(frows, "FETCH_SIZE"), copy_reading(wrows, "WRITE_SIZE")
    f_scale = kib / f_cal if f_cal else None
    w_scale = kib / w_cal if w_cal else None
    sq = defaultdict(dict)
    for d in a.sq:
        c, _ = read_counters(d)
        for k, v in c.items():
            for n, vals in v.items():
                sq[k][n] = sum(vals) / len(vals)

    os.makedirs(a.out, exist_ok=True)
    # (the headline C3 is bench.py's default configuration)
    cfg = "" if a.workload == "C3" else f" --config {a.workload}"
    cmd_bench = f"python3 bench.py{cfg} --no-cpu --no-d64 --no-features"
    cmd_cnt = f"{cmd_bench} --steps 3 --warmup 1 --copy-calibration {a.copy_mib}"
    cmd_sq = f"{cmd_bench} --steps 3 --warmup 1"
    sq_sets = [
        "SQ_WAVES SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_INSTS_MFMA SQ_INSTS_VALU SQ_INSTS_LDS "
        "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE",
        "SQ_ACTIVE_INST_LDS SQ_ACTIVE_INST_VALU SQ_INSTS_VALU_TRANS_F32 SQ_LDS_BANK_CONFLICT "
        "SQ_WAIT_INST_LDS"]
    for k in ("fwd", "bwd_main", "bwd_preprocess"):
        if k not in stats:
            continue
        fk = sum(fetch[k]["FETCH_SIZE"]) / len(fetch[k]["FETCH_SIZE"]) if fetch[k]["FETCH_SIZE"] else None
        wk = sum(write[k]["WRITE_SIZE"]) / len(write[k]["WRITE_SIZE"]) if write[k]["WRITE_SIZE"] else None
        hbm = None
        if fk is not None and wk is not None and f_scale and w_scale:
            hbm = (fk * f_scale + wk * w_scale) * 1024
        s = stats[k]
        lines = [
            f"# {k} kernel, workload {a.workload}",
            "",
            "Commands (run from the repository root, with `cd /tmp && export TMPDIR=/tmp` first "
            "for rocprofv3's scratch files):",
            "",
            f"    rocprofv3 --kernel-trace --stats -d OUT/trace -o trace --output-format csv -- {cmd_bench}",
            f"    rocprofv3 --pmc FETCH_SIZE -d OUT/fetch -o fetch --output-format csv -- {cmd_cnt}",
            f"    rocprofv3 --pmc WRITE_SIZE -d OUT/write -o write --output-format csv -- {cmd_cnt}",
            *[f"    rocprofv3 --pmc {sq_sets[i]} -d OUT/sq{i} -o sq{i} --output-format csv -- {cmd_sq}"
              for i in range(min(len(a.sq or []), len(sq_sets)))],
            f"    python rocprof_summary.py --workload {a.workload} --trace OUT/trace "
            "--fetch OUT/fetch --write OUT/write" + (" --sq " + " ".join(f"OUT/sq{i}" for i in range(len(a.sq))) if a.sq else ""),
            "",
            "| quantity | value |",
            "|---|---|",
            f"| dispatches traced | {s['calls']} |",
            f"| average duration | {s['avg_us']:.2f} us (min {s['min_us']:.2f}, max {s['max_us']:.2f}) |",
            f"| share of traced GPU time | {s['pct']:.1f}% |",
        ]
        if fk is not None:
            lines.append(f"| FETCH_SIZE per dispatch | {fk:.0f} KiB (copy calibration x{f_scale:.3f}) |")
        if wk is not None:
            lines.append(f"| WRITE_SIZE per dispatch | {wk:.0f} KiB (copy calibration x{w_scale:.3f}) |")
        if hbm is not None:
            lines.append(f"| HBM traffic per dispatch | {hbm / 2**20:.1f} MiB |")
        for n, v in sorted(sq.get(k, {}).items()):
            lines.append(f"| {n} | {v:.0f} |")
        with open(os.path.join(a.out, f"{k}_{a.workload}.md"), "w") as f:
            f.write("\n".join(lines) + "\n")
        if k == "bwd_main" and hbm is not None:
            with open(os.path.join(a.out, f"traffic_bwd_main_{a.workload}.json"), "w") as f:
                json.dump({"kernel": "bwd_main", "workload": a.workload,
                           "hbm_bytes_per_dispatch": round(hbm),
                           "fetch_kib": fk, "write_kib": wk,
                           "fetch_scale": f_scale, "write_scale": w_scale,
                           "avg_us": s["avg_us"]}, f, indent=1)
        print(k, s["avg_us"], fk, wk, hbm)


if __name__ == "__main__":
    main()
