#!/usr/bin/env python3
"""Summarise rocprofv3 CSV output into the short text records kept under profiles/.

    profile_summary.py trace  --dir D --command "..." [--kernel REGEX]
        Kernel table of a `rocprofv3 --kernel-trace --stats -f csv -d D -- ...` run.

    profile_summary.py traffic --fetch D1 --write D2 --copy-fetch D3 --copy-write D4
                               --kernel REGEX --command "..." [--algorithmic-bytes N] [--launches K]
        HBM bytes per launch of the kernel matching REGEX from one FETCH_SIZE and
        one WRITE_SIZE pass (`rocprofv3 --pmc FETCH_SIZE -f csv -d D1 -- ...`),
        each scaled by what the same counter reads for g4bench's plain copy kernel
        (512 MiB read and 512 MiB written per launch).

    profile_summary.py gaps --dir D --command "..." [--kernel REGEX] [--max-gap US]
        From the per-dispatch kernel trace: median duration per kernel, and the median idle
        time between one kernel's end and the next kernel's start for each pair of kernels that
        follow each other on the stream (gaps above --max-gap, default 20 us, are left out: host
        waits between timed sections).

    profile_summary.py mfma --dir D --kernel REGEX --command "..." [--simds N] [--algorithmic-flops F]
        MFMA utilisation of the kernel matching REGEX from one pass of
        `rocprofv3 --pmc SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE SQ_INSTS_VALU_MFMA_MOPS_F16 -f csv -d D`:
        busy cycles summed over SIMDs / (active cycles of one XCD x SIMDs) (rocprofv3's
        MfmaUtil expression; the CSV's GRBM_GUI_ACTIVE is the sum of the XCDs' equal
        readings), next to rocprofv3's own MfmaUtil, and the f16 MFMA flops issued
        (512 per MOP).

    profile_summary.py counters --dir D [--dir D2 ...] --kernel REGEX --command "..."
        Every counter found for the kernel matching REGEX in the given `--pmc` passes, as a mean
        per dispatch (the rows of one dispatch summed), and each SQ_INSTS_* counter per wave
        when SQ_WAVES is among them.

Counter values are KiB per dispatch. The summary prints `hbm_bytes_per_launch:`,
which bench.py reads as the roofline's `traffic`.
"""
from __future__ import annotations

import argparse
import csv
import re
import statistics
import sys
from pathlib import Path

COPY_BYTES = 512 << 20


def _csvs(d: str, suffix: str) -> list[Path]:
    files = sorted(Path(d).rglob(f"*{suffix}"))
    if not files:
        raise SystemExit(f"no *{suffix} under {d}")
    return files


def counter_per_dispatch(d: str, counter: str, kernel_re: str, reduce: str = "sum") -> tuple[float, int]:
    """Mean counter value over matching dispatches; the rows of one dispatch (one per hardware
    instance) are summed, or with reduce="max" the largest is taken (GRBM_GUI_ACTIVE reads one
    row per XCD, each the whole dispatch's active cycles)."""
    per_dispatch: dict[str, float] = {}
    rx = re.compile(kernel_re)
    for f in _csvs(d, "counter_collection.csv"):
        for row in csv.DictReader(f.open()):
            if row["Counter_Name"] != counter or not rx.search(row["Kernel_Name"]):
                continue
            key = f"{f}:{row['Dispatch_Id']}"
            v = float(row["Counter_Value"])
            if reduce == "max":
                per_dispatch[key] = max(per_dispatch.get(key, 0.0), v)
            else:
                per_dispatch[key] = per_dispatch.get(key, 0.0) + v
    if not per_dispatch:
        raise SystemExit(f"no {counter} rows for kernel /{kernel_re}/ under {d}")
    return statistics.fmean(per_dispatch.values()), len(per_dispatch)


def cmd_trace(a) -> None:
    rows = []
    for f in _csvs(a.dir, "kernel_stats.csv"):
        rows += list(csv.DictReader(f.open()))
    print(f"command: {a.command}")
    print("kernel stats (rocprofv3 --kernel-trace --stats; durations in us)" +
          (f"; kernels matching /{a.kernel}/" if a.kernel else ""))
    print(f"{'kernel':60s} {'calls':>6s} {'avg':>9s} {'min':>9s} {'max':>9s} {'pct':>6s}")
    for r in sorted(rows, key=lambda r: -float(r["TotalDurationNs"])):
        name = r["Name"]
        if a.kernel and not re.search(a.kernel, name):
            continue
        print(f"{name[:60]:60s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.2f} "
              f"{float(r['MinNs']) / 1e3:9.2f} {float(r['MaxNs']) / 1e3:9.2f} {float(r['Percentage']):6.2f}")


def _short(name: str) -> str:
    m = re.search(r"(k_\w+(?:<[^>]*>)?)", name)
    return m.group(1) if m else name[:40]


def cmd_gaps(a) -> None:
    disp = []
    for f in _csvs(a.dir, "kernel_trace.csv"):
        for r in csv.DictReader(f.open()):
            disp.append((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), _short(r["Kernel_Name"])))
    disp.sort()
    dur: dict[str, list[float]] = {}
    gap: dict[tuple[str, str], list[float]] = {}
    for i, (s0, e0, k) in enumerate(disp):
        dur.setdefault(k, []).append((e0 - s0) / 1e3)
        if i + 1 < len(disp):
            s1, _, k1 = disp[i + 1]
            g = (s1 - e0) / 1e3
            if 0 <= g <= a.max_gap:
                gap.setdefault((k, k1), []).append(g)
    rx = re.compile(a.kernel) if a.kernel else None
    print(f"command: {a.command}")
    print("per-dispatch kernel trace (rocprofv3 --kernel-trace); durations and gaps in us, medians" +
          (f"; kernels matching /{a.kernel}/" if a.kernel else ""))
    print(f"{'kernel':44s} {'dispatches':>10s} {'median':>8s}")
    for k, v in sorted(dur.items(), key=lambda kv: -sum(kv[1])):
        if rx and not rx.search(k):
            continue
        print(f"{k:44s} {len(v):10d} {statistics.median(v):8.2f}")
    print(f"{'gap: end of -> start of':60s} {'count':>6s} {'median':>8s}")
    for (k0, k1), v in sorted(gap.items(), key=lambda kv: -len(kv[1])):
        if rx and not (rx.search(k0) and rx.search(k1)):
            continue
        print(f"{k0 + ' -> ' + k1:60s} {len(v):6d} {statistics.median(v):8.2f}")


def cmd_traffic(a) -> None:
    copy_re = r"k_copy"
    cf, _ = counter_per_dispatch(a.copy_fetch, "FETCH_SIZE", copy_re)
    cw, _ = counter_per_dispatch(a.copy_write, "WRITE_SIZE", copy_re)
    fetch_scale = COPY_BYTES / (cf * 1024.0)
    write_scale = COPY_BYTES / (cw * 1024.0)
    kf, nf = counter_per_dispatch(a.fetch, "FETCH_SIZE", a.kernel)
    kw, nw = counter_per_dispatch(a.write, "WRITE_SIZE", a.kernel)
    fetch_b = kf * 1024.0 * fetch_scale
    write_b = kw * 1024.0 * write_scale
    print(f"command: {a.command}")
    print(f"kernel: /{a.kernel}/ ({nf} dispatches in the FETCH_SIZE pass, {nw} in the WRITE_SIZE pass)")
    print(f"copy calibration: FETCH_SIZE {cf:.1f} KiB and WRITE_SIZE {cw:.1f} KiB per 512 MiB copy launch")
    print(f"fetch_scale: {fetch_scale:.4f}")
    print(f"write_scale: {write_scale:.4f}")
    print(f"fetch_kib_per_launch: {kf:.1f}")
    print(f"write_kib_per_launch: {kw:.1f}")
    print(f"hbm_read_bytes_per_launch: {fetch_b:.0f}")
    print(f"hbm_write_bytes_per_launch: {write_b:.0f}")
    print(f"hbm_bytes_per_launch: {fetch_b + write_b:.0f}")
    if a.launches > 1:
        # a step of several launches of the kernel (one per head_dim group), one of each per step:
        # the per-dispatch mean times the launches is the step's bytes
        per_step = (fetch_b + write_b) * a.launches
        print(f"launches_per_step: {a.launches}")
        print(f"hbm_bytes_per_step: {per_step:.0f}")
        if a.algorithmic_bytes:
            print(f"algorithmic_bytes_per_step: {a.algorithmic_bytes}")
            print(f"traffic_over_algorithmic: {per_step / a.algorithmic_bytes:.4f}")
    elif a.algorithmic_bytes:
        print(f"algorithmic_bytes_per_launch: {a.algorithmic_bytes}")
        print(f"traffic_over_algorithmic: {(fetch_b + write_b) / a.algorithmic_bytes:.4f}")


def cmd_mfma(a) -> None:
    busy, n = counter_per_dispatch(a.dir, "SQ_VALU_MFMA_BUSY_CYCLES", a.kernel)
    active_sum, _ = counter_per_dispatch(a.dir, "GRBM_GUI_ACTIVE", a.kernel)
    active = active_sum / a.xcds  # the CSV sums the XCDs' readings; each counts the dispatch's active cycles
    mops, _ = counter_per_dispatch(a.dir, "SQ_INSTS_VALU_MFMA_MOPS_F16", a.kernel)
    try:
        derived, _ = counter_per_dispatch(a.dir, "MfmaUtil", a.kernel)
    except SystemExit:
        derived = None
    print(f"command: {a.command}")
    print(f"kernel: /{a.kernel}/ ({n} dispatches)")
    print(f"sq_valu_mfma_busy_cycles_per_dispatch: {busy:.0f}")
    print(f"grbm_gui_active_cycles_per_dispatch: {active_sum:.0f} (summed over {a.xcds} XCDs; {active:.0f} each)")
    print(f"simds: {a.simds}")
    print(f"mfma_util: {busy / (active * a.simds):.4f}")
    if derived is not None:
        print(f"rocprof_MfmaUtil_percent: {derived:.2f}")
    flops = mops * 512.0
    print(f"mfma_f16_flops_issued_per_dispatch: {flops:.4e}")
    if a.algorithmic_flops:
        print(f"algorithmic_flops_per_dispatch: {a.algorithmic_flops:.4e}")
        print(f"issued_over_algorithmic: {flops / a.algorithmic_flops:.4f}")


def cmd_counters(a) -> None:
    rx = re.compile(a.kernel)
    names: list[str] = []
    for d in a.dir:
        for f in _csvs(d, "counter_collection.csv"):
            for row in csv.DictReader(f.open()):
                if rx.search(row["Kernel_Name"]) and row["Counter_Name"] not in names:
                    names.append(row["Counter_Name"])
    print(f"command: {a.command}")
    vals: dict[str, float] = {}
    for name in names:
        for d in a.dir:
            try:
                v, n = counter_per_dispatch(d, name, a.kernel)
            except SystemExit:
                continue
            vals[name] = v
            print(f"{name}: {v:.0f} per dispatch ({n} dispatches)")
            break
    waves = vals.get("SQ_WAVES")
    if waves:
        for name, v in vals.items():
            if name.startswith("SQ_INSTS_"):
                print(f"{name.lower()}_per_wave: {v / waves:.1f}")


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    sub = ap.add_subparsers(dest="mode", required=True)
    t = sub.add_parser("trace")
    t.add_argument("--dir", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--kernel", default="")
    g = sub.add_parser("gaps")
    g.add_argument("--dir", required=True)
    g.add_argument("--command", required=True)
    g.add_argument("--kernel", default="")
    g.add_argument("--max-gap", type=float, default=20.0)
    f = sub.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        f.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    f.add_argument("--kernel", required=True)
    f.add_argument("--command", required=True)
    f.add_argument("--algorithmic-bytes", type=int, default=0, help="per step when --launches > 1")
    f.add_argument("--launches", type=int, default=1, help="launches of the kernel per step (one of each kind)")
    m = sub.add_parser("mfma")
    m.add_argument("--dir", required=True)
    m.add_argument("--kernel", required=True)
    m.add_argument("--command", required=True)
    m.add_argument("--simds", type=int, default=1024)
    m.add_argument("--xcds", type=int, default=8)
    m.add_argument("--algorithmic-flops", type=float, default=0.0)
    c = sub.add_parser("counters")
    c.add_argument("--dir", required=True, action="append")
    c.add_argument("--kernel", required=True)
    c.add_argument("--command", required=True)
    a = ap.parse_args()
    {"trace": cmd_trace, "gaps": cmd_gaps, "traffic": cmd_traffic, "mfma": cmd_mfma, "counters": cmd_counters}[a.mode](a)


if __name__ == "__main__":
    sys.exit(main())
