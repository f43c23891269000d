"""Summaries of rocprofv3 output for the correction pass (text in, text out; nothing here touches a GPU).

    python -m appcorr_amd.profiling kernel-stats <run_kernel_stats.csv> <passes> <title> <command>
        Markdown table of per-pass kernel time from a `rocprofv3 --kernel-trace --stats -f csv` run of
        bench.py (kernels whose call count is a multiple of the pass count belong to the pass).

    python -m appcorr_amd.profiling traffic <fetch_counter_collection.csv> <write_counter_collection.csv>
            <kernel substring> <calibration kernel substring> <calibration bytes> <json out> <key> <command>
        HBM traffic per launch of one kernel from two `rocprofv3 --pmc FETCH_SIZE` / `--pmc WRITE_SIZE`
        runs. FETCH_SIZE counts 128-byte read requests as 64 bytes on this part, so both counters are
        scaled by what they read for a plain copy of known size in the same run (bench.py
        --calib-copy-mib: the library's row-copy kernel, 16-byte lanes like the GEMM operand loads).
        Prints a markdown summary and merges {key: {...}} into the JSON file that bench.py reads.

    python -m appcorr_amd.profiling kernels <kernel_trace.csv> <fetch_counter_collection.csv>
            <write_counter_collection.csv> <calibration kernel substring> <calibration bytes>
            <kernel substrings, comma-separated> <title> <command>
        Markdown table per (kernel, grid size): median duration from a `--kernel-trace` run and HBM
        read / write bytes per dispatch from the two counter runs, scaled as in `traffic`. For the
        standalone kernels of `python -m appcorr_amd.kernel_bench --calib-copy-mib 1024`.

    python -m appcorr_amd.profiling bench-table <title> <command> <bench line file>...
        Markdown table of bench.py lines (one JSON line per file; FILE.args beside FILE.json holds the
        arguments of that run).

    python -m appcorr_amd.profiling stalls <kernel_trace.csv> <counter_collection.csv,...>
            <kernel substrings, comma-separated> <title> <command>
        Markdown table per kernel of the memory-path and issue counters of several `rocprofv3 --pmc`
        runs (L2 latency and hit rate, fabric latency of L2 misses, texture-data waits, LDS bank
        conflicts, wave issue / wait fractions, TLB misses).

    python -m appcorr_amd.profiling mfma <kernel_trace.csv> <sq_counter_collection.csv>
            <kernel substrings, comma-separated> <title> <command>
        Markdown table per (kernel, grid size) of the matrix-core counters of one `rocprofv3 --pmc`
        run (SQ_INSTS_MFMA, SQ_INSTS_VALU, SQ_INSTS_VALU_MFMA_MOPS_BF16, SQ_VALU_MFMA_BUSY_CYCLES) with
        the median duration from a `--kernel-trace` run.
"""

from __future__ import annotations

import csv
import json
import os
import re
import sys
from collections import defaultdict


def _short(name: str) -> str:
    n = re.sub(r"\(.*", "", name).replace("void ", "")
    return n if len(n) < 90 else n[:87] + "..."


def kernel_stats(path: str, passes: int, title: str, cmd: str) -> str:
    rows = list(csv.DictReader(open(path)))
    per = [r for r in rows if int(r["Calls"]) % passes == 0]
    setup = [r for r in rows if int(r["Calls"]) % passes != 0]
    ptot = sum(float(r["TotalDurationNs"]) for r in per)
    out = [f"# {title}", "", "Command (run from the repository root on one MI355X):", "", "```", cmd, "```", "",
           f"`rocprofv3 --kernel-trace --stats` kernel_stats.csv, {passes} passes in the trace "
           "(warm-up + timed); per-pass time = total / passes.", "",
           "| kernel | calls | avg us | per-pass us | share |", "|---|---:|---:|---:|---:|"]
    for r in sorted(per, key=lambda r: -float(r["TotalDurationNs"])):
        t = float(r["TotalDurationNs"])
        if t / ptot < 0.001:
            continue
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{t / passes / 1e3:.1f} | {100 * t / ptot:.1f}% |")
    out.append(f"| **one pass, all kernels** | | | **{ptot / passes / 1e3:.1f}** | 100% |")
    out += ["", "One-time setup kernels in the same trace (synthetic data and cache generation, not part of a pass):",
            ""]
    out += [f"- `{_short(r['Name'])}`: {r['Calls']} calls, {float(r['TotalDurationNs']) / 1e3:.0f} us total"
            for r in setup if float(r["TotalDurationNs"]) > 20000]
    return "\n".join(out)


def traffic(fetch_csv: str, write_csv: str, kernel: str, calib: str, calib_bytes: float, json_out: str, key: str,
            cmd: str) -> str:
    f, w = _groups(fetch_csv, "Counter_Value"), _groups(write_csv, "Counter_Value")

    def pick(d, sub):
        # the launch grid with the most dispatches of the kernel (a pass's launches, not set-up work
        # such as the approximate pass that fills the caches, which may run the same kernel on more rows)
        groups = [k for k in d if sub in k[0]]
        if not groups:
            raise SystemExit(f"no kernel matching {sub!r}")
        key = max(groups, key=lambda k: len(d[k]))
        vals = d[key]
        return key[0], sum(vals) / len(vals), len(vals)

    def largest(d, sub):  # the calibration copy is the largest dispatch of its kernel in the run
        vals = [v for k in d if sub in k[0] for v in d[k]]
        if not vals:
            raise SystemExit(f"no kernel matching {sub!r}")
        return max(vals)

    kname, kf, nk = pick(f, kernel)
    _, kw, _ = pick(w, kernel)
    cf, cw = largest(f, calib), largest(w, calib)
    # The calibration copy reads its rows plus 16 bytes of row indices per 4 KiB row.
    f_scale = calib_bytes * (1.0 + 16.0 / 4096.0) / (cf * 1024.0)
    w_scale = calib_bytes / (cw * 1024.0)
    fetch_b = kf * 1024.0 * f_scale
    write_b = kw * 1024.0 * w_scale
    rec = {"kernel": _short(kname), "fetch_bytes": round(fetch_b), "write_bytes": round(write_b),
           "traffic_bytes": round(fetch_b + write_b), "fetch_kib_raw": round(kf, 1), "write_kib_raw": round(kw, 1),
           "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4), "dispatches": nk}
    data = {}
    if os.path.exists(json_out):
        data = json.load(open(json_out))
    data[key] = rec
    with open(json_out, "w") as fh:
        json.dump(data, fh, indent=1, sort_keys=True)
        fh.write("\n")
    lines = [f"# HBM traffic per launch: {key}", "", "Commands (run from the repository root on one MI355X):", "",
             "```", cmd, "```", "",
             f"- kernel: `{rec['kernel']}` ({nk} dispatches averaged)",
             f"- FETCH_SIZE {kf:.1f} KiB/dispatch x {f_scale:.4f} = {fetch_b / 1e6:.2f} MB",
             f"- WRITE_SIZE {kw:.1f} KiB/dispatch x {w_scale:.4f} = {write_b / 1e6:.2f} MB",
             f"- traffic per launch: {(fetch_b + write_b) / 1e6:.2f} MB",
             f"- scale factors: the same counters over a {calib_bytes / 2**20:.0f} MiB row copy "
             f"(`{calib}`) read {cf:.0f} / {cw:.0f} KiB for {calib_bytes / 1024:.0f} KiB moved each way"]
    return "\n".join(lines)


def _groups(path: str, value_col: str):
    """{(kernel name, grid threads): [values]} of a rocprofv3 CSV (per-dispatch rows)."""
    acc = defaultdict(list)
    for r in csv.DictReader(open(path)):
        if "Grid_Size" in r:
            thr = int(r["Grid_Size"])
        else:
            thr = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        v = (float(r["End_Timestamp"]) - float(r["Start_Timestamp"])) if value_col == "duration" else \
            float(r[value_col])
        acc[(r["Kernel_Name"], thr)].append(v)
    return acc


def kernels(trace_csv: str, fetch_csv: str, write_csv: str, calib: str, calib_bytes: float, subs, title: str,
            cmd: str) -> str:
    """Per (kernel, grid) of every kernel whose name contains one of `subs`: dispatches, average
    duration (kernel trace) and HBM bytes per dispatch (FETCH_SIZE / WRITE_SIZE runs, scaled by what
    the same counters read for the calibration copy, as in `traffic`)."""
    dur = _groups(trace_csv, "duration")
    f = _groups(fetch_csv, "Counter_Value")
    w = _groups(write_csv, "Counter_Value")
    cf = max(v for (n, _), vals in f.items() if calib in n for v in vals)
    cw = max(v for (n, _), vals in w.items() if calib in n for v in vals)
    f_scale = calib_bytes * (1.0 + 16.0 / 4096.0) / (cf * 1024.0)
    w_scale = calib_bytes / (cw * 1024.0)
    lines = [f"# {title}", "", "Commands (run from the repository root on one MI355X):", "", "```", cmd, "```", "",
             f"Scale factors from the calibration copy (`{calib}`, {calib_bytes / 2**20:.0f} MiB of 4 KiB rows, "
             f"the largest dispatch of that kernel in each run): FETCH_SIZE x {f_scale:.4f}, WRITE_SIZE x "
             f"{w_scale:.4f}.", "",
             "| kernel | grid threads | dispatches | avg us (trace) | HBM read MB | HBM write MB | HBM GB/s |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for key in sorted(dur, key=lambda k: (_short(k[0]), k[1])):
        name, thr = key
        if not any(sub in name for sub in subs) or key not in f or key not in w:
            continue
        d = sorted(dur[key])
        # the calibration copy is not a timed launch of its kernel: leave out the largest dispatch
        if calib in name and len(d) > 1:
            d = d[:-1]
        us = d[len(d) // 2] / 1e3
        fb = sum(f[key]) / len(f[key]) * 1024.0 * f_scale
        wb = sum(w[key]) / len(w[key]) * 1024.0 * w_scale
        lines.append(f"| `{_short(name)}` | {thr} | {len(d)} | {us:.2f} | {fb / 1e6:.2f} | {wb / 1e6:.2f} | "
                     f"{(fb + wb) / (us * 1e3):.0f} |")
    return "\n".join(lines)


def mfma(trace_csv: str, sq_csv: str, subs, title: str, cmd: str) -> str:
    """Per (kernel, grid) of the kernels named by `subs`: MFMA and VALU instruction counts, the bf16 MFMA
    work (SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 FLOP), the matrix-pipe busy cycles, and the median
    duration from a kernel-trace run; the pipe's busy fraction is taken against 1024 SIMDs at the
    2.4 GHz the 2.5 PFLOP/s dense bf16 peak is quoted at."""
    dur = _groups(trace_csv, "duration")
    cnt = defaultdict(lambda: defaultdict(list))
    for r in csv.DictReader(open(sq_csv)):
        thr = int(r["Grid_Size"]) if "Grid_Size" in r else \
            int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
        cnt[(r["Kernel_Name"], thr)][r["Counter_Name"]].append(float(r["Counter_Value"]))
    lines = [f"# {title}", "", "Commands (run from the repository root on one MI355X):", "", "```", cmd, "```", "",
             "Counters averaged per dispatch; FLOP = SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512; MFMA busy = "
             "SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x 2.4 GHz x duration).", "",
             "| kernel | grid threads | dispatches | avg us (trace) | GFLOP | TFLOP/s | MFMA insts | VALU insts | "
             "VALU : MFMA | MFMA busy |", "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for key in sorted(cnt, key=lambda k: (_short(k[0]), k[1])):
        name, thr = key
        if not any(sub in name for sub in subs) or key not in dur:
            continue
        c = {n: sum(v) / len(v) for n, v in cnt[key].items()}
        d = sorted(dur[key])
        us = d[len(d) // 2] / 1e3
        flop = c.get("SQ_INSTS_VALU_MFMA_MOPS_BF16", 0.0) * 512.0
        mf, va = c.get("SQ_INSTS_MFMA", 0.0), c.get("SQ_INSTS_VALU", 0.0)
        busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (1024 * 2.4e3 * us)
        n = len(next(iter(cnt[key].values())))
        lines.append(f"| `{_short(name)}` | {thr} | {n} | {us:.2f} | {flop / 1e9:.2f} | {flop / us / 1e6:.0f} | "
                     f"{mf:.0f} | {va:.0f} | {va / mf if mf else float('nan'):.1f} | {100 * busy:.1f}% |")
    return "\n".join(lines)


# Derived figures of the stall summary: (label, numerator counter, denominator counter, format).
_STALL_RATIOS = [
    ("L2 read latency seen by the vector L1 (clk)", "TCP_TCC_READ_REQ_LATENCY_sum", "TCP_TCC_READ_REQ_sum", "{:.0f}"),
    ("L2 hit rate", "TCC_HIT_sum", None, "{:.2f}"),
    ("L2-miss fabric latency (clk)", "TCC_EA0_RDREQ_LEVEL_sum", "TCC_EA0_RDREQ_sum", "{:.0f}"),
    ("TD waiting on L2 data / TD busy", "TD_TC_STALL_sum", "TD_TD_BUSY_sum", "{:.2f}"),
    ("LDS bank-conflict cycles / LDS-active cycles", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "{:.3f}"),
    ("wave cycles waiting (any)", "SQ_WAIT_ANY", "SQ_WAVE_CYCLES", "{:.2f}"),
    ("wave cycles waiting to issue", "SQ_WAIT_INST_ANY", "SQ_WAVE_CYCLES", "{:.2f}"),
    ("wave cycles issuing", "SQ_ACTIVE_INST_ANY", "SQ_WAVE_CYCLES", "{:.2f}"),
    ("UTCL1 (TLB) misses per dispatch", "TCP_UTCL1_TRANSLATION_MISS_sum", None, "{:.0f}"),
]


def stalls(trace_csv: str, counter_csvs, subs, title: str, cmd: str) -> str:
    """Per (kernel, grid) of the kernels named by `subs`: the memory-path and issue counters of several
    `rocprofv3 --pmc` runs (one counter group each) averaged per dispatch, and the ratios of
    _STALL_RATIOS, with the median duration from a `--kernel-trace` run."""
    dur = _groups(trace_csv, "duration")
    cnt = defaultdict(lambda: defaultdict(list))
    for path in counter_csvs:
        for r in csv.DictReader(open(path)):
            thr = int(r["Grid_Size"]) if "Grid_Size" in r else \
                int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            cnt[(r["Kernel_Name"], thr)][r["Counter_Name"]].append(float(r["Counter_Value"]))
    keys = [k for k in sorted(cnt, key=lambda k: (_short(k[0]), k[1])) if any(x in k[0] for x in subs) and k in dur]
    lines = [f"# {title}", "", "Commands (run from the repository root on one MI355X):", "", "```", cmd, "```", "",
             "Counters averaged per dispatch (each counter group from its own run of the same command).", "",
             "| figure | " + " | ".join(f"`{_short(k[0])}`" for k in keys) + " |",
             "|---|" + "---:|" * len(keys)]
    avg = [{n: sum(v) / len(v) for n, v in cnt[k].items()} for k in keys]
    lines.append("| median duration (us, trace) | " +
                 " | ".join(f"{sorted(dur[k])[len(dur[k]) // 2] / 1e3:.2f}" for k in keys) + " |")
    for label, num, den, fmt in _STALL_RATIOS:
        vals = []
        for c in avg:
            if num not in c or (den is not None and den not in c):
                vals.append("-")
                continue
            if num == "TCC_HIT_sum":
                tot = c["TCC_HIT_sum"] + c.get("TCC_MISS_sum", 0.0)
                vals.append(fmt.format(c[num] / tot) if tot else "-")
            elif den is None:
                vals.append(fmt.format(c[num]))
            else:
                vals.append(fmt.format(c[num] / c[den]) if c[den] else "-")
        lines.append(f"| {label} | " + " | ".join(vals) + " |")
    return "\n".join(lines)


def bench_table(paths, title: str, cmd: str) -> str:
    """Markdown table of bench.py lines: each path is a file whose last line is one bench JSON line, and
    the same path with `.args` in place of `.json` holds the arguments it ran with."""
    lines = [f"# {title}", "", "Commands (run from the repository root on one MI355X):", "", "```", cmd, "```", "",
             "| args | workload | B | keep | rows M | precision | ms / pass | corrected tokens/s | pass TFLOP/s | "
             "dominant site (frac of peak) | sites (us) |", "|---|---|---:|---:|---:|---|---:|---:|---:|---|---|"]
    for path in paths:
        d = json.loads(open(path).read().strip().splitlines()[-1])
        ap = path[:-5] + ".args" if path.endswith(".json") else path + ".args"
        args = open(ap).read().strip() if os.path.exists(ap) else ""
        c = d["config"]
        roof = d.get("roofline") or {}
        sites = ", ".join(f"{k} {v['avg_us']:.1f}" for k, v in (roof.get("sites") or {}).items())
        dom = f"{roof.get('kernel')} ({roof.get('frac', 0):.3f})" if roof else "-"
        lines.append(f"| `{args or '(default)'}` | {c['workload']} | {c['batch']} | {c['keep_ratio']} | "
                     f"{c['selected_rows']} | {c['correct_precision']} | {d['ms_per_step']:.3f} | {d['value']:,.0f} | "
                     f"{c['pass_tflops_achieved']} | {dom} | {sites} |")
    return "\n".join(lines)


def main(argv):
    if len(argv) >= 5 and argv[0] == "kernel-stats":
        print(kernel_stats(argv[1], int(argv[2]), argv[3], argv[4]))
    elif len(argv) >= 9 and argv[0] == "traffic":
        print(traffic(argv[1], argv[2], argv[3], argv[4], float(argv[5]), argv[6], argv[7], argv[8]))
    elif len(argv) >= 6 and argv[0] == "mfma":
        print(mfma(argv[1], argv[2], argv[3].split(","), argv[4], argv[5]))
    elif len(argv) >= 4 and argv[0] == "bench-table":
        print(bench_table(argv[3:], argv[1], argv[2]))
    elif len(argv) >= 6 and argv[0] == "stalls":
        print(stalls(argv[1], argv[2].split(","), argv[3].split(","), argv[4], argv[5]))
    elif len(argv) >= 9 and argv[0] == "kernels":
        print(kernels(argv[1], argv[2], argv[3], argv[4], float(argv[5]), argv[6].split(","), argv[7], argv[8]))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
