"""Summarise rocprofv3 CSV output into the short text tables kept under profiles/.

    python -m neutrongt_amd.profsum trace <dir>/run_kernel_stats.csv
    python -m neutrongt_amd.profsum pmc <fetch_dir> <write_dir> [<tcc_dir>]
    python -m neutrongt_amd.profsum counters <dir>
    python -m neutrongt_amd.profsum traffic <config> <fetch_dir> <write_dir>

``trace`` prints per-kernel call count and mean/min/max duration.  ``counters``
prints the mean per dispatch of every counter of one ``--pmc`` run for the
library's kernels.  ``traffic`` prints the calibrated read/write bytes per
dispatch as the JSON records bench.py reads (keyed ``config:timer name``).  ``pmc``
prints per-kernel FETCH_SIZE / WRITE_SIZE (KiB per dispatch, mean over the
dispatches of that kernel) and their values scaled by the calibration factor
read from the largest plain device copy in the same run (a 512 MiB
``__amd_rocclr_copyBuffer`` when bench.py runs with --calib-copy):
factor = copy bytes / counter reading.
"""
from __future__ import annotations

import collections
import csv
import re
import sys
from pathlib import Path


def short_name(name: str) -> str:
    m = re.search(r"ngt::\(anonymous namespace\)::(\w+)<([^>]*)>", name)
    if m:
        t = m.group(2).replace("ngt::bf16_t", "bf16").replace("float", "f32").replace(" ", "")
        return f"{m.group(1)}<{t}>"
    m = re.search(r"ngt::\(anonymous namespace\)::(\w+)", name)
    if m:
        return m.group(1)
    return name.split("(")[0][:60]


def trace_table(stats_csv: str) -> str:
    rows = list(csv.DictReader(open(stats_csv)))
    out = ["| kernel | calls | mean us | min us | max us | % time |", "|---|---|---|---|---|---|"]
    for r in rows:
        out.append(f"| {short_name(r['Name'])} | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
                   f"{float(r['Percentage']):.2f} |")
    return "\n".join(out)


def _counters(d: str):
    vals = collections.defaultdict(lambda: collections.defaultdict(list))
    f = next(Path(d).rglob("*counter_collection.csv"))
    for r in csv.DictReader(open(f)):
        vals[r["Kernel_Name"]][r["Counter_Name"]].append(float(r["Counter_Value"]))
    return vals


def pmc_table(fetch_dir: str, write_dir: str, tcc_dir: str | None = None) -> str:
    fe, wr = _counters(fetch_dir), _counters(write_dir)
    tc = _counters(tcc_dir) if tcc_dir else {}
    copy = [k for k in fe if "copyBuffer" in k]
    cf = cw = 1.0
    note = "no calibration copy found: factors 1.0"
    if copy:
        f_max = max(max(fe[k]["FETCH_SIZE"]) for k in copy)
        w_max = max(max(wr[k]["WRITE_SIZE"]) for k in copy if k in wr)
        copy_kib = 512 * 1024.0
        cf, cw = copy_kib / f_max, copy_kib / w_max
        note = (f"calibration: 512 MiB device copy read FETCH_SIZE={f_max:.0f} KiB, "
                f"WRITE_SIZE={w_max:.0f} KiB -> factors read x{cf:.3f}, write x{cw:.3f}")
    out = [note, "",
           "| kernel | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | L2->fabric read MB (scaled) | "
           "L2->fabric write MB (scaled) | L2 hit |",
           "|---|---|---|---|---|---|---|"]
    for k, c in fe.items():
        if "ngt::" not in k:
            continue
        f = sum(c["FETCH_SIZE"]) / len(c["FETCH_SIZE"])
        w = wr.get(k, {}).get("WRITE_SIZE", [float("nan")])
        w = sum(w) / len(w)
        hit = ""
        if k in tc and tc[k].get("TCC_HIT_sum"):
            h = sum(tc[k]["TCC_HIT_sum"])
            m = sum(tc[k]["TCC_MISS_sum"])
            hit = f"{h / max(h + m, 1):.2f}"
        out.append(f"| {short_name(k)} | {len(c['FETCH_SIZE'])} | {f:.0f} | {w:.0f} | "
                   f"{f * cf * 1024 / 1e6:.1f} | {w * cw * 1024 / 1e6:.1f} | {hit} |")
    return "\n".join(out)


# kernel symbol -> the timer name the library records for its launches
TIMER_NAMES = {"k_fwd": "sparse_fwd", "k_bwd_kv": "sparse_bwd_kv", "k_bwd_q": "sparse_bwd_q",
               "k_rowstat": "sparse_rowstat", "k_mf_fwd": "dense_fwd",
               "k_mf_bwd_kv": "dense_bwd_kv", "k_mf_bwd_q": "dense_bwd_q",
               "k_dense_fwd": "dense_fwd", "k_dense_bwd_kv": "dense_bwd_kv",
               "k_dense_bwd_q": "dense_bwd_q", "k_dense_rowstat": "dense_rowstat",
               "k_dense_combine": "dense_combine", "k_dense_scores": "dense_scores"}


def _calibration(fe, wr):
    copy = [k for k in fe if "copyBuffer" in k]
    if not copy:
        raise SystemExit("no calibration copy in the run (bench.py --calib-copy)")
    f_max = max(max(fe[k]["FETCH_SIZE"]) for k in copy)
    w_max = max(max(wr[k]["WRITE_SIZE"]) for k in copy if k in wr)
    return 512 * 1024.0 / f_max, 512 * 1024.0 / w_max


def counters_table(d: str) -> str:
    vals = _counters(d)
    names = sorted({c for k in vals for c in vals[k]})
    out = ["| kernel | dispatches | " + " | ".join(names) + " |",
           "|---|---|" + "---|" * len(names)]
    for k, c in vals.items():
        if "ngt::" not in k:
            continue
        n = max(len(v) for v in c.values())
        cells = [f"{sum(c[m]) / len(c[m]):.4g}" if c.get(m) else "" for m in names]
        out.append(f"| {short_name(k)} | {n} | " + " | ".join(cells) + " |")
    return "\n".join(out)


def traffic_json(config: str, fetch_dir: str, write_dir: str) -> str:
    import json

    fe, wr = _counters(fetch_dir), _counters(write_dir)
    cf, cw = _calibration(fe, wr)
    rec = {}
    for k, c in fe.items():
        base = short_name(k).split("<")[0]
        if base not in TIMER_NAMES or k not in wr:
            continue
        f = sum(c["FETCH_SIZE"]) / len(c["FETCH_SIZE"]) * 1024 * cf
        w = sum(wr[k]["WRITE_SIZE"]) / len(wr[k]["WRITE_SIZE"]) * 1024 * cw
        rec[f"{config}:{TIMER_NAMES[base]}"] = {"read_bytes": round(f), "write_bytes": round(w)}
    return json.dumps(rec, indent=1)


def main(argv):
    if len(argv) >= 2 and argv[0] == "trace":
        print(trace_table(argv[1]))
    elif len(argv) >= 3 and argv[0] == "pmc":
        print(pmc_table(argv[1], argv[2], argv[3] if len(argv) > 3 else None))
    elif len(argv) >= 2 and argv[0] == "counters":
        print(counters_table(argv[1]))
    elif len(argv) >= 4 and argv[0] == "traffic":
        print(traffic_json(argv[1], argv[2], argv[3]))
    else:
        print(__doc__)
        return 2
    return 0


if __name__ == "__main__":
    sys.exit(main(sys.argv[1:]))
