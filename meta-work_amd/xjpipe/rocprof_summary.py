"""Summaries of rocprofv3 CSV output for the decode benchmark.

    python -m xjpipe.rocprof_summary trace <dir with *_kernel_stats.csv and *_kernel_trace.csv>
    python -m xjpipe.rocprof_summary traffic <FETCH_SIZE dir> <WRITE_SIZE dir> <copy bytes> [out.json]
    python -m xjpipe.rocprof_summary passes <dir with *_kernel_trace.csv> <number of passes>
    python -m xjpipe.rocprof_summary kernels <FETCH_SIZE dir> <WRITE_SIZE dir> <copy bytes>

trace    per-kernel statistics, and the decode step broken down by kernel
         (steps delimited by the argmax launch that ends each of them)
traffic  HBM bytes per single-token GEMV launch from FETCH_SIZE / WRITE_SIZE
         (KiB per dispatch), each scaled by the factor that makes the same
         counter read the known size of the calibration copy (the largest
         runtime copy-kernel dispatch of the run); the same per dispatch for
         the attention, DeltaNet and prefill kernels (KERNELS_OF_INTEREST)
kernels  HBM bytes per dispatch of every kernel of the run (by template name),
         calibrated as for traffic
passes   the dispatches after the run's longest idle gap (a pause the
         program makes before its timed passes), per pass and kernel

Single-token GEMV launches are the gemv_kernel<1, ...> and gemv_cu_kernel
dispatches (the two launch forms of the same fused dequant-GEMV).
"""
import collections
import csv
import glob
import json
import os
import re
import statistics
import sys


def _one(d, suffix):
    f = glob.glob(os.path.join(d, "*" + suffix))
    if not f:
        raise SystemExit(f"no *{suffix} in {d}")
    return f[0]


def _norm(name):
    return name.replace("void ", "").replace("(anonymous namespace)::", "")


def _short(name):
    return _norm(name).split("(")[0]


def _gemv1(name):
    n = _norm(name)
    return n.startswith("xjk::gemv_kernel<1,") or n.startswith("xjk::gemv_cu_kernel<1,")


def trace(d):
    out = ["| kernel | calls | avg us | total ms | % |", "|---|---:|---:|---:|---:|"]
    for r in list(csv.DictReader(open(_one(d, "_kernel_stats.csv"))))[:16]:
        out.append(f"| `{_short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                   f"{float(r['TotalDurationNs']) / 1e6:.2f} | {float(r['Percentage']):.1f} |")
    rows = list(csv.DictReader(open(_one(d, "_kernel_trace.csv"))))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    # a decode step ends with its argmax launch (which also embeds the next
    # token); steps are the spans between consecutive argmax launches that
    # hold single-token GEMVs only
    ends = [i for i, r in enumerate(rows) if r["Kernel_Name"].startswith("xjk::finalize")]
    several = re.compile(r"xjk::(gemv_kernel|gemv_cu_kernel)<[2-9],|xjk::(gemm_mfma|dc_|conv_silu|prep_kernel)")
    steps = [rows[a + 1:b + 1] for a, b in zip(ends, ends[1:])
             if any(_gemv1(r["Kernel_Name"]) for r in rows[a + 1:b + 1])
             and not any(several.match(_norm(r["Kernel_Name"])) for r in rows[a + 1:b + 1])][2:]
    per = collections.defaultdict(list)
    busy, wall = [], []
    for seg in steps:
        acc = collections.defaultdict(lambda: [0.0, 0])
        for r in seg:
            k = f"{_short(r['Kernel_Name'])} grid {int(r['Grid_Size_X']) // int(r['Workgroup_Size_X'])}x{r['Grid_Size_Y']}"
            acc[k][0] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
            acc[k][1] += 1
        for k, v in acc.items():
            per[k].append(v)
        busy.append(sum(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for r in seg))
        wall.append(int(seg[-1]["End_Timestamp"]) - int(seg[0]["Start_Timestamp"]))
    if not steps:   # a run without decode steps (prefill only): the kernel table alone
        return "\n".join(out)
    out += ["", f"Decode steps analysed: {len(steps)}; kernels per step: {len(steps[-1]) if steps else 0}; "
            f"sum of kernel durations per step (median) {statistics.median(busy) / 1e3:.1f} us; "
            f"first start to last end {statistics.median(wall) / 1e3:.1f} us.", "",
            "| kernel (grid in work-groups) | launches/step | us/step | us/launch |", "|---|---:|---:|---:|"]
    # means over the analysed steps (a decode call's set-up, e.g. its first
    # embedding and copies, falls into one step of each call)
    ns = len(steps)
    for k, v in sorted(per.items(), key=lambda kv: -sum(x[0] for x in kv[1])):
        t, n = sum(x[0] for x in v) / ns / 1e3, sum(x[1] for x in v) / ns
        out.append(f"| `{k}` | {n:.2f} | {t:.1f} | {t / n:.2f} |")
    g1 = [int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) for seg in steps for r in seg
          if _gemv1(r["Kernel_Name"])]
    if g1:
        out += ["", f"Single-token GEMV launches in the decode steps: {len(g1)}, average duration "
                f"{sum(g1) / len(g1) / 1e3:.3f} us."]
    return "\n".join(out)


# kernels whose traffic the summary also lists: decode attention, the DeltaNet
# step, and the prefill's GEMM and chunked-rule kernels
KERNELS_OF_INTEREST = ("attn_part_kernel", "attn_combine_kernel", "kv_store_kernel", "delta_part_kernel",
                       "delta_head_kernel", "gemm_mfma_kernel", "gemm_reduce_kernel", "rms_scale_kernel", "dc_prep",
                       "dc_scan", "delta_prefill_prep_kernel", "conv_silu_kernel", "prep_kernel")


def _counter(d, name):
    rows = list(csv.DictReader(open(_one(d, "_counter_collection.csv"))))
    return [(r["Kernel_Name"], float(r["Counter_Value"])) for r in rows if r["Counter_Name"] == name]


def traffic(dfetch, dwrite, copy_bytes, out_json=None):
    res = {}
    for name, d in (("FETCH_SIZE", dfetch), ("WRITE_SIZE", dwrite)):
        vals = _counter(d, name)
        copies = [v for k, v in vals if k.startswith("__amd_rocclr_copyBuffer")]
        factor = copy_bytes / (max(copies) * 1024.0)
        g1 = [v for k, v in vals if _gemv1(k)]
        res[name] = {"factor": factor, "launches": len(g1), "kib_per_launch_raw": sum(g1) / len(g1),
                     "bytes_per_launch": sum(g1) / len(g1) * 1024.0 * factor}
    total = res["FETCH_SIZE"]["bytes_per_launch"] + res["WRITE_SIZE"]["bytes_per_launch"]
    # the other kernels of the run (by full template name): HBM bytes per dispatch
    others = {}
    for name, d in (("FETCH_SIZE", dfetch), ("WRITE_SIZE", dwrite)):
        factor = res[name]["factor"]
        per = collections.defaultdict(list)
        for k, v in _counter(d, name):
            if any(_norm(k).startswith("xjk::" + f) for f in KERNELS_OF_INTEREST):
                per[_short(k)].append(v)
        for k, v in per.items():
            others.setdefault(k, {"dispatches": len(v)})[name.split("_")[0].lower() + "_bytes"] = round(
                sum(v) / len(v) * 1024.0 * factor)
    doc = {"kernel": "gemv_kernel<1,...> / gemv_cu_kernel (single-token GEMV launches of the decode step)",
           "bytes_per_launch": round(total), "fetch": res["FETCH_SIZE"], "write": res["WRITE_SIZE"],
           "calibration_copy_bytes": copy_bytes, "other_kernels": others}
    if out_json:
        with open(out_json, "w") as f:
            json.dump(doc, f, indent=1)
    return doc


def kernels(dfetch, dwrite, copy_bytes):
    per = collections.defaultdict(dict)
    for name, d in (("FETCH_SIZE", dfetch), ("WRITE_SIZE", dwrite)):
        vals = _counter(d, name)
        factor = copy_bytes / (max(v for k, v in vals if k.startswith("__amd_rocclr_copyBuffer")) * 1024.0)
        acc = collections.defaultdict(list)
        for k, v in vals:
            if not k.startswith("__amd_rocclr"):
                acc[_short(k)].append(v * 1024.0 * factor)
        for k, v in acc.items():
            per[k]["dispatches"] = len(v)
            per[k][name] = sum(v) / len(v)
    out = ["| kernel | dispatches | FETCH MB / dispatch | WRITE MB / dispatch |", "|---|---:|---:|---:|"]
    for k, v in sorted(per.items(), key=lambda kv: -kv[1].get("FETCH_SIZE", 0)):
        out.append(f"| `{k}` | {v['dispatches']} | {v.get('FETCH_SIZE', 0) / 1e6:.2f} | {v.get('WRITE_SIZE', 0) / 1e6:.3f} |")
    return "\n".join(out)


def passes(d, n):
    ev = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                for r in csv.DictReader(open(_one(d, "_kernel_trace.csv"))))
    gap, i0 = max((ev[i + 1][0] - ev[i][1], i) for i in range(len(ev) - 1))
    tail = ev[i0 + 1:]
    acc = collections.defaultdict(lambda: [0, 0])
    for s, e, k in tail:
        acc[_short(k)][0] += 1
        acc[_short(k)][1] += e - s
    busy = sum(v[1] for v in acc.values())
    out = [f"Dispatches after the {gap / 1e6:.1f} ms gap: {len(tail)}; per pass: kernel time {busy / n / 1e3:.1f} us, "
           f"first start to last end {(tail[-1][1] - tail[0][0]) / n / 1e3:.1f} us.", "",
           "| kernel | launches/pass | us/pass | us/launch |", "|---|---:|---:|---:|"]
    for k, (c, t) in sorted(acc.items(), key=lambda x: -x[1][1]):
        out.append(f"| `{k}` | {c / n:.1f} | {t / n / 1e3:.1f} | {t / c / 1e3:.2f} |")
    return "\n".join(out)


if __name__ == "__main__":
    if len(sys.argv) >= 3 and sys.argv[1] == "trace":
        print(trace(sys.argv[2]))
    elif len(sys.argv) >= 5 and sys.argv[1] == "kernels":
        print(kernels(sys.argv[2], sys.argv[3], int(sys.argv[4])))
    elif len(sys.argv) >= 4 and sys.argv[1] == "passes":
        print(passes(sys.argv[2], int(sys.argv[3])))
    elif len(sys.argv) >= 5 and sys.argv[1] == "traffic":
        print(json.dumps(traffic(sys.argv[2], sys.argv[3], int(sys.argv[4]),
                                 sys.argv[5] if len(sys.argv) > 5 else None), indent=1))
    else:
        raise SystemExit(__doc__)
