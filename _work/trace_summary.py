"""Summarise a rocprofv3 kernel trace (``--kernel-trace --output-format csv``) per kernel and
launch shape: launches, mean and minimum duration, and the idle time between consecutive
dispatches.

    python -m dotnetfoundryllm_amd.trace_summary <run_kernel_trace.csv> [--last N] [--from NAME] [--match TEXT]

``--last N`` keeps only the last N dispatches (the timed decode steps at the end of a bench run);
``--from NAME`` starts at the last dispatch of kernel NAME (e.g. ``k_pf_embed``: the last batched
prefill); ``--match TEXT`` keeps the kernels whose name contains TEXT.
"""
import argparse
import collections
import csv


def _short(name):
    return name.split("(")[0].replace("void ", "").replace("fllm::", "")


def summarise(path, last=0, start=None, match=None):
    rows = list(csv.DictReader(open(path)))
    rows.sort(key=lambda r: int(r["Start_Timestamp"]))
    if start:
        idx = [i for i, r in enumerate(rows) if _short(r["Kernel_Name"]).startswith(start)]
        rows = rows[idx[-1]:] if idx else []
    if match:
        rows = [r for r in rows if match in r["Kernel_Name"]]
    if last:
        rows = rows[-last:]
    agg = collections.OrderedDict()
    gaps = []
    prev_end = None
    for r in rows:
        s, e = int(r["Start_Timestamp"]), int(r["End_Timestamp"])
        key = (_short(r["Kernel_Name"]), int(r["Grid_Size_X"]), int(r["Grid_Size_Y"]), int(r["Workgroup_Size_X"]))
        a = agg.setdefault(key, {"n": 0, "ns": 0, "min": None, "vgpr": r["VGPR_Count"], "lds": r["LDS_Block_Size"]})
        a["n"] += 1
        a["ns"] += e - s
        a["min"] = e - s if a["min"] is None else min(a["min"], e - s)
        if prev_end is not None:
            gaps.append(s - prev_end)
        prev_end = e
    return agg, sorted(gaps)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("trace")
    ap.add_argument("--last", type=int, default=0)
    ap.add_argument("--from", dest="start", default=None)
    ap.add_argument("--match", default=None)
    a = ap.parse_args()
    agg, gaps = summarise(a.trace, a.last, a.start, a.match)
    total = sum(v["ns"] for v in agg.values())
    print("| kernel | grid (threads) | workgroup | VGPRs | launches | mean us | min us | share |")
    print("|---|---|---|---|---|---|---|---|")
    for (name, gx, gy, wg), v in sorted(agg.items(), key=lambda kv: -kv[1]["ns"]):
        grid = f"{gx}x{gy}" if gy > 1 else f"{gx}"
        print(f"| {name} | {grid} | {wg} | {v['vgpr']} | {v['n']} | {v['ns'] / v['n'] / 1e3:.2f} | "
              f"{v['min'] / 1e3:.2f} | {100.0 * v['ns'] / total:.1f}% |")
    print(f"\nkernel time {total / 1e6:.2f} ms over {sum(v['n'] for v in agg.values())} dispatches")
    if gaps:
        print(f"idle between dispatches: median {gaps[len(gaps) // 2] / 1e3:.2f} us, "
              f"p90 {gaps[(9 * len(gaps)) // 10] / 1e3:.2f} us over {len(gaps)} gaps")


if __name__ == "__main__":
    main()
