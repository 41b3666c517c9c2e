"""Summaries of rocprofv3 output for the decode path (kernel-trace statistics and PMC
counter passes), written as the short text/JSON files kept under profiles/.

Usage (after the rocprofv3 runs named in each summary):
  python3 -m aethermind_amd.profiling stats  <kernel_stats.csv> --out profiles/X.md --cmd "..."
  python3 -m aethermind_amd.profiling traffic --fetch <counter_collection.csv> --write <counter_collection.csv>
          --copy-fetch <csv> --copy-write <csv> --copy-bytes N --out-md profiles/X.md --out-json profiles/X.json
          --cmd "..."

Traffic method: FETCH_SIZE and WRITE_SIZE (KiB per dispatch, summed over the TCC
channels) are taken for every dispatch of the GEMV kernels in the timed decode tokens,
and each counter is scaled by what it reads for a device-to-device copy of a known
size (factor = copy bytes / (counter KiB * 1024)).
"""

import argparse
import collections
import csv
import json
import re

GEMV_PREFIX = "gemv_kernel"


def _short(name: str) -> str:
    n = re.sub(r"\(anonymous namespace\)::", "", name)
    n = n.replace("am::", "").replace("void ", "")
    n = re.sub(r"\((?:[^()]|\([^()]*\))*\)$", "", n)  # drop the parameter list
    return n.strip()


def _gemv_epilogue(name: str):
    """EPI template argument of a gemv_kernel or gemv_ksplit_kernel instance (0 plain
    store, 1 residual, 2 qkv, 3 gate/up, 4 lm_head), None for other kernels"""
    m = re.search(GEMV_PREFIX + r"<\w+, (\d+), (?:true|false), (\d+),", name)
    if m:
        return int(m.group(2))
    m = re.search(r"gemv_ksplit_kernel<\w+, (\d+), (\d+)>", name)
    return int(m.group(2)) if m else None


def kernel_stats(path: str):
    """rows of (name, calls, total_ns, avg_ns, pct) from a rocprofv3 kernel_stats.csv"""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            rows.append((_short(r["Name"]), int(r["Calls"]), float(r["TotalDurationNs"]), float(r["AverageNs"]),
                         float(r["Percentage"])))
    rows.sort(key=lambda x: -x[2])
    return rows


def counters(path: str, counter: str):
    """{short kernel name: [value per dispatch]} for one counter of a counter_collection.csv"""
    out = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] == counter:
                out[_short(r["Kernel_Name"])].append(float(r["Counter_Value"]))
    return out


def copy_factor(path: str, counter: str, nbytes: int) -> float:
    """bytes per counter KiB, from the copy kernel(s) of a calibration run"""
    vals = []
    for name, v in counters(path, counter).items():
        if "copyBuffer" in name or "copy" in name.lower():
            vals.extend(v)
    if not vals:
        raise SystemExit(f"no copy kernel found in {path}")
    return nbytes / (max(vals) * 1024.0)


def cmd_stats(a):
    rows = kernel_stats(a.csv)
    lines = [f"# rocprofv3 kernel statistics: {a.title}", "", "Command:", "", f"    {a.cmd}", "",
             "| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for name, calls, tot, avg, pct in rows[: a.top]:
        lines.append(f"| `{name[:110]}` | {calls} | {tot / 1e6:.3f} | {avg / 1e3:.2f} | {pct:.1f} |")
    open(a.out, "w").write("\n".join(lines) + "\n")


def cmd_traffic(a):
    ff = copy_factor(a.copy_fetch, "FETCH_SIZE", a.copy_bytes)
    fw = copy_factor(a.copy_write, "WRITE_SIZE", a.copy_bytes)
    fetch = counters(a.fetch, "FETCH_SIZE")
    write = counters(a.write, "WRITE_SIZE")
    per_kernel = {}
    tokens = 0
    for name, vals in fetch.items():
        epi = _gemv_epilogue(name)
        if epi is None or epi == 0:  # the fused decode GEMVs only (not the prefill's plain GEMV rows)
            continue
        if epi == 4:  # one norm + lm_head + argmax launch per decode token
            tokens = len(vals)
        w = write.get(name, [0.0])
        per_kernel[name] = {
            "dispatches": len(vals),
            "fetch_bytes_avg": sum(vals) / len(vals) * 1024.0 * ff,
            "write_bytes_avg": sum(w) / len(w) * 1024.0 * fw,
        }
    tot_launch = sum(k["dispatches"] for k in per_kernel.values())
    tot_bytes = sum(k["dispatches"] * (k["fetch_bytes_avg"] + k["write_bytes_avg"]) for k in per_kernel.values())
    res = {
        "method": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes, each scaled by the same counter for a "
                  f"{a.copy_bytes}-byte device-to-device copy",
        "fetch_factor_bytes_per_kib": ff * 1024.0,
        "write_factor_bytes_per_kib": fw * 1024.0,
        "gemv_launches": tot_launch,
        "tokens": tokens,
        "hbm_bytes_per_token": tot_bytes / tokens if tokens else None,
        "algorithmic_bytes_per_token": a.algorithmic,
        "per_kernel": per_kernel,
        "command": a.cmd,
    }
    json.dump(res, open(a.out_json, "w"), indent=1)
    lines = [f"# HBM traffic of the decode GEMV kernels ({a.title})", "", "Commands:", "", f"    {a.cmd}", "",
             f"Copy calibration: FETCH_SIZE {ff * 1024:.1f} B/KiB-counted, WRITE_SIZE {fw * 1024:.1f} B/KiB-counted "
             f"({a.copy_bytes} B device-to-device copy).", "",
             f"GEMV launches in {tokens} tokens: {tot_launch}; measured HBM bytes per token "
             f"{res['hbm_bytes_per_token'] / 1e9 if res['hbm_bytes_per_token'] else 0:.4f} GB vs algorithmic "
             f"{a.algorithmic / 1e9:.4f} GB.", "",
             "| kernel | dispatches | fetch MB avg | write KB avg |", "|---|---:|---:|---:|"]
    for name, k in sorted(per_kernel.items(), key=lambda kv: -kv[1]["dispatches"] * kv[1]["fetch_bytes_avg"]):
        lines.append(f"| `{name[:100]}` | {k['dispatches']} | {k['fetch_bytes_avg'] / 1e6:.3f} | "
                     f"{k['write_bytes_avg'] / 1e3:.2f} |")
    open(a.out_md, "w").write("\n".join(lines) + "\n")


def main():
    ap = argparse.ArgumentParser()
    sp = ap.add_subparsers(dest="cmd_name", required=True)
    s = sp.add_parser("stats")
    s.add_argument("csv")
    s.add_argument("--out", required=True)
    s.add_argument("--cmd", required=True)
    s.add_argument("--title", default="decode benchmark")
    s.add_argument("--top", type=int, default=20)
    t = sp.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--algorithmic", type=int, required=True)
    t.add_argument("--out-md", required=True)
    t.add_argument("--out-json", required=True)
    t.add_argument("--cmd", required=True)
    t.add_argument("--title", default="INT4 8B-shape decode")
    a = ap.parse_args()
    if a.cmd_name == "stats":
        cmd_stats(a)
    else:
        cmd_traffic(a)


if __name__ == "__main__":
    main()
