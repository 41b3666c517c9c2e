"""Summaries of rocprofv3 output for the decode path (kernel-trace statistics and PMC
counter passes), written as the short text/JSON files kept under profiles/.

Usage (after the rocprofv3 runs named in each summary):
  python3 -m aethermind_amd.profiling stats  <kernel_stats.csv> --out profiles/X.md --cmd "..."
  python3 -m aethermind_amd.profiling traffic --fetch <counter_collection.csv> --write <counter_collection.csv>
          --copy-fetch <csv> --copy-write <csv> --copy-bytes N [--trace <kernel_trace.csv>]
          [--kernels REGEX] --out-md profiles/X.md --out-json profiles/X.json --cmd "..."
  python3 -m aethermind_amd.profiling mfma --pmc <counter_collection.csv> --trace <kernel_trace.csv>
          [--kernels REGEX] [--shape "KERNEL@GRID[@BUSY]=label:MxNxK" ...] --out profiles/X.md --cmd "..."
  python3 -m aethermind_amd.profiling digest      (the source digest of the native library)

Traffic method: FETCH_SIZE and WRITE_SIZE (KiB per dispatch, summed over the TCC
channels) are taken for every dispatch of the selected kernels (default: the fused
decode GEMVs and decode attention), and each counter is scaled by what it reads for a
device-to-device copy of a known size (factor = copy bytes / (counter KiB * 1024)).
With --trace, each kernel's average device duration from a kernel-trace run of the
same command gives its achieved GB/s (measured bytes / duration).

Every summary records the source digest of the native library it was measured on
(sha256 over aethermind_amd/csrc/**/*.{hip,cpp,h}, path and content), so a reader
can tell whether the figures still describe the current code.
"""

import argparse
import collections
import csv
import hashlib
import json
import os
import re
import subprocess

GEMV_PREFIX = "gemv_kernel"
DEFAULT_KERNELS = r"^(gemv_kernel|gemv_ksplit_kernel|attention_decode_kernel)<"
CSRC = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc")


def source_digest(root: str = CSRC) -> str:
    """sha256 over the native library's sources (relative path and bytes of every
    .hip / .cpp / .h under csrc, in sorted order)"""
    h = hashlib.sha256()
    files = []
    for d, dirs, names in os.walk(root):
        dirs[:] = sorted(x for x in dirs if not x.startswith("_"))
        files += [os.path.join(d, n) for n in names if n.endswith((".hip", ".cpp", ".h"))]
    for f in sorted(files):
        h.update(os.path.relpath(f, root).encode() + b"\0")
        with open(f, "rb") as fh:
            h.update(fh.read())
        h.update(b"\0")
    return h.hexdigest()


def git_commit() -> str:
    try:
        return subprocess.run(["git", "rev-parse", "--short=12", "HEAD"], cwd=CSRC, capture_output=True, text=True,
                              check=True).stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return "unknown"


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


def durations(path: str):
    """{short kernel name: [device ns per dispatch]} from a rocprofv3 kernel_trace.csv"""
    out = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            out[_short(r["Kernel_Name"])].append(float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
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


def _grouped(path: str, value_of):
    """{(short kernel name, grid threads): [value per dispatch]} over a rocprofv3 csv"""
    out = collections.defaultdict(list)
    with open(path) as f:
        for r in csv.DictReader(f):
            grid = r.get("Grid_Size")
            if grid is None:
                grid = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
            v = value_of(r)
            if v is not None:
                out[(_short(r["Kernel_Name"]), int(grid))].append(v)
    return out


def _median(v):
    v = sorted(v)
    return v[len(v) // 2] if len(v) % 2 else 0.5 * (v[len(v) // 2 - 1] + v[len(v) // 2])


MFMA_SIMDS = 1024      # 256 CUs x 4 SIMDs
MFMA_CLOCK_HZ = 2.4e9  # peak engine clock
BF16_PEAK_TFLOPS = 2500.0


def cmd_mfma(a):
    busy = _grouped(a.pmc, lambda r: float(r["Counter_Value"]) if r["Counter_Name"] == "SQ_VALU_MFMA_BUSY_CYCLES"
                    else None)
    dur = _grouped(a.trace, lambda r: float(r["End_Timestamp"]) - float(r["Start_Timestamp"]))
    shapes = {}
    for sh in a.shape:  # KERNEL@GRID[@BUSY]=label:MxNxK
        key, val = sh.split("=", 1)
        parts = key.split("@")
        label, mnk = val.split(":")
        m, n, k = (int(x) for x in mnk.lower().split("x"))
        shapes[(parts[0], int(parts[1]), int(parts[2]) if len(parts) > 2 else 0)] = (label, m, n, k)
    sel = re.compile(a.kernels)
    lines = [f"# Prefill GEMM on MFMA: utilisation per shape ({a.title})", "", "Commands:", ""]
    lines += [f"    {c}" for c in a.cmd] + ["",
              f"Measured at commit {a.commit or git_commit()} (native source digest {source_digest()[:16]}).", "",
              "Duration: median device time over the dispatches of the kernel-trace run.  MFMA busy: median "
              "SQ_VALU_MFMA_BUSY_CYCLES per dispatch (16 per v_mfma_f32_16x16x32_bf16, summed over the SIMDs); "
              f"busy / SIMD-cycles = busy / (duration x {MFMA_CLOCK_HZ / 1e9:.1f} GHz x {MFMA_SIMDS} SIMDs).  "
              "TFLOP/s counts the useful 2 M N K only.", "",
              "| kernel | grid (threads) | projection | M x N x K | dispatches | median us | TFLOP/s | % of 2.5 PF "
              "| MFMA busy cycles | busy / SIMD-cycles |", "|---|---:|---|---|---:|---:|---:|---:|---:|---:|"]
    rows = []
    for key in busy:
        name, grid = key
        if not sel.search(name) or key not in dur:
            continue
        # one (kernel, grid) can serve several shapes (e.g. o_proj and down_proj): split
        # its dispatches by their exact MFMA busy count, and its trace durations in the
        # same proportions, the smaller busy count taking the shorter durations
        clusters = collections.Counter(busy[key])
        d_sorted = sorted(dur[key])
        total = sum(clusters.values())
        at = 0
        for b, cnt in sorted(clusters.items()):
            take = max(1, round(len(d_sorted) * cnt / total))
            part = d_sorted[at:at + take] or d_sorted[-1:]
            at += take
            rows.append((name, grid, b, len(part), _median(part) / 1e3))
    for name, grid, b, n_disp, us in sorted(rows, key=lambda r: -r[2]):
        util = b / (us * 1e-6 * MFMA_CLOCK_HZ * MFMA_SIMDS)
        label, m, n, k = shapes.get((name, grid, int(b)), shapes.get((name, grid, 0), ("?", 0, 0, 0)))
        tf = 2.0 * m * n * k / (us * 1e-6) / 1e12 if m else 0.0
        lines.append(f"| `{name[:60]}` | {grid} | {label} | {m} x {n} x {k} | {n_disp} | {us:.1f} | "
                     f"{tf:.0f} | {100 * tf / BF16_PEAK_TFLOPS:.1f} | {b:.0f} | {100 * util:.1f}% |")
    if a.note:
        lines += ["", a.note]
    open(a.out, "w").write("\n".join(lines) + "\n")


def cmd_stats(a):
    rows = kernel_stats(a.csv)
    lines = [f"# rocprofv3 kernel statistics: {a.title}", "", "Command:", "", f"    {a.cmd}", "",
             f"Measured at commit {a.commit or git_commit()} (native source digest {source_digest()[:16]}).", "",
             "| kernel | calls | total ms | avg us | % |", "|---|---:|---:|---:|---:|"]
    for name, calls, tot, avg, pct in rows[: a.top]:
        lines.append(f"| `{name[:110]}` | {calls} | {tot / 1e6:.3f} | {avg / 1e3:.2f} | {pct:.1f} |")
    open(a.out, "w").write("\n".join(lines) + "\n")


def cmd_traffic(a):
    ff = copy_factor(a.copy_fetch, "FETCH_SIZE", a.copy_bytes)
    fw = copy_factor(a.copy_write, "WRITE_SIZE", a.copy_bytes)
    fetch = counters(a.fetch, "FETCH_SIZE")
    write = counters(a.write, "WRITE_SIZE")
    dur = durations(a.trace) if a.trace else {}
    sel = re.compile(a.kernels)
    per_kernel = {}
    tokens = 0
    gemv_bytes = 0.0
    for name, vals in fetch.items():
        if not sel.search(name):
            continue
        epi = _gemv_epilogue(name)
        if epi == 0:  # the prefill's plain GEMV rows are not part of a decode token
            continue
        if epi == 4:  # one norm + lm_head + argmax launch per decode token
            tokens = len(vals)
        w = write.get(name, [0.0])
        k = {
            "dispatches": len(vals),
            "fetch_bytes_avg": sum(vals) / len(vals) * 1024.0 * ff,
            "write_bytes_avg": sum(w) / len(w) * 1024.0 * fw,
        }
        if name in dur:
            d = dur[name]
            k["trace_dispatches"] = len(d)
            k["duration_ns_avg"] = sum(d) / len(d)
            k["achieved_gbs"] = (k["fetch_bytes_avg"] + k["write_bytes_avg"]) / k["duration_ns_avg"]
        if epi is not None:
            gemv_bytes += k["dispatches"] * (k["fetch_bytes_avg"] + k["write_bytes_avg"])
        per_kernel[name] = k
    res = {
        "method": "rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE passes, each scaled by the same counter for a "
                  f"{a.copy_bytes}-byte device-to-device copy" +
                  ("; durations from a --kernel-trace run of the same command" if a.trace else ""),
        "source_digest": source_digest(),
        "commit": a.commit or git_commit(),
        "fetch_factor_bytes_per_kib": ff * 1024.0,
        "write_factor_bytes_per_kib": fw * 1024.0,
        "gemv_launches": sum(k["dispatches"] for n, k in per_kernel.items() if _gemv_epilogue(n) is not None),
        "tokens": tokens,
        "hbm_bytes_per_token": gemv_bytes / tokens if tokens else None,
        "algorithmic_bytes_per_token": a.algorithmic,
        "per_kernel": per_kernel,
        "command": a.cmd,
    }
    json.dump(res, open(a.out_json, "w"), indent=1)
    lines = [f"# HBM traffic per kernel ({a.title})", "", "Commands:", "", f"    {a.cmd}", "",
             f"Measured at commit {res['commit']} (native source digest {res['source_digest'][:16]}).", "",
             f"Copy calibration: FETCH_SIZE {ff * 1024:.1f} B/KiB-counted, WRITE_SIZE {fw * 1024:.1f} B/KiB-counted "
             f"({a.copy_bytes} B device-to-device copy).", ""]
    if tokens:
        lines += [f"GEMV launches in {tokens} tokens: {res['gemv_launches']}; measured HBM bytes per token "
                  f"{res['hbm_bytes_per_token'] / 1e9:.4f} GB vs algorithmic {a.algorithmic / 1e9:.4f} GB.", ""]
    lines += ["| kernel | dispatches | fetch MB avg | write KB avg | avg us (trace) | measured GB/s |",
              "|---|---:|---:|---:|---:|---:|"]
    for name, k in sorted(per_kernel.items(), key=lambda kv: -kv[1]["dispatches"] * kv[1]["fetch_bytes_avg"]):
        us = f"{k['duration_ns_avg'] / 1e3:.2f}" if "duration_ns_avg" in k else "-"
        gbs = f"{k['achieved_gbs']:.0f}" if "achieved_gbs" in k else "-"
        lines.append(f"| `{name[:100]}` | {k['dispatches']} | {k['fetch_bytes_avg'] / 1e6:.3f} | "
                     f"{k['write_bytes_avg'] / 1e3:.2f} | {us} | {gbs} |")
    if a.note:
        lines += ["", a.note]
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
    s.add_argument("--commit", default=None)
    t = sp.add_parser("traffic")
    for k in ("fetch", "write", "copy_fetch", "copy_write"):
        t.add_argument("--" + k.replace("_", "-"), dest=k, required=True)
    t.add_argument("--copy-bytes", type=int, required=True)
    t.add_argument("--algorithmic", type=int, default=0)
    t.add_argument("--trace", default=None)
    t.add_argument("--kernels", default=DEFAULT_KERNELS)
    t.add_argument("--commit", default=None)
    t.add_argument("--note", default="")
    t.add_argument("--out-md", required=True)
    t.add_argument("--out-json", required=True)
    t.add_argument("--cmd", required=True)
    t.add_argument("--title", default="INT4 8B-shape decode")
    mf = sp.add_parser("mfma")
    mf.add_argument("--pmc", required=True)
    mf.add_argument("--trace", required=True)
    mf.add_argument("--kernels", default=r"^gemm")
    mf.add_argument("--shape", action="append", default=[])
    mf.add_argument("--out", required=True)
    mf.add_argument("--cmd", action="append", required=True)
    mf.add_argument("--commit", default=None)
    mf.add_argument("--note", default="")
    mf.add_argument("--title", default="INT4 8B-shape, 512-token prompt")
    sp.add_parser("digest")
    a = ap.parse_args()
    if a.cmd_name == "stats":
        cmd_stats(a)
    elif a.cmd_name == "mfma":
        cmd_mfma(a)
    elif a.cmd_name == "digest":
        print(source_digest())
    else:
        cmd_traffic(a)


if __name__ == "__main__":
    main()
