"""The rocprofv3 summary tool behind profiles/ and the bench line's traffic figures:
copy-scaled byte counts, per-kernel durations, MFMA utilisation split by shape, and
the source digest that tells bench.py whether a committed summary still describes
the code being run."""

import csv
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from aethermind_amd import profiling as P  # noqa: E402

GEMV = "void am::(anonymous namespace)::gemv_kernel<am::ActBF16, 3, true, 3, 2, 1, 8, false>(GemvArgs)"
HEAD = "void am::(anonymous namespace)::gemv_kernel<am::ActBF16, 3, true, 4, 2, 2, 12, false>(GemvArgs)"
PLAIN = "void am::(anonymous namespace)::gemv_kernel<am::ActBF16, 3, false, 0, 2, 1, 8, false>(GemvArgs)"
ATT = "void am::(anonymous namespace)::attention_decode_kernel<128, 4>(AttnArgs)"
COPY = "__amd_rocclr_copyBuffer"


def _counters(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writerows(rows)


def _trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp", "End_Timestamp"])
        w.writerows(rows)


def test_source_digest_tracks_every_source_file(tmp_path):
    (tmp_path / "kernels").mkdir()
    (tmp_path / "kernels" / "a.hip").write_text("x")
    (tmp_path / "host.cpp").write_text("y")
    (tmp_path / "notes.txt").write_text("ignored")
    d0 = P.source_digest(str(tmp_path))
    (tmp_path / "notes.txt").write_text("changed")
    assert P.source_digest(str(tmp_path)) == d0
    (tmp_path / "kernels" / "a.hip").write_text("x2")
    d1 = P.source_digest(str(tmp_path))
    assert d1 != d0
    (tmp_path / "kernels" / "a.hip").rename(tmp_path / "kernels" / "b.hip")  # same bytes, other name
    assert P.source_digest(str(tmp_path)) not in (d0, d1)
    assert len(P.source_digest()) == 64


def test_traffic_scales_by_the_copy_and_counts_tokens(tmp_path):
    copy_bytes = 1 << 20
    # the copy reads 512 "KiB" units and writes 1024 for 1 MiB: factors 2048 B and 1024 B per unit
    _counters(tmp_path / "cf.csv", [[COPY, 1, "FETCH_SIZE", 512.0]])
    _counters(tmp_path / "cw.csv", [[COPY, 1, "WRITE_SIZE", 1024.0]])
    _counters(tmp_path / "f.csv", [[GEMV, 1, "FETCH_SIZE", 100.0], [GEMV, 1, "FETCH_SIZE", 300.0],
                                   [HEAD, 1, "FETCH_SIZE", 50.0], [PLAIN, 1, "FETCH_SIZE", 9999.0],
                                   [ATT, 1, "FETCH_SIZE", 10.0]])
    _counters(tmp_path / "w.csv", [[GEMV, 1, "WRITE_SIZE", 2.0], [GEMV, 1, "WRITE_SIZE", 4.0],
                                   [HEAD, 1, "WRITE_SIZE", 1.0], [ATT, 1, "WRITE_SIZE", 3.0]])
    _trace(tmp_path / "t.csv", [[ATT, 256, 8, 1, 1000, 6000], [ATT, 256, 8, 1, 2000, 5000]])
    out_json, out_md = tmp_path / "s.json", tmp_path / "s.md"
    subprocess.run([sys.executable, "-m", "aethermind_amd.profiling", "traffic", "--fetch", str(tmp_path / "f.csv"),
                    "--write", str(tmp_path / "w.csv"), "--copy-fetch", str(tmp_path / "cf.csv"), "--copy-write",
                    str(tmp_path / "cw.csv"), "--copy-bytes", str(copy_bytes), "--algorithmic", "123",
                    "--trace", str(tmp_path / "t.csv"), "--out-md", str(out_md), "--out-json", str(out_json),
                    "--cmd", "test", "--commit", "abc"], cwd=ROOT, check=True)
    d = json.loads(out_json.read_text())
    k = d["per_kernel"]
    assert d["commit"] == "abc" and d["source_digest"] == P.source_digest()
    assert d["fetch_factor_bytes_per_kib"] == pytest.approx(2048.0)
    assert d["write_factor_bytes_per_kib"] == pytest.approx(1024.0)
    g = k["gemv_kernel<ActBF16, 3, true, 3, 2, 1, 8, false>"]
    assert g["fetch_bytes_avg"] == pytest.approx(200.0 * 2048) and g["write_bytes_avg"] == pytest.approx(3.0 * 1024)
    assert "gemv_kernel<ActBF16, 3, false, 0, 2, 1, 8, false>" not in k  # prefill rows are not decode traffic
    assert d["tokens"] == 1  # one lm_head launch per token
    per_token = 2 * (200.0 * 2048 + 3.0 * 1024) + (50.0 * 2048 + 1024)
    assert d["hbm_bytes_per_token"] == pytest.approx(per_token)  # attention is not a GEMV
    a = k["attention_decode_kernel<128, 4>"]
    assert a["duration_ns_avg"] == pytest.approx(4000.0)
    assert a["achieved_gbs"] == pytest.approx((10.0 * 2048 + 3.0 * 1024) / 4000.0)
    assert "commit abc" in out_md.read_text()


def test_mfma_splits_one_kernel_by_shape(tmp_path):
    k = "void am::(anonymous namespace)::gemm_i4_kernel<1, 2>(I4Args)"
    _counters(tmp_path / "p.csv", [[k, 512, "SQ_VALU_MFMA_BUSY_CYCLES", 100.0], [k, 512, "SQ_VALU_MFMA_BUSY_CYCLES",
                                                                                 350.0],
                                   [k, 512, "SQ_BUSY_CYCLES", 7.0]])
    _trace(tmp_path / "t.csv", [[k, 512, 1, 1, 0, 10000], [k, 512, 1, 1, 0, 40000]])
    out = tmp_path / "m.md"
    subprocess.run([sys.executable, "-m", "aethermind_amd.profiling", "mfma", "--pmc", str(tmp_path / "p.csv"),
                    "--trace", str(tmp_path / "t.csv"), "--out", str(out), "--cmd", "test", "--commit", "abc",
                    "--shape", "gemm_i4_kernel<1, 2>@512@100=small:16x16x32",
                    "--shape", "gemm_i4_kernel<1, 2>@512@350=big:16x16x128"], cwd=ROOT, check=True)
    rows = [r for r in out.read_text().splitlines() if r.startswith("| `gemm_i4")]
    assert len(rows) == 2
    big, small = rows  # sorted by busy cycles
    assert "| big |" in big and "| 40.0 |" in big
    assert "| small |" in small and "| 10.0 |" in small
