"""bench.py --traffic: calibrated HBM bytes from rocprofv3 counter files (CPU).

The counter runs behind the profiles' traffic tables read FETCH_SIZE and
WRITE_SIZE in KiB per dispatch; bench.py scales each by what the counter reads
for the 1 GiB copy probe and compares the kernel's bytes with its algorithmic
bytes. These tests feed it synthetic counter files with known values, so a
swapped scale, a dropped factor of 1024 or a kernel matched by the wrong name
changes the numbers checked here.
"""

from __future__ import annotations

import csv
import json
import pathlib
import subprocess
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SLAB = 4096 * 2048 * 2  # B*T*D*2 bytes at T=4096, D=2048, bf16
PROBE = "sy::(anonymous namespace)::k_probe_copy(char const*, char*, long)"
COLUMNS = ["Correlation_Id", "Dispatch_Id", "Kernel_Name", "Counter_Name", "Counter_Value"]


def _write(d: pathlib.Path, counter: str, rows: list[tuple[str, float]]) -> None:
    d.mkdir(parents=True)
    with open(d / "1_counter_collection.csv", "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_ALL)
        w.writerow(COLUMNS)
        for i, (name, value) in enumerate(rows):
            w.writerow([i + 1, i + 1, name, counter, value])


def _run(tmp_path, fetch_rows, write_rows, traffic_set):
    fdir, wdir = tmp_path / "fetch", tmp_path / "write"
    _write(fdir, "FETCH_SIZE", fetch_rows)
    _write(wdir, "WRITE_SIZE", write_rows)
    out = tmp_path / "traffic.json"
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--traffic", str(fdir), str(wdir),
                        "--traffic-set", traffic_set, "--json-out", str(out)],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    return json.loads(out.read_text())


def test_calibration_scales_each_counter_by_the_copy_probe(tmp_path):
    # The probe moves 1 GiB each way; its counters read half of that (fetch)
    # and all of it (write), as FETCH_SIZE and WRITE_SIZE do on MI355X.
    gib_kib = float(1 << 20)
    fwd, bwd, sol = "void sy::k_fwd_res<sy::BF16, 1, 4, 9>(x)", "void sy::k_bwd<sy::BF16, 1, 4, 9, true, 0>(x)", \
        "void sy::k_sol_res<sy::BF16, 1, 4, 9>(x)"
    fetch = [(PROBE, gib_kib / 2), (PROBE, gib_kib / 2), (fwd, 1000.0), (fwd, 3000.0), (bwd, 5000.0), (sol, 7000.0)]
    write = [(PROBE, gib_kib), (fwd, 100.0), (bwd, 200.0), (sol, 300.0)]
    rec = _run(tmp_path, fetch, write, "config2")
    assert rec["fetch_scale"] == pytest.approx(2.0)
    assert rec["write_scale"] == pytest.approx(1.0)
    # dispatches of one kernel are averaged; KiB -> bytes
    assert rec["fwd_bytes_per_launch"] == round((2000.0 * 2 + 100.0) * 1024)
    assert rec["bwd_main_bytes_per_launch"] == round((5000.0 * 2 + 200.0) * 1024)
    assert rec["sol_bytes_per_launch"] == round((7000.0 * 2 + 300.0) * 1024)
    # algorithmic bytes at config 2: (N+1) slabs forward, (2N+1) backward
    assert rec["fwd_algorithmic_bytes"] == 10 * SLAB
    assert rec["bwd_main_algorithmic_bytes"] == 19 * SLAB
    assert rec["fwd_traffic_over_algorithmic"] == pytest.approx(rec["fwd_bytes_per_launch"] / (10 * SLAB))


@pytest.mark.parametrize("traffic_set,n,fwd_name,fwd_key,bwd_name", [
    ("n4", 4, "void sy::k_fwd_res<sy::BF16, 1, 4, 4>(x)", "fwd", "void sy::k_bwd<sy::BF16, 1, 4, 4, true, 0>(x)"),
    ("n16", 16, "void sy::k_fwd<sy::BF16, 1, 4, 4>(x)", "fwd_chunked", "void sy::k_bwd<sy::BF16, 1, 4, 16, true, 0>(x)"),
])
def test_n_sweep_sets_match_their_kernels(tmp_path, traffic_set, n, fwd_name, fwd_key, bwd_name):
    gib_kib = float(1 << 20)
    reduce = "sy::(anonymous namespace)::k_dw_reduce4(float const*, int, int, void*, int)"
    fetch = [(PROBE, gib_kib / 2), (fwd_name, 10.0), (bwd_name, 20.0), (reduce, 999.0)]
    write = [(PROBE, gib_kib), (fwd_name, 1.0), (bwd_name, 2.0), (reduce, 999.0)]
    rec = _run(tmp_path, fetch, write, traffic_set)
    assert rec["workload"] == f"N={n} B=1 T=4096 D=2048 bf16"
    assert rec[f"{fwd_key}_bytes_per_launch"] == round((10.0 * 2 + 1.0) * 1024)
    assert rec["bwd_main_bytes_per_launch"] == round((20.0 * 2 + 2.0) * 1024)
    assert rec[f"{fwd_key}_algorithmic_bytes"] == (n + 1) * SLAB
    assert rec["bwd_main_algorithmic_bytes"] == (2 * n + 1) * SLAB


def test_fp32_d8192_set_matches_the_eight_wave_tiles(tmp_path):
    """The d-sweep's fp32 counter run holds every D of the set: only the
    eight-wave kernels of D=8192 count, at fp32 slabs."""
    gib_kib = float(1 << 20)
    fwd8 = "void sy::k_fwd_res<sy::F32, 8, 4, 9, false, false>(x)"
    bwd8 = "void sy::k_bwd<sy::F32, 8, 4, 9, true, 0>(x)"
    other = [("void sy::k_fwd_res<sy::F32, 4, 4, 9, false, false>(x)", 999.0),
             ("void sy::k_bwd<sy::F32, 4, 4, 9, true, 0>(x)", 999.0)]
    fetch = [(PROBE, gib_kib / 2), (fwd8, 10.0), (bwd8, 20.0), *other]
    write = [(PROBE, gib_kib), (fwd8, 1.0), (bwd8, 2.0), *other]
    rec = _run(tmp_path, fetch, write, "d8192f32")
    slab = 4096 * 8192 * 4
    assert rec["workload"] == "N=9 B=1 T=4096 D=8192 fp32"
    assert rec["fwd_bytes_per_launch"] == round((10.0 * 2 + 1.0) * 1024)
    assert rec["bwd_main_bytes_per_launch"] == round((20.0 * 2 + 2.0) * 1024)
    assert rec["fwd_algorithmic_bytes"] == 10 * slab
    assert rec["bwd_main_algorithmic_bytes"] == 19 * slab


def test_a_missing_kernel_is_an_error(tmp_path):
    gib_kib = float(1 << 20)
    fetch = [(PROBE, gib_kib / 2)]
    write = [(PROBE, gib_kib)]
    fdir, wdir = tmp_path / "fetch", tmp_path / "write"
    _write(fdir, "FETCH_SIZE", fetch)
    _write(wdir, "WRITE_SIZE", write)
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--traffic", str(fdir), str(wdir)],
                       capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode != 0
    assert "no dispatch of" in (r.stdout + r.stderr)


def test_summarize_turns_kernel_stats_into_microseconds(tmp_path):
    d = tmp_path / "trace" / "host"
    d.mkdir(parents=True)
    with open(d / "7_kernel_stats.csv", "w", newline="") as fh:
        w = csv.writer(fh, quoting=csv.QUOTE_ALL)
        w.writerow(["Name", "Calls", "TotalDurationNs", "AverageNs", "Percentage", "MinNs", "MaxNs", "StdDev"])
        w.writerow(["void sy::k_bwd<sy::BF16, 1, 4, 9, true, 0>(x)", 490, 27781000, 56696.0, 60.0, 53350.0,
                    65870.0, 1.0])
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--summarize", str(tmp_path / "trace"),
                        "--title", "t"], capture_output=True, text=True, cwd=ROOT, timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "| `void sy::k_bwd<sy::BF16, 1, 4, 9, true, 0>(x)` | 490 | 56.70 | 53.35 | 65.87 |" in r.stdout
