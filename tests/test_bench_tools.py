"""CPU tests of bench.py's counter summaries on synthetic rocprofv3 databases
(the tables and columns the summaries read: kernels(name, duration) of a
--kernel-trace run, counters_collection(counter_name, kernel_name, value) of
a --pmc run)."""
import os
import sqlite3
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _db(path, kernels=None, counters=None):
    os.makedirs(os.path.dirname(path), exist_ok=True)
    c = sqlite3.connect(path)
    if kernels is not None:
        c.execute("create table kernels (name text, duration integer)")
        c.executemany("insert into kernels values (?, ?)", kernels)
    if counters is not None:
        c.execute("create table counters_collection (counter_name text, kernel_name text, value real)")
        c.executemany("insert into counters_collection values (?, ?, ?)", counters)
    c.commit()
    c.close()


def _bench(*args):
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    return r.stdout


def test_clock_summary(tmp_path):
    gu = "void (anonymous namespace)::moe_gu_m3_kernel<15>((anonymous namespace)::GroupedArgs)"
    # 500 us launches (durations in ns) and 8 XCDs x 1.75 GHz x 500 us busy clocks
    _db(str(tmp_path / "kt" / "a" / "kt_results.db"), kernels=[(gu, 500_000), (gu, 510_000), (gu, 490_000)])
    _db(str(tmp_path / "pmc" / "a" / "p_results.db"),
        counters=[("GRBM_GUI_ACTIVE", gu, 8 * 1.75e9 * 500e-6)] * 3 + [("SQ_WAVES", gu, 1.0)])
    out = _bench("--clock-summary", str(tmp_path / "kt"), str(tmp_path / "pmc"))
    row = [line for line in out.splitlines() if line.startswith("moe_gu_m3_kernel<15>")]
    assert len(row) == 1, out
    f = row[0].split()
    assert f[1] == "3" and abs(float(f[2]) - 500.0) < 1e-6 and abs(float(f[4]) - 1.75) < 1e-3, row


def test_pmc_summary_scales_by_the_copy(tmp_path):
    gu = "void (anonymous namespace)::moe_gu_m3_kernel<15>((anonymous namespace)::GroupedArgs)"
    neg = "void at::native::neg_kernel_cuda(at::TensorIteratorBase&)"
    # the copy reads 64 MiB and FETCH_SIZE reports half of it; WRITE_SIZE all
    copy_kib = 64 * 1024
    _db(str(tmp_path / "p" / "a" / "x_results.db"),
        counters=[("FETCH_SIZE", gu, 1000.0), ("WRITE_SIZE", gu, 300.0),
                  ("FETCH_SIZE", neg, copy_kib / 2), ("WRITE_SIZE", neg, copy_kib)])
    out = _bench("--pmc-summary", str(tmp_path / "p"))
    vals = {line.split(":")[0]: int(line.split(":")[1]) for line in out.splitlines() if "_bytes_per_launch:" in line}
    assert vals["fetch_bytes_per_launch"] == 2 * 1000 * 1024, out
    assert vals["write_bytes_per_launch"] == 300 * 1024, out
    assert vals["traffic_bytes_per_launch"] == 2 * 1000 * 1024 + 300 * 1024, out
