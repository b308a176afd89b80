"""bench.py's host-side paths, which need no GPU: the refusal of more than
one GPU, and the two kernel-trace summaries that the committed profiles
are made with (rocprofv3 kernel-trace CSV in, JSON out)."""
import csv
import json
import subprocess
import sys

import pytest

import bench

FIELDS = ["Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_X", "Workgroup_Size_X"]


def write_trace(path, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for name, start, end in rows:
            w.writerow({"Kernel_Name": name, "Start_Timestamp": start, "End_Timestamp": end,
                        "Grid_Size_X": 524288, "Workgroup_Size_X": 1024})


@pytest.mark.parametrize("args", [["--gpus", "2"], ["--gpus", "8", "--model", "llama3-8b"]])
def test_more_than_one_gpu_is_refused(args):
    result = subprocess.run([sys.executable, "bench.py", *args], capture_output=True, text=True, timeout=300,
                            cwd=bench.Path(bench.__file__).resolve().parent)
    assert result.returncode == 2
    assert "one GPU" in result.stderr


def test_trace_summary_takes_the_last_dispatches(tmp_path, capsys):
    kernel = "void (anonymous namespace)::nz_decode_kernel<2, true, false, false, 16>(...)"
    rows = [(kernel, 1000 * i, 1000 * i + 500) for i in range(5)]          # earlier launches: 0.5 us
    rows += [(kernel, 10_000 + 1000 * i, 10_000 + 1000 * i + 200 + i) for i in range(20)]   # timed: 0.2-0.219 us
    rows += [("void (anonymous namespace)::nz_decode_kernel<2, true, false, false, 8>(...)", 50_000, 60_000),
             ("Cijk_something", 70_000, 71_000)]
    write_trace(tmp_path / "t.csv", rows)
    assert bench.trace_summary(str(tmp_path / "t.csv"), steps=20) == 0
    out = json.loads(capsys.readouterr().out)
    assert out["dispatches"] == 25 and out["timed_dispatches"] == 20
    assert out["timed_mean_us"] == pytest.approx(sum(0.2 + i / 1000 for i in range(20)) / 20, abs=1e-3)
    assert out["timed_grid"] == [524288] and out["timed_workgroup"] == [1024]
    assert out["span_of_timed_us"] == pytest.approx((19_000 + 219) / 1000, abs=0.05)   # rounded to 0.1 us
    with pytest.raises(SystemExit, match="fewer than 30"):
        bench.trace_summary(str(tmp_path / "t.csv"), steps=30)


def test_trace_windows_splits_replay_loops_by_kind(tmp_path, capsys):
    spin = "at::cuda::spin_kernel(long)"
    us = 1000   # timestamps are in ns; the summary rounds to whole microseconds
    rows = [(spin, 0, 100 * us)]
    # two replays of a step: a GEMM, a decode overlapping it, another kernel, and a gap
    for base in (1000 * us, 3000 * us):
        rows += [("Cijk_Alik_x", base, base + 400 * us),
                 ("nz_decode_kernel<2, true, false, false, 8>", base + 200 * us, base + 900 * us),
                 ("elementwise", base + 1000 * us, base + 1100 * us)]
    rows += [(spin, 5000 * us, 5100 * us)]
    rows += [(spin, 6000 * us, 6100 * us), ("nz_matvec_kernel<2, true, false, 1>", 6200 * us, 6300 * us),
             (spin, 6400 * us, 6500 * us)]
    write_trace(tmp_path / "w.csv", rows)
    assert bench.trace_windows(str(tmp_path / "w.csv"), steps=2) == 0
    first, second = json.loads(capsys.readouterr().out)
    # window 100 .. 5000 us over 2 steps; busy per step = 900 (GEMM and decode overlap) + 100
    assert first["window_ms"] == pytest.approx(4.9 / 2)
    assert first["busy_ms"] == pytest.approx(1.0) and first["gaps_ms"] == pytest.approx(2.45 - 1.0)
    assert first["gemm_ms"] == pytest.approx(0.4)
    assert first["decode_ms"] == pytest.approx(0.7)
    assert first["other_ms"] == pytest.approx(0.1)
    assert first["kernels_per_step"] == 3
    assert second["matvec_ms"] == pytest.approx(0.05) and second["gemm_ms"] == 0
