"""bench.py's host-side logic, without a GPU: the HBM-traffic figure it
derives from two rocprofv3 counter runs, and its refusal of more than one
GPU."""
import csv
import io
import os
import subprocess
import sys
import types
from contextlib import redirect_stdout

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def _counter_csv(path, counter, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=["Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        w.writeheader()
        for name, grid, kib in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size": grid, "Counter_Name": counter, "Counter_Value": kib})


def test_traffic_scales_counters_by_the_calibration_copy(tmp_path):
    """Each counter is divided by what it reads for the 256 MiB copy; one
    group per GEMM shape in run order; the verify figure weights the shapes
    by their launches per target forward.  Planted values: the fetch counter
    reads the copy as 1/1.9 of its bytes (factor 1.9; MI355X reads about one
    half), the write counter as 1/1.25 (factor 1.25); a second, small copy is
    not a calibration; shape i fetches (i+1) MB and writes (i+1)/10 MB in
    scaled bytes."""
    cal = 256 << 20
    kinds = ["void vx_vg_kernel<2, 9, 2, 4, 4, 2, 1>(vx_gemm_args)",
             "void vx_gemm_kernel<2, 9, false, 8, 2>(vx_gemm_args)"]
    fetch_rows = [("__amd_rocclr_copyBuffer", 1, cal / 1.9 / 1024), ("__amd_rocclr_copyBuffer", 1, 100.0)]
    write_rows = [("__amd_rocclr_copyBuffer", 1, cal / 1.25 / 1024)]
    want = {}
    for i, (shape, r, c, bpb) in enumerate(bench.GEMM_SHAPES):
        name, grid = kinds[i % 2], 1000 + i
        f_b, w_b = (i + 1) * 1e6, (i + 1) * 1e5
        for _ in range(3):   # three launches per shape
            fetch_rows.append((name, grid, f_b / 1.9 / 1024))
            write_rows.append((name, grid, w_b / 1.25 / 1024))
        want[shape] = f_b + w_b
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    _counter_csv(fp, "FETCH_SIZE", fetch_rows)
    _counter_csv(wp, "WRITE_SIZE", write_rows)
    out = io.StringIO()
    with redirect_stdout(out):
        bench.run_traffic(types.SimpleNamespace(k=8, fetch=str(fp), write=str(wp)))
    text = out.getvalue()
    assert "factor 1.9000" in text and "factor 1.2500" in text
    n = sum(bench.VERIFY_MIX.values())
    expect = sum(want[s] * c for s, c in bench.VERIFY_MIX.items()) / n
    got = float(text.split("traffic_bytes_per_launch:")[1].split()[0])
    assert got == pytest.approx(expect, rel=1e-9, abs=1.0)
    # per-shape traffic/alg column: algorithmic bytes = weights + fp32 input and output rows
    for shape, r, c, bpb in bench.GEMM_SHAPES:
        alg = r * c // 32 * bpb + 4 * 9 * c + 4 * 9 * r
        line = next(l for l in text.splitlines() if l.startswith(shape))
        assert float(line.split()[-1]) == pytest.approx(want[shape] / alg, abs=6e-4)


def test_traffic_refuses_a_missing_shape(tmp_path):
    cal = 256 << 20
    rows = [("__amd_rocclr_copyBuffer", 1, cal / 1024),
            ("void vx_gemm_kernel<2, 9, false, 8, 2>(vx_gemm_args)", 7, 10.0)]
    fp, wp = tmp_path / "f.csv", tmp_path / "w.csv"
    _counter_csv(fp, "FETCH_SIZE", rows)
    _counter_csv(wp, "WRITE_SIZE", rows)
    with pytest.raises(SystemExit):
        with redirect_stdout(io.StringIO()):
            bench.run_traffic(types.SimpleNamespace(k=8, fetch=str(fp), write=str(wp)))


@pytest.mark.parametrize("argv,env", [(["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "4"})])
def test_more_than_one_gpu_is_refused(argv, env):
    e = dict(os.environ, **env)
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py")] + argv, capture_output=True, text=True,
                       env=e, timeout=120)
    assert r.returncode == 2
    assert "ONE GPU" in r.stderr
    assert r.stdout == ""
