"""bench.py's host logic on the CPU: the rocprofv3 summarizer (kernel statistics split by GEMM launch
segment, copy-calibrated traffic per launch, the traffic file bench.py reads back) and the refusal of
more than one GPU."""
import csv
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402

GEMM_A = "void h3mi::(anonymous namespace)::w8a8_gemm_direct_kernel<h3mi::DTile<256, 384, 128>, false>(int)"
GEMM_B = "void h3mi::(anonymous namespace)::w8a8_gemm_direct_kernel<h3mi::DTile<256, 256, 128>, false>(int)"
COPY = "__amd_rocclr_copyBuffer"
NORM = "void h3mi::(anonymous namespace)::norm_stream_kernel<256, 64, 10, false, 0>(int)"


def _trace(d, rows):
    """rows: (kernel, grid, start_ns, duration_ns) -> a rocprofv3 kernel_trace.csv under d."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_kernel_trace.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp", "End_Timestamp"])
        for name, grid, start, dur in rows:
            w.writerow([name, grid, 1, 1, start, start + dur])


def _counters(d, rows):
    """rows: (dispatch id, kernel, grid, counter, value) -> a counter_collection.csv under d."""
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "run_counter_collection.csv"), "w", newline="") as f:
        w = csv.writer(f)
        w.writerow(["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"])
        for r in rows:
            w.writerow(r)


def test_summarize_splits_gemm_rows_by_launch_segment(tmp_path, capsys):
    # a resident grid has one size for every shape: A, then B, then A again are three segments
    seq = [(GEMM_A, 131072, 2000)] * 3 + [(NORM, 65536, 100)] + [(GEMM_B, 131072, 250)] * 2 + \
          [(GEMM_A, 131072, 1800)] * 2
    rows, t = [], 0
    for name, grid, us in seq:
        rows.append((name, grid, t, us * 1000))
        t += us * 1000 + 500
    _trace(str(tmp_path / "s"), rows)
    bench.summarize([str(tmp_path / "s")], None)
    out = capsys.readouterr().out
    lines = [ln for ln in out.splitlines() if "w8a8_gemm" in ln]
    seg = {ln.split("(segment ")[1].split(")")[0]: ln for ln in lines}
    assert set(seg) == {"1", "2", "3"}
    assert "| 3 | 2000.0 |" in seg["1"] and "| 2 | 250.0 |" in seg["2"] and "| 2 | 1800.0 |" in seg["3"]
    assert any("norm_stream_kernel" in ln and "segment" not in ln for ln in out.splitlines())


def test_summarize_calibrates_traffic_and_writes_the_file(tmp_path, capsys):
    # the device copy of COPY_BYTES reads half its bytes by FETCH_SIZE (KiB) and all of them by WRITE_SIZE
    cb = bench.COPY_BYTES
    f_rows, w_rows = [], []
    for i, (name, grid, fetch, write) in enumerate([
            (COPY, 65536, cb / 2 / 1024, cb / 1024),
            (GEMM_A, 131072, 1.5e9 / 1024, 1.0e9 / 1024),   # the full workload
            (GEMM_B, 131072, 0.25e9 / 1024, 0.125e9 / 1024),  # the shard
            (GEMM_A, 131072, 1.5e9 / 1024, 1.0e9 / 1024)]):
        f_rows.append((i, name, grid, "FETCH_SIZE", fetch))
        w_rows.append((i, name, grid, "WRITE_SIZE", write))
    _counters(str(tmp_path / "f"), f_rows)
    _counters(str(tmp_path / "w"), w_rows)
    tfile = str(tmp_path / "traffic.txt")
    bench.summarize([str(tmp_path / "f"), str(tmp_path / "w")], tfile)
    out = capsys.readouterr().out
    assert "scale factor 2.0000" in out and "scale factor 1.0000" in out
    got = dict(ln.split() for ln in open(tfile) if not ln.startswith("#"))
    # fetch 1.5e9 x 2 + write 1.0e9: the group that moves the most bytes per launch (segments 1 and 3 are both A)
    assert abs(float(got["w8a8_gemm"]) - 4.0e9) < 1e3


@pytest.mark.parametrize("kernel,tag", [
    ("void h3mi::(anonymous namespace)::gate_norm_split_kernel<5, 0>(unsigned short*, int)", "gate_norm_mod_"),
    ("void h3mi::(anonymous namespace)::norm_stream_kernel<256, 64, 10, true, 0>(int)", "gate_norm_mod_"),
    ("void h3mi::(anonymous namespace)::gate_norm_split_kernel<5, 1>(unsigned short*, int)", "gate_norm_mod_h3")])
def test_both_gate_norm_mod_kernels_count_as_gate_norm_mod(tmp_path, capsys, kernel, tag):
    """Every kernel that serves gate_norm_mod_ at the bench's shapes (the one-row-per-workgroup kernel at
    N = 1024 IT and at 1024 IT + 256, the row stream) counts under its traffic tag."""
    cb = bench.COPY_BYTES
    f_rows, w_rows = [], []
    for i, (name, grid, fetch, write) in enumerate([(COPY, 65536, cb / 2 / 1024, cb / 1024),
                                                     (kernel, 65536, 0.3e9 / 1024, 0.6e9 / 1024)]):
        f_rows.append((i, name, grid, "FETCH_SIZE", fetch))
        w_rows.append((i, name, grid, "WRITE_SIZE", write))
    _counters(str(tmp_path / "f"), f_rows)
    _counters(str(tmp_path / "w"), w_rows)
    tfile = str(tmp_path / "traffic.txt")
    bench.summarize([str(tmp_path / "f"), str(tmp_path / "w")], tfile)
    capsys.readouterr()
    got = dict(ln.split() for ln in open(tfile) if not ln.startswith("#"))
    assert abs(float(got[tag]) - 1.2e9) < 1e3


def test_read_traffic_returns_the_committed_gemm_bytes():
    v = bench.read_traffic("w8a8_gemm")
    assert v is None or v > 1e9


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr


@pytest.mark.parametrize("name", ["qkv", "up", "down", "c0"])
def test_workloads_are_the_configured_shapes(name):
    M, N, K, _, kind, _, _ = bench.WORKLOADS[name]
    assert K % 128 == 0 and N % 4 == 0
    assert (M, N, K) in {(32768, 15360, 5120), (32768, 13824, 5120), (32768, 5120, 13824), (2048, 3072, 3072)}
    assert kind in ("randn", "gelu")
