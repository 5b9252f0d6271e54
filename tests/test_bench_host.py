"""Host-side logic of bench.py (no GPU): the committed rocprofv3 summaries it reads `roofline.traffic`
from, and the single-GPU guard."""
import os
import subprocess
import sys

import bench

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_traffic_summaries_parse():
    """Each line that carries a `traffic` figure reads it from a committed summary, and the figure is
    at least the kernel's compulsory bytes (a counter that under-reads would show below them)."""
    decode = bench.read_traffic(bench.PROFILE_SUMMARY)
    assert decode is not None and decode >= bench.algo_bytes(5, 34816, 5120)
    assert decode <= 1.05 * bench.algo_bytes(5, 34816, 5120)  # one pass over the weights
    M, N, K = 2048, 34816, 5120
    w8a8 = bench.read_traffic(bench.W8A8_PROFILE)
    assert w8a8 is not None and w8a8 >= N * K + 4 * N + M * K + 4 * M + 2 * M * N
    assert bench.read_traffic(bench.ATTN_PROFILE) is not None


def test_read_traffic_missing_file(tmp_path):
    assert bench.read_traffic(str(tmp_path / "absent.txt")) is None
    p = tmp_path / "partial.txt"
    p.write_text("fetch_bytes_per_launch: 100\n")
    assert bench.read_traffic(str(p)) is None  # both counters are needed
    p.write_text("fetch_bytes_per_launch: 100\nwrite_bytes_per_launch: 28\n")
    assert bench.read_traffic(str(p)) == 128.0


def test_more_than_one_gpu_is_refused():
    """This build measures one GPU: --gpus above 1 exits with a message before touching a device."""
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--steps", "1",
                        "--warmup", "0"], capture_output=True, text=True, timeout=120, cwd=ROOT)
    assert r.returncode != 0
    assert "one GPU" in (r.stderr + r.stdout)
    assert r.stdout.strip() == ""  # no JSON line
