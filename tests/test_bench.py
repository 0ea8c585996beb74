"""bench.py contract checks that need no GPU."""

import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_traffic_row_of_headline_kernel_is_found():
    # roofline.traffic comes from the committed rocprofv3 summary; the row
    # must exist for the kernel the headline leg runs, and the measured HBM
    # bytes must be close to the algorithmic K+V bytes of C2 (2.4617 GB)
    traffic = bench.profiled_traffic(bench.DECODE_KERNEL, bench.DECODE_WORKGROUPS)
    assert traffic is not None
    assert abs(traffic / 2_461_696_000 - 1.0) < 0.02


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr + r.stdout
