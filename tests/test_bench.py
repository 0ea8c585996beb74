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


def test_cpu_baselines_of_the_secondary_legs():
    # the prefill and pack legs carry their own CPU oracle timings; small
    # samples here, the shapes and fields of the JSON objects are the contract
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "hetero-serve_amd"))
    from hsbench.cases import build_prefill

    pk = bench.cpu_pack_baseline(n=8, pool_blocks=16)
    assert pk["unit"] == "GB/s" and pk["value"] > 0 and pk["cores"] == 1
    assert pk["kind"] == "port" and "export_blocks" in pk["sample"]
    case = build_prefill("t", np.array([30, 0]), np.array([17, 40]), 4, 4, 32, 16,
                         torch.float32, "cpu", seed=3)
    pf = bench.cpu_prefill_baseline(case, heads=2)
    assert pf["unit"] == "TFLOP/s" and pf["value"] > 0 and pf["kind"] == "port"
    assert "2 of 4 heads" in pf["sample"]
