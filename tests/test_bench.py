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
    traffic = bench.leg_traffic("C2")
    assert traffic is not None
    assert abs(traffic / 2_461_696_000 - 1.0) < 0.02


def test_every_leg_has_a_traffic_row():
    # each leg's roofline reads its kernel's HBM bytes from the same summary;
    # the copy legs move exactly 2 GiB (1 GiB read + 1 GiB written)
    for leg in bench.LEG_KERNELS:
        assert bench.leg_traffic(leg) is not None, leg
    for leg in ("C5_pack", "C5_unpack"):
        assert abs(bench.leg_traffic(leg) / 2 ** 31 - 1.0) < 0.01


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stderr + r.stdout


def test_cpu_baselines_and_parity_helpers():
    # the CPU legs return their oracle outputs beside the timing; the parity
    # helpers compare a GPU output with them.  Small CPU cases here: the
    # shapes and fields of the JSON objects are the contract.
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "hetero-serve_amd"))
    from hsbench.cases import build_decode, build_prefill

    case = build_prefill("t", np.array([30, 0]), np.array([17, 40]), 4, 4, 32, 16,
                         torch.float32, "cpu", seed=3)
    pf, pouts = bench.cpu_prefill_baseline(case, heads=2)
    assert pf["unit"] == "TFLOP/s" and pf["value"] > 0 and pf["kind"] == "port"
    assert "2 of 4 heads" in pf["sample"] and "cpu=" in pf["sample"]
    assert sorted(pouts) == [0, 1] and pouts[1].shape == (40, 2, 32)
    got = torch.cat([pouts[0], pouts[1]])
    assert bench.max_err_prefill(case, got, pouts, heads=2) == 0.0
    got[20, 1, 5] += 1e-2
    assert abs(bench.max_err_prefill(case, got, pouts, heads=2) - 1e-2) < 1e-6

    dc = build_decode("d", np.array([5, 40, 17]), 4, 2, 32, 16, torch.float32, "cpu", seed=4)
    cpu, outs = bench.cpu_decode_baseline(dc)
    assert cpu["unit"] == "GB/s" and cpu["value"] > 0 and "all 3 d sequences" in cpu["sample"]
    whole, want = bench.cpu_decode_batched(dc)
    assert whole["unit"] == "GB/s" and want.shape == (3, 4, 32)
    assert bench.max_err_decode(want, outs) < 1e-5
    sub, sub_outs = bench.cpu_decode_baseline(dc, n_seq=2)
    assert len(sub_outs) == 2 and "a seeded sample of 2" in sub["sample"]


def test_roofline_fields():
    r = bench.roofline("hbm", "k", 8e9, 2.0)           # 8 GB in 2 ms
    assert r["achieved"] == 4000.0 and r["frac"] == 0.5 and r["unit"] == "GB/s"
    assert r["traffic"] is None and "traffic_source" not in r
    r = bench.roofline("mfma", "k", 2.5e12, 2.0, traffic=123)
    assert r["unit"] == "TFLOP/s" and r["frac"] == 0.5 and "traffic_source" in r
