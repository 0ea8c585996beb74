#!/usr/bin/env python3
"""Benchmark of hetero-serve's paged-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps 50] [--warmup 5] [--no-secondary] [--no-cpu]

One step is one call of the decode attention (hs_decode: the partition
kernel plus the log-sum-exp merge) over one layer of the whole batch, with
every input already resident in HBM.  The headline workload is configuration
C2 (ragged decode, batch 64, 32 heads, head_dim 128, bf16 KV, block_size 16,
context lognormal(median 2048, sigma 0.8) clipped to [64, 8192]); `value` is
its algorithmic HBM throughput in GB/s (K and V of every context token read
once, divided by the step time).

Every leg is checked before its number counts, as the reference's benchmark
does before timing (scripts/bench_kernel.py:193-201 for decode, :285-292 for
prefill): attention outputs against the CPU oracle computed on the same inputs
(max abs error <= 2e-3, the north-star bar; the reference gates at 2e-2 and
3e-2), pack and unpack bit for bit.  The line carries each leg's error; when
any check fails, "parity" is "fail" and the process exits with status 1.

The JSON line also carries:

  roofline      the dominant kernel alone, timed with HIP events that the
                library records around that launch on its own stream, against
                MI355X's 8 TB/s HBM peak (or the 2.5 PFLOP/s dense fp16 MFMA
                peak for prefill)
  cpu_baseline  the CPU oracle (oracle/) on this host's cores, on the same
                inputs, with the CPU model and thread count
  secondary     C1 (small decode), C3 (long-context decode), batch 64 at a 4k
                context (the decode target's shape), C2 at Llama-3-8B's
                grouped-query geometry, C4 chunked prefill, the C5 migration
                pack and unpack of 4096 blocks with a plain-copy ceiling, the
                C5 KV write and the C5 mixed step

Only rank 0 of a one-GPU run exists: there is no multi-GPU path on this box.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "hetero-serve_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "decode µs/step + HBM GB/s (% peak); prefill TFLOP/s (% MFMA peak)"
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0
TOL = 2e-3                     # north-star max abs error for fp16/bf16 caches


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


# HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE,
# calibrated on a 1 GiB copy) in separate profiled runs of this script;
# summarised in the committed profile below, whose tables this reads.
TRAFFIC_PROFILE = ROOT / "profiles" / "bench_legs_trace_and_traffic.md"
# Each leg's dominant kernel as rocprofv3 names it, its grid in workgroups
# (None: the only grid that kernel ran with) and the profile's table that
# holds it.  C2, C3 and B64-4k run the multi-head even split, whose grid (16
# two-head workgroups x one range per resident workgroup) is the same for all
# three, so the run of every leg averages them in one row: each is profiled
# alone.
LEG_KERNELS = {
    "C2": ("hs::row_attn_even_kernel<hs::Bf16, 128>", None, "C2 alone"),
    "C3": ("hs::row_attn_even_kernel<hs::Bf16, 128>", None, "C3 alone"),
    "B64-4k": ("hs::row_attn_even_kernel<hs::Bf16, 128>", None, "B64-4k alone"),
    "C1": ("hs::row_attn_wg_kernel<_Float16, 64, true, 1, 16>", None, "every leg"),
    "C2-gqa": ("hs::splitmm_even_kernel<hs::Bf16Ops, 128, true, 4>", None, "every leg"),
    "C4": ("hs::prefill_stream_kernel<hs::Bf16, 128>", None, "every leg"),
    "C5_pack": ("hs::page_copy_kernel<false, true>", None, "every leg"),
    "C5_unpack": ("hs::page_copy_kernel<true, true>", None, "every leg"),
}


def profiled_traffic(kernel: str, workgroups, table: str = "every leg"):
    """HBM read + write bytes of one launch of `kernel` (with `workgroups`
    workgroups, when given) from the committed PMC summary's table `table`."""
    names = (kernel,) if workgroups is None else (kernel, f"{kernel} [{workgroups} workgroups]")
    try:
        text = TRAFFIC_PROFILE.read_text()
        text = text[text.index(f"# HBM traffic per launch: {table}"):]
        end = text.find("\n# ", 1)
        for line in (text if end < 0 else text[:end]).splitlines():
            cells = [c.strip(" `") for c in line.split("|")]
            if len(cells) == 7 and cells[1] in names and "." in cells[4]:
                return int(round((float(cells[4]) + float(cells[5])) * 1e9))
    except (OSError, ValueError):
        pass
    return None


def leg_traffic(leg: str):
    kernel, wg, table = LEG_KERNELS[leg]
    return profiled_traffic(kernel, wg, table)


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform

    return platform.processor() or platform.machine()


def host_threads() -> int:
    return int(os.environ.get("OMP_NUM_THREADS") or os.cpu_count() or 1)


def roofline(kind: str, kernel: str, amount: float, kernel_ms: float, traffic=None) -> dict:
    """achieved = algorithmic bytes (or FLOPs) of one launch / its mean time."""
    if kind == "hbm":
        achieved = amount / (kernel_ms * 1e-3) / 1e9
        peak, unit = HBM_PEAK_GBS, "GB/s"
    else:
        achieved = amount / (kernel_ms * 1e-3) / 1e12
        peak, unit = MFMA_F16_PEAK_TFLOPS, "TFLOP/s"
    out = {"bound": kind, "kernel": kernel, "achieved": round(achieved, 2), "peak": peak,
           "unit": unit, "frac": round(achieved / peak, 4), "traffic": traffic,
           "algorithmic": int(amount), "kernel_us": round(kernel_ms * 1e3, 2)}
    if traffic is not None:
        out["traffic_source"] = (f"profiles/{TRAFFIC_PROFILE.name}: rocprofv3 --pmc FETCH_SIZE + "
                                 "WRITE_SIZE of this kernel's launch in profiled runs of bench.py")
    return out


def median_time(fn, runs: int = 3) -> float:
    """Median seconds of `runs` calls after one warm-up call."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


# ---------------------------------------------------------------------------
# GPU legs
# ---------------------------------------------------------------------------


def decode_leg(case, steps: int, warmup: int, partition_tokens: int = 0,
               warm_ms: float = 0.0) -> dict:
    """Time hs_decode on `case`; returns step/kernel times, throughputs and the
    output of the last step."""
    import torch

    from heteroserve import _hip
    from hsbench.timing import time_steps

    lib = _hip.lib()
    B, H, D = case.q.shape
    kc, vc = case.k_cache, case.v_cache
    NB, BS, Hkv, _ = kc.shape
    MB = case.block_tables.shape[1]
    out = torch.empty((B, H, D), dtype=torch.float32, device=case.q.device)
    ws_bytes = lib.hs_decode_workspace_bytes(B, H, Hkv, D, BS, MB, 0, partition_tokens)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=case.q.device)
    stream = torch.cuda.current_stream().cuda_stream
    dt = _hip.dtype_code(kc.dtype)
    args = (case.q.data_ptr(), kc.data_ptr(), vc.data_ptr(), dt, NB,
            case.block_tables.data_ptr(), case.context_lens.data_ptr(), out.data_ptr(),
            B, H, Hkv, D, BS, MB, float(case.scale), 0, partition_tokens, ws.data_ptr(),
            ws_bytes, stream)

    def step():
        _hip.check(lib.hs_decode(*args))

    def arm(s, e):
        _hip.check(lib.hs_profile_next_launch(s.handle, e.handle))

    step_ms, kernel_ms, wall = time_steps(step, steps, warmup, stream, arm, warm_ms)
    nbytes = case.decode_bytes()
    k_ms = statistics.mean(kernel_ms)
    return dict(step_ms=step_ms, kernel_ms=k_ms, kernel_ms_min=min(kernel_ms), wall_s=wall,
                bytes=nbytes, step_gbs=nbytes / (step_ms * 1e-3) / 1e9,
                kernel_gbs=nbytes / (k_ms * 1e-3) / 1e9, out=out)


def prefill_leg(case, steps: int, warmup: int) -> dict:
    import torch

    from heteroserve import _hip
    from hsbench.timing import time_steps

    lib = _hip.lib()
    T, H, D = case.q.shape
    kc, vc = case.k_cache, case.v_cache
    NB, BS, Hkv, _ = kc.shape
    B, MB = case.block_tables.shape
    out = torch.empty((T, H, D), dtype=torch.float32, device=case.q.device)
    stream = torch.cuda.current_stream().cuda_stream
    max_rows = int(case.q_lens.max())
    ws, ws_bytes = _hip._prefill_workspace(lib, B, max_rows, H, D, True, True, case.q.device)
    args = (case.q.data_ptr(), case.cu_seqlens.data_ptr(), max_rows,
            kc.data_ptr(), vc.data_ptr(), _hip.dtype_code(kc.dtype), NB,
            case.block_tables.data_ptr(), case.context_lens.data_ptr(), out.data_ptr(),
            B, H, Hkv, D, BS, MB, float(case.scale), 1,
            ws.data_ptr() if ws is not None else None, ws_bytes, stream)

    def step():
        _hip.check(lib.hs_prefill_varlen(*args))

    def arm(s, e):
        _hip.check(lib.hs_profile_next_launch(s.handle, e.handle))

    step_ms, kernel_ms, wall = time_steps(step, steps, warmup, stream, arm)
    flops = case.prefill_flops()
    k_ms = statistics.mean(kernel_ms)
    return dict(step_ms=step_ms, kernel_ms=k_ms, flops=flops,
                step_tflops=flops / (step_ms * 1e-3) / 1e12,
                kernel_tflops=flops / (k_ms * 1e-3) / 1e12, out=out)


def _copy_timed(step, steps: int, warmup: int) -> tuple:
    """(mean step ms, mean kernel ms) of a libhsattn copy call."""
    import torch

    from heteroserve import _hip
    from hsbench.timing import time_steps

    lib = _hip.lib()
    stream = torch.cuda.current_stream().cuda_stream

    def arm(s, e):
        _hip.check(lib.hs_profile_next_launch(s.handle, e.handle))

    step_ms, kernel_ms, _ = time_steps(step, steps, warmup, stream, arm)
    return step_ms, statistics.mean(kernel_ms)


def migration_legs(steps: int, warmup: int, with_cpu: bool) -> dict:
    """C5's migration copies on one pool [1, 2, 65536, 16, 32, 128] bf16 (17.2 GB):
    the pack of 4096 random blocks (1 GiB payload, export_blocks_device,
    torch_blocks.py:137-148), its unpack into another pool at the same ids
    (write_blocks_device, :150-154), and two plain-copy ceilings of the same
    1 GiB (torch's contiguous copy_, and the pack kernel on 4096 consecutive
    blocks).  The pack is checked bit for bit against the CPU torch oracle
    (the reference's own expression on a host copy of the pool) and the
    unpack against torch's GPU indexing; the CPU forms are also timed."""
    import torch

    from heteroserve import _hip
    from hsbench import cases
    from hsbench.timing import Event

    lib = _hip.lib()
    nb = cases.C5_POOL_BLOCKS
    dev = "cuda:0"
    stream = torch.cuda.current_stream().cuda_stream
    pool = torch.empty((1, 2, nb, 16, 32, 128), dtype=torch.bfloat16, device=dev)
    cases._fill_pool(pool, torch.Generator(device=dev).manual_seed(41))
    id_list = cases.c5_pack_ids(nb)
    ids = torch.as_tensor(id_list, dtype=torch.int64, device=dev)
    n = ids.numel()
    out = torch.empty((n, 1, 2, 16, 32, 128), dtype=torch.bfloat16, device=dev)
    page = pool[0, 0, 0].numel() * pool.element_size()
    nbytes = 2 * out.numel() * out.element_size()      # read + write

    def pack():
        _hip.check(lib.hs_kv_pack(pool.data_ptr(), 1, nb, page, ids.data_ptr(), n,
                                  out.data_ptr(), stream))

    pk_step, pk_kernel = _copy_timed(pack, steps, warmup)
    res = {"pack": {"us_per_step": round(pk_step * 1e3, 2),
                    "gbs": round(nbytes / (pk_kernel * 1e-3) / 1e9, 1),
                    "bytes_moved": nbytes,
                    "roofline": roofline("hbm", "page_copy_kernel<false, true>", nbytes, pk_kernel,
                                         leg_traffic("C5_pack"))}}
    log(f"C5 pack: {pk_kernel * 1e3:.1f} us, {res['pack']['gbs']:.0f} GB/s")

    # unpack into a zeroed pool at the same ids
    dst = torch.zeros_like(pool)

    def unpack():
        _hip.check(lib.hs_kv_unpack(dst.data_ptr(), 1, nb, page, ids.data_ptr(), n,
                                    out.data_ptr(), stream))

    up_step, up_kernel = _copy_timed(unpack, steps, warmup)
    got = dst[:, :, ids].permute(2, 0, 1, 3, 4, 5)
    up_exact = bool(torch.equal(got.contiguous().view(torch.int16), out.view(torch.int16)))
    dst.index_fill_(2, ids, 0)
    up_exact = up_exact and not bool(dst.view(torch.int16).any())     # nothing else written
    del dst, got
    res["unpack"] = {"us_per_step": round(up_step * 1e3, 2),
                     "gbs": round(nbytes / (up_kernel * 1e-3) / 1e9, 1),
                     "bytes_moved": nbytes, "bit_exact": up_exact,
                     "check": "torch GPU indexing of the unpacked pool == payload; "
                              "every other block untouched",
                     "roofline": roofline("hbm", "page_copy_kernel<true, true>", nbytes, up_kernel,
                                          leg_traffic("C5_unpack"))}
    log(f"C5 unpack: {up_kernel * 1e3:.1f} us, {res['unpack']['gbs']:.0f} GB/s, exact={up_exact}")

    # plain-copy ceilings of the same 1 GiB (into their own buffer: `out`
    # keeps the payload for the checks below)
    seq = torch.arange(n, dtype=torch.int64, device=dev)
    seq_out = torch.empty_like(out)

    def pack_seq():
        _hip.check(lib.hs_kv_pack(pool.data_ptr(), 1, nb, page, seq.data_ptr(), n,
                                  seq_out.data_ptr(), stream))

    _, seq_kernel = _copy_timed(pack_seq, steps, warmup)
    src = pool[0, :, :n // 2].contiguous()               # 1 GiB, contiguous
    cdst = torch.empty_like(src)
    for _ in range(warmup):
        cdst.copy_(src)
    e0, e1 = Event(), Event()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        cdst.copy_(src)
    e1.record(stream)
    copy_ms = e0.elapsed_ms(e1) / steps
    cbytes = 2 * src.numel() * src.element_size()
    res["copy_ceiling"] = {
        "pack_consecutive_blocks_gbs": round(nbytes / (seq_kernel * 1e-3) / 1e9, 1),
        "torch_copy_gbs": round(cbytes / (copy_ms * 1e-3) / 1e9, 1),
        "bytes_moved": nbytes,
        "note": "the same 1 GiB read + written: the pack kernel on blocks 0..4095, and "
                "torch's contiguous copy_ (a step, not a kernel event)"}
    log(f"copy ceilings: pack of consecutive blocks {res['copy_ceiling']['pack_consecutive_blocks_gbs']}"
        f" GB/s, torch copy_ {res['copy_ceiling']['torch_copy_gbs']} GB/s")
    del src, cdst, seq_out

    if with_cpu:
        from oracle.kvpack import export_blocks_torch, write_blocks_torch

        torch.set_num_threads(host_threads())
        hpool = pool.cpu()
        del pool
        torch.cuda.empty_cache()
        payload = {}

        def cpu_pack():
            payload["x"] = export_blocks_torch(hpool, id_list)

        t_pack = median_time(cpu_pack)
        exact = bool(torch.equal(out.cpu().view(torch.int16), payload["x"].view(torch.int16)))
        res["pack"]["bit_exact"] = exact
        res["pack"]["check"] = "GPU payload == CPU torch oracle payload, bit for bit"
        res["pack"]["cpu_baseline"] = {
            "value": round(nbytes / t_pack / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"the whole C5 pack (4096 random blocks of a 65536-block host pool, "
                       f"1 GiB payload): oracle/kvpack.py export_blocks_torch, the reference's "
                       f"pool[:, :, idx].permute(2, 0, 1, 3, 4, 5).contiguous() in torch on "
                       f"{torch.get_num_threads()} threads, median of 3 after 1 warm-up: "
                       f"{t_pack * 1e3:.1f} ms; cpu={cpu_model()}")}
        x = payload["x"]
        t_unpack = median_time(lambda: write_blocks_torch(hpool, id_list, x))
        res["unpack"]["cpu_baseline"] = {
            "value": round(nbytes / t_unpack / 1e9, 3), "unit": "GB/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": (f"the whole C5 unpack (4096 blocks of 256 KiB into the host pool): "
                       f"oracle/kvpack.py write_blocks_torch, the reference's per-block loop "
                       f"pool[:, :, blk] = data[i] in torch, median of 3 after 1 warm-up: "
                       f"{t_unpack * 1e3:.1f} ms; cpu={cpu_model()}")}
        log(f"C5 pack cpu: {res['pack']['cpu_baseline']['value']} GB/s, exact={exact}; "
            f"unpack cpu: {res['unpack']['cpu_baseline']['value']} GB/s")
        del hpool, payload, x
    else:
        want = pool[:, :, ids].permute(2, 0, 1, 3, 4, 5).contiguous()
        res["pack"]["bit_exact"] = bool(torch.equal(out.view(torch.int16), want.view(torch.int16)))
        res["pack"]["check"] = "GPU payload == torch GPU indexing, bit for bit (no CPU leg)"
        del pool, want
    del out
    torch.cuda.empty_cache()
    return res


def kv_write_leg(steps: int, warmup: int) -> dict:
    """C5's prefill chunk written into the cache: 1024 tokens at positions
    2048..3071 of one sequence, K and V as strided fp32 slices of a fused QKV
    output [1024, 3 * 4096], cast into a bf16 layer cache (the engine's step at
    torch_engine.py:294-308).  Checked bit for bit against the reference's own
    ``fk[slots] = k.to(dtype)`` on the same GPU, which is also timed."""
    import torch

    from heteroserve import _hip
    from hsbench.timing import Event, time_steps

    lib = _hip.lib()
    dev = "cuda:0"
    nb, bs, h, d, T, start = 8192, 16, 32, 128, 1024, 2048
    g = torch.Generator(device=dev).manual_seed(43)
    kc = torch.zeros((nb, bs, h, d), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    table = torch.randperm(nb, generator=g, device=dev)[: (start + T) // bs].to(torch.int32)
    bt = table.view(1, -1).contiguous()
    pos = torch.arange(start, start + T, dtype=torch.int32, device=dev)
    seq = torch.zeros(T, dtype=torch.int32, device=dev)
    kvd = h * d
    qkv = torch.randn((T, 3 * kvd), generator=g, device=dev)
    k, v = qkv[:, kvd:2 * kvd], qkv[:, 2 * kvd:]
    stream = torch.cuda.current_stream().cuda_stream
    args = (kc.data_ptr(), vc.data_ptr(), _hip.dtype_code(kc.dtype), nb, bs, h, d, bt.data_ptr(),
            bt.shape[0], bt.shape[1], pos.data_ptr(), seq.data_ptr(), T, k.data_ptr(),
            v.data_ptr(), _hip.DTYPE_F32, qkv.stride(0), stream)

    def step():
        _hip.check(lib.hs_kv_append(*args))

    def arm(s_, e_):
        _hip.check(lib.hs_profile_next_launch(s_.handle, e_.handle))

    step_ms, kernel_ms, _ = time_steps(step, steps, warmup, stream, arm)
    # the reference's code path on the same device: slots_for + index_put
    slots = (table.long()[pos.long() // bs] * bs + pos.long() % bs)
    fk, fv = kc.clone().view(nb * bs, h, d), vc.clone().view(nb * bs, h, d)
    fk.zero_()
    fv.zero_()

    def ref_step():
        fk[slots] = k.view(T, h, d).to(kc.dtype)
        fv[slots] = v.view(T, h, d).to(vc.dtype)

    for _ in range(warmup):
        ref_step()
    e0, e1 = Event(), Event()
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        ref_step()
    e1.record(stream)
    ref_ms = e0.elapsed_ms(e1) / steps
    exact = bool(torch.equal(fk.view(torch.int16), kc.view(nb * bs, h, d).view(torch.int16)) and
                 torch.equal(fv.view(torch.int16), vc.view(nb * bs, h, d).view(torch.int16)))
    nbytes = 2 * T * kvd * (4 + 2)        # read fp32 rows, write bf16 rows, K and V
    k_ms = statistics.mean(kernel_ms)
    del kc, vc, fk, fv, qkv
    torch.cuda.empty_cache()
    return dict(step_ms=step_ms, kernel_ms=k_ms, ref_ms=ref_ms, bytes=nbytes, bit_exact=exact,
                kernel_gbs=nbytes / (k_ms * 1e-3) / 1e9)


def tables_leg(steps: int) -> dict:
    """C5's decode batch (255 sequences) prepared for one decode step as the
    engine does it (torch_engine.py:215-240): the int32 block-table tensor,
    the slot of each sequence's new token, and that token's K/V written into
    a bf16 layer cache.  The reference builds the table with one host-to-device
    copy per sequence (TorchBlockAllocator.block_table_tensor,
    torch_blocks.py:75-85) and the slots with one device-to-host ``.tolist()``
    per sequence (torch_engine.py:221-227), then ``fk[slots] = k``; here the
    lists go up in one packed copy (hs_block_tables) and hs_kv_append computes
    the slots on the device.  Both are timed on the host clock around a
    synchronised step (host work included: that is what the rewrite removes);
    tables and caches are compared bit for bit."""
    import numpy as np
    import torch

    from heteroserve import _hip
    from heteroserve.kv import pack
    from hsbench import cases

    dev = "cuda:0"
    ctx, tables = cases.c5_decode_tables()
    B, nb, bs, h, d = len(tables), cases.C5_POOL_BLOCKS, 16, 32, 128
    width = max(len(t) for t in tables)
    pos_np = (ctx - 1).astype(np.int64)
    g = torch.Generator(device=dev).manual_seed(45)
    kvd = h * d
    qkv = torch.randn((B, 3 * kvd), generator=g, device=dev)
    k, v = qkv[:, kvd:2 * kvd], qkv[:, 2 * kvd:]
    pos = torch.as_tensor(pos_np, dtype=torch.int32, device=dev)
    caches = [torch.zeros((nb, bs, h, d), dtype=torch.bfloat16, device=dev) for _ in range(4)]

    def ours():
        bt = pack.block_table_tensor(tables, pad_to=width, device=dev)
        _hip.kv_append(caches[0], caches[1], bt, pos, k.view(B, h, d), v.view(B, h, d))
        return bt

    fk, fv = caches[2].view(nb * bs, h, d), caches[3].view(nb * bs, h, d)

    def reference():
        out = torch.full((B, width), -1, dtype=torch.int32, device=dev)
        for i, t in enumerate(tables):
            out[i, :len(t)] = torch.as_tensor(t[:width], dtype=torch.int32, device=dev)
        slots = []
        for b in range(B):
            ids = torch.as_tensor(out[b][out[b] >= 0].tolist(), dtype=torch.long, device=dev)
            p = torch.as_tensor(pos_np[b:b + 1], dtype=torch.long, device=dev)
            slots.append((ids[p // bs] * bs + p % bs)[0])
        slots = torch.stack(slots)
        fk[slots] = k.view(B, h, d).to(fk.dtype)
        fv[slots] = v.view(B, h, d).to(fv.dtype)
        return out

    def host_timed(fn) -> float:
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            fn()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) / steps * 1e3

    ours_ms = host_timed(ours)
    ref_ms = host_timed(reference)
    exact = bool(torch.equal(ours(), reference()))
    torch.cuda.synchronize()
    for a_, b_ in ((caches[0], caches[2]), (caches[1], caches[3])):
        exact = exact and bool(torch.equal(a_.view(torch.int16), b_.view(torch.int16)))
    del caches, fk, fv
    torch.cuda.empty_cache()
    return {"us_per_step": round(ours_ms * 1e3, 1), "reference_torch_us": round(ref_ms * 1e3, 1),
            "speedup": round(ref_ms / ours_ms, 1), "bit_exact": exact, "batch": B,
            "note": "host clock around a synchronised step: block table + new-token slots + "
                    "K/V write of one layer; reference = torch_blocks.block_table_tensor + "
                    "the engine's per-sequence slot loop + fk[slots] = k"}


def c5_step_leg(steps: int, warmup: int, with_cpu: bool) -> dict:
    """C5 as one serving step on one stream: the prefill chunk's K/V written
    into its cache (1024 tokens at positions 2048..3071, fp32 slices of a fused
    QKV output), its causal attention on the matrix cores, the 255 decode
    tokens' K/V appended at ctx - 1, the decode of those 255 sequences (half
    of them sharing a 1024-token prefix: hs_decode_shared, which reads a
    partition that several sequences hold once for all of them), and the
    4096-block migration pack of the decode pool.  Returns the step time,
    each part timed alone, and the plain hs_decode of the same batch.

    With with_cpu, both attention outputs of the last step are checked
    against the oracle on the pools as the step's own writes left them
    (the engine's write-then-attend order, torch_engine.py:215-245 and
    :294-313): the chunk's every row and head against prefill_one (B = 1,
    the engine's call shape), every decode sequence against decode_one,
    each timed on the host cores as that part's CPU baseline."""
    import torch

    from heteroserve import _hip
    from hsbench import cases
    from hsbench.timing import Event

    lib = _hip.lib()
    dev = "cuda:0"
    stream = torch.cuda.current_stream().cuda_stream
    dc, pc = cases.c5_decode(dev), cases.c5_prefill(dev)
    g = torch.Generator(device=dev).manual_seed(44)
    T, H, D = pc.q.shape
    kvd = H * D
    pkc, pvc = pc.k_cache, pc.v_cache
    pnb, bs, hkv, _ = pkc.shape
    qkv_p = torch.randn((T, 3 * kvd), generator=g, device=dev)
    ppos = torch.arange(2048, 2048 + T, dtype=torch.int32, device=dev)
    pseq = torch.zeros(T, dtype=torch.int32, device=dev)
    pout = torch.empty((T, H, D), dtype=torch.float32, device=dev)
    B = dc.q.shape[0]
    dkc, dvc = dc.k_cache, dc.v_cache
    dnb = dkc.shape[0]
    dmb = dc.block_tables.shape[1]
    qkv_d = torch.randn((B, 3 * kvd), generator=g, device=dev)
    dpos = (dc.context_lens - 1).to(torch.int32).contiguous()
    dseq = torch.arange(B, dtype=torch.int32, device=dev)
    dout = torch.empty((B, H, D), dtype=torch.float32, device=dev)
    ws_bytes = lib.hs_decode_shared_workspace_bytes(B, H, hkv, D, bs, dmb, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    ids = torch.as_tensor(cases.c5_pack_ids(dnb), dtype=torch.int64, device=dev)
    pool = dc.pool
    page = pool[0, 0, 0].numel() * pool.element_size()
    pack_out = torch.empty((ids.numel(), 1, 2, bs, hkv, D), dtype=pool.dtype, device=dev)
    f32 = _hip.DTYPE_F32
    kdt = _hip.dtype_code(dkc.dtype)
    pws, pws_bytes = _hip._prefill_workspace(lib, 1, T, H, D, True, True, dev)
    parts = {
        "kv_write_chunk": lambda: lib.hs_kv_append(
            pkc.data_ptr(), pvc.data_ptr(), kdt, pnb, bs, hkv, D, pc.block_tables.data_ptr(),
            pc.block_tables.shape[0], pc.block_tables.shape[1], ppos.data_ptr(), pseq.data_ptr(),
            T, qkv_p[:, kvd:].data_ptr(), qkv_p[:, 2 * kvd:].data_ptr(), f32, qkv_p.stride(0),
            stream),
        "prefill": lambda: lib.hs_prefill_varlen(
            pc.q.data_ptr(), pc.cu_seqlens.data_ptr(), T, pkc.data_ptr(), pvc.data_ptr(), kdt,
            pnb, pc.block_tables.data_ptr(), pc.context_lens.data_ptr(), pout.data_ptr(), 1, H,
            hkv, D, bs, pc.block_tables.shape[1], float(pc.scale), 1,
            pws.data_ptr() if pws is not None else None, pws_bytes, stream),
        "kv_write_decode": lambda: lib.hs_kv_append(
            dkc.data_ptr(), dvc.data_ptr(), kdt, dnb, bs, hkv, D, dc.block_tables.data_ptr(), B,
            dmb, dpos.data_ptr(), dseq.data_ptr(), B, qkv_d[:, kvd:].data_ptr(),
            qkv_d[:, 2 * kvd:].data_ptr(), f32, qkv_d.stride(0), stream),
        "decode": lambda: lib.hs_decode_shared(
            dc.q.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), kdt, dnb,
            dc.block_tables.data_ptr(), dc.context_lens.data_ptr(), dout.data_ptr(), B, H, hkv,
            D, bs, dmb, float(dc.scale), 0, ws.data_ptr(), ws_bytes, stream),
        "pack": lambda: lib.hs_kv_pack(pool.data_ptr(), 1, dnb, page, ids.data_ptr(),
                                       ids.numel(), pack_out.data_ptr(), stream),
    }

    def timed(fns) -> float:
        for _ in range(warmup):
            for f in fns:
                _hip.check(f())
        e0, e1 = Event(), Event()
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            for f in fns:
                _hip.check(f())
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_ms(e1) / steps

    step_ms = timed(list(parts.values()))
    part_ms = {k: timed([f]) for k, f in parts.items()}
    plain_ms = timed([lambda: lib.hs_decode(
        dc.q.data_ptr(), dkc.data_ptr(), dvc.data_ptr(), kdt, dnb, dc.block_tables.data_ptr(),
        dc.context_lens.data_ptr(), dout.data_ptr(), B, H, hkv, D, bs, dmb, float(dc.scale), 0,
        0, ws.data_ptr(), ws_bytes, stream)])
    work = {
        "kv_write_chunk": ("GB/s", 2 * T * kvd * (4 + 2) / 1e9),
        "prefill": ("TFLOP/s", pc.prefill_flops() / 1e12),
        "kv_write_decode": ("GB/s", 2 * B * kvd * (4 + 2) / 1e9),
        "decode": ("GB/s", dc.unique_decode_bytes() / 1e9),
        "pack": ("GB/s", 2 * pack_out.numel() * pack_out.element_size() / 1e9),
    }
    peak = {"GB/s": HBM_PEAK_GBS, "TFLOP/s": MFMA_F16_PEAK_TFLOPS}
    out = {"us_per_step": round(step_ms * 1e3, 2), "parts": {}}
    for k, ms in part_ms.items():
        unit, amount = work[k]
        rate = amount / (ms * 1e-3)
        out["parts"][k] = {"us": round(ms * 1e3, 2), unit: round(rate, 1),
                           "frac": round(rate / peak[unit], 4)}
    out["parts"]["decode"]["basis"] = "unique K/V bytes (shared prefix counted once)"
    out["parts"]["decode"]["path"] = "hs_decode_shared"
    out["decode_plain_us"] = round(plain_ms * 1e3, 2)
    # the outputs of the last timed step: the shared-page decode and the
    # chunk prefill, on the pools after the step's writes
    for f in (parts["decode"], parts["prefill"]):
        _hip.check(f())
    torch.cuda.synchronize()
    if with_cpu:
        pcpu, pouts = cpu_prefill_baseline(pc)
        perr = max_err_prefill(pc, pout, pouts)
        out["parts"]["prefill"].update(cpu_baseline=pcpu, max_abs_err=perr,
                                       parity_sample="every row of the chunk, all heads")
        del pouts
        dcpu, douts = cpu_decode_baseline(dc, n_seq=0)
        derr = max_err_decode(dout, douts)
        out["parts"]["decode"].update(cpu_baseline=dcpu, max_abs_err=derr,
                                      parity_sample="every sequence")
        del douts
        log(f"C5 step parity: prefill {perr:.2e} (cpu {pcpu['value']} TFLOP/s), "
            f"shared-page decode {derr:.2e} (cpu {dcpu['value']} GB/s)")
    del dc, pc, pool, pack_out, qkv_p, qkv_d, ws
    torch.cuda.empty_cache()
    return out


# ---------------------------------------------------------------------------
# every entry point of the reference's harness (scripts/bench_kernel.py)
# ---------------------------------------------------------------------------


def _timed_calls(fn, iters: int) -> tuple:
    """(host µs per call, device µs per call) over `iters` calls after one
    warm-up call: the host clock between synchronisations, as the
    reference's harness times (scripts/bench_kernel.py:53-60, Python and
    allocation overhead included), and HIP events around the same calls on
    the launch stream."""
    import torch

    from hsbench.timing import Event

    stream = torch.cuda.current_stream().cuda_stream
    fn()
    torch.cuda.synchronize()
    e0, e1 = Event(), Event()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(iters):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    host = (time.perf_counter() - t0) / iters
    return host * 1e6, e0.elapsed_ms(e1) / iters * 1e3


def _entry_row(fn, want, nbytes: int, iters: int, rate_unit: str = "GB/s") -> dict:
    """Check one entry point's output against the oracle, then time it."""
    got = fn()
    err = (got.detach().float().cpu() - want).abs().max().item()
    host_us, dev_us = _timed_calls(fn, iters)
    row = {"us_per_call": round(host_us, 2), "device_us_per_call": round(dev_us, 2),
           "max_abs_err": float(f"{err:.3e}")}
    if rate_unit == "GB/s":
        row["gbs"] = round(nbytes / (host_us * 1e-6) / 1e9, 1)
        row["hbm_frac"] = round(row["gbs"] / HBM_PEAK_GBS, 4)
    else:
        row["tflops"] = round(nbytes / (host_us * 1e-6) / 1e12, 2)
        row["mfma_frac"] = round(row["tflops"] / MFMA_F16_PEAK_TFLOPS, 4)
    return row


def c2_entry_points(case, outs: dict, iters: int) -> dict:
    """v2 (one pass) and v3 with the reference's choose_num_splits at C2,
    through the drop-in functions, checked against the headline's per-sequence
    oracle outputs (`outs`)."""
    import torch

    from heteroserve.model import paged_attn_v2, paged_attn_v3

    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
            case.scale)
    B, H, _ = case.q.shape
    splits = paged_attn_v3.choose_num_splits(B, H, case.block_tables.shape[1] * 16)
    nbytes = case.decode_bytes()
    res = {}
    for key, fn in (("v2_paged_attention_v2", lambda: paged_attn_v2.paged_attention_v2(*args)),
                    (f"v3_paged_attention_v3_choose_num_splits_{splits}",
                     lambda: paged_attn_v3.paged_attention_v3(*args, splits))):
        got = fn()
        err = max_err_decode(got, outs)
        host_us, dev_us = _timed_calls(fn, iters)
        res[key] = {"us_per_call": round(host_us, 2), "device_us_per_call": round(dev_us, 2),
                    "gbs": round(nbytes / (host_us * 1e-6) / 1e9, 1),
                    "hbm_frac": round(nbytes / (host_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                    "max_abs_err": float(f"{err:.3e}")}
        log(f"C2 {key}: {host_us:.1f} us/call, err {err:.2e}")
    del got
    torch.cuda.empty_cache()
    return res


# The reference's published decode rows (README :332-346, :423-430): one
# layer of GPT-2 shape (ModelConfig(): 12 heads, head dim 64), fp16 KV,
# block_size 16, every context at the same length, on one T4.
REF_SHAPES = ((16, 512, 16, 128), (32, 2048, 64, 512))   # (B, ctx, published splits, prefill S)
REF_SWEEP_SPLITS = (1, 2, 4, 8, 16, 32, 64)


def reference_harness_leg(with_cpu: bool, iters: int = 50) -> dict:
    """scripts/bench_kernel.py on MI355X: for each published shape, the
    gather controls (gather + dense attention, gather + PyTorch SDPA), v1,
    v2, v3 with choose_num_splits and v3 at the published split count, each
    through its drop-in Python function, checked against the oracle
    (paged_attention_torch on the CPU, same inputs) and timed as the
    reference times them; the v3 split sweep at B16/ctx512; and the prefill
    half (--prefill S: the scalar and the matrix-core kernel at chunk S of
    the same contexts, against prefill_one per sequence).  Inputs as the
    harness makes them: N(0, 1) K/V and queries, scale 1/8, a pool of
    B * (ctx / 16 + 4) blocks; the tables here are a seeded permutation
    (scattered pages) rather than the allocator's order."""
    import numpy as np
    import torch

    from heteroserve.kv import pack
    from heteroserve.model import (paged_attn, paged_attn_prefill, paged_attn_v2,
                                   paged_attn_v3, paged_attn_wmma)
    from hsbench import cases
    from oracle.attention import paged_attention_torch, prefill_one

    dev = "cuda:0"
    torch.set_num_threads(host_threads())
    res = {}
    for B, ctx, pub_splits, S in REF_SHAPES:
        name = f"B{B}_ctx{ctx}"
        case = cases.build_decode(name, np.full(B, ctx), 12, 12, 64, max(64, B * (ctx // 16 + 4)),
                                  torch.float16, dev, seed=60 + B)
        args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                case.scale)
        host = [t.cpu() for t in args[:5]]
        want = paged_attention_torch(*host, case.scale)
        nbytes = case.decode_bytes()
        splits = paged_attn_v3.choose_num_splits(B, 12, case.block_tables.shape[1] * 16)

        def gather_dense():
            ks, vs = pack.gather_kv_batch(case.pool, case.tables, ctx, 0)
            sc = torch.einsum("bhd,bkhd->bhk", case.q, ks.float()) * case.scale
            return torch.einsum("bhk,bkhd->bhd", torch.softmax(sc, -1), vs.float())

        def gather_sdpa():
            ks, vs = pack.gather_kv_batch(case.pool, case.tables, ctx, 0)
            o = torch.nn.functional.scaled_dot_product_attention(
                case.q.unsqueeze(2), ks.permute(0, 2, 1, 3).float().contiguous(),
                vs.permute(0, 2, 1, 3).float().contiguous(), scale=case.scale)
            return o.squeeze(2)

        entries = [
            ("gather + dense attention (control)", gather_dense),
            ("gather + PyTorch SDPA (control)", gather_sdpa),
            ("v1 paged_attention", lambda: paged_attn.paged_attention(*args)),
            ("v2 paged_attention_v2", lambda: paged_attn_v2.paged_attention_v2(*args)),
            (f"v3 paged_attention_v3, choose_num_splits = {splits}",
             lambda: paged_attn_v3.paged_attention_v3(*args, splits)),
        ]
        if pub_splits != splits:
            entries.append((f"v3 paged_attention_v3, {pub_splits} splits (the published row)",
                            lambda: paged_attn_v3.paged_attention_v3(*args, pub_splits)))
        rows = {}
        for label, fn in entries:
            rows[label] = _entry_row(fn, want, nbytes, iters)
        shape = {"batch": B, "context": ctx, "heads": 12, "head_dim": 64, "kv_dtype": "float16",
                 "bytes_per_call": nbytes, "rows": rows}
        if with_cpu:
            t = median_time(lambda: paged_attention_torch(*host, case.scale))
            shape["cpu_baseline"] = {
                "value": float(f"{nbytes / t / 1e9:.4g}"), "unit": "GB/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": (f"the whole batch in one call of oracle/attention.py "
                           f"paged_attention_torch (torch fp32 CPU), median of 3 after 1 "
                           f"warm-up: {t * 1e3:.2f} ms; cpu={cpu_model()}")}
        if B == 16:
            sweep = {}
            for sp in REF_SWEEP_SPLITS:
                sweep[str(sp)] = _entry_row(
                    lambda sp=sp: paged_attn_v3.paged_attention_v3(*args, sp), want, nbytes, iters)
            shape["v3_split_sweep"] = sweep
        res[f"decode_{name}"] = shape
        log(f"reference shapes, decode {name}: " + ", ".join(
            f"{k.split(' (')[0]} {v['us_per_call']:.1f} us" for k, v in rows.items()))

        # --prefill S: S query rows at the end of every context
        q4 = torch.randn((B, S, 12, 64), generator=torch.Generator(device=dev).manual_seed(B),
                         device=dev)
        pargs = (q4, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                 case.scale)
        qh = q4.cpu()
        kh, vh = host[1], host[2]
        pwant = torch.stack([prefill_one(qh[b], kh, vh, host[3][b], ctx, case.scale)
                             for b in range(B)])
        flops = 4 * 12 * 64 * B * (S * (ctx - S) + S * (S + 1) // 2)
        prows = {
            "prefill kernel (scalar fused), paged_attention_prefill": _entry_row(
                lambda: paged_attn_prefill.paged_attention_prefill(*pargs), pwant, flops,
                max(5, iters // 3), "TFLOP/s"),
            "prefill kernel (matrix cores), paged_attention_prefill_wmma": _entry_row(
                lambda: paged_attn_wmma.paged_attention_prefill_wmma(*pargs), pwant, flops,
                max(5, iters // 3), "TFLOP/s"),
        }
        res[f"prefill_{name}_S{S}"] = {"batch": B, "context": ctx, "chunk": S,
                                       "useful_flops": flops, "rows": prows}
        log(f"reference shapes, prefill {name} S{S}: " + ", ".join(
            f"{k.split(',')[0]} {v['us_per_call']:.1f} us" for k, v in prows.items()))
        del case, args, host, q4, pargs
        torch.cuda.empty_cache()
    return res


def gqa_one_partition_leg(iters: int = 20) -> dict:
    """Rows that one fixed partition covers, on the grouped-query path: 64
    sequences of 100..700 tokens, 32 query heads on 8 KV heads, D 128, bf16.
    The library default (fixed partitions here: one round of the device
    holds them, so the even split does not apply) against explicit 768-token
    partitions, one a row, on the split-operand matrix-core kernel, and v2
    (one pass), which runs the VALU kernel.  Each checked against the
    oracle, then timed."""
    import numpy as np
    import torch

    from heteroserve import _hip
    from heteroserve.model import paged_attn, paged_attn_v2
    from hsbench import cases
    from oracle.attention import paged_attention_torch

    rng = np.random.default_rng(5)
    lens = rng.integers(100, 700, size=64, endpoint=True)
    case = cases.build_decode("gqa-one-partition", lens, 32, 8, 128, 4096, torch.bfloat16,
                              "cuda:0", seed=5)
    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
            case.scale)
    want = paged_attention_torch(*[t.cpu() for t in args[:5]], case.scale)
    nbytes = case.decode_bytes()
    res = {"library default (matrix cores)": _entry_row(
               lambda: paged_attn.paged_attention(*args), want, nbytes, iters),
           "768-token partitions (matrix cores, one a row)": _entry_row(
               lambda: _hip.decode(*args, 0, partition_tokens=768), want, nbytes, iters),
           "v2 one pass (VALU)": _entry_row(
               lambda: paged_attn_v2.paged_attention_v2(*args), want, nbytes, iters)}
    log("GQA one-partition rows: " + ", ".join(
        f"{k.split(' (')[0]} {v['device_us_per_call']:.1f} us" for k, v in res.items()))
    del case, args
    torch.cuda.empty_cache()
    return res


# ---------------------------------------------------------------------------
# CPU baselines: the oracle on this host's cores, on the same inputs; their
# outputs are the parity reference of the GPU legs
# ---------------------------------------------------------------------------


def cpu_decode_baseline(case, n_seq: int = 0, seed: int = 7):
    """Per-sequence torch oracle (oracle/attention.py decode_one) over the
    case's sequences, all of them when n_seq is 0, else a seeded sample of
    n_seq; returns (baseline dict, {sequence: oracle output})."""
    import numpy as np
    import torch

    from oracle.attention import decode_one

    torch.set_num_threads(host_threads())
    rng = np.random.default_rng(seed)
    n_pick = len(case.ctx) if n_seq <= 0 else min(n_seq, len(case.ctx))
    pick = sorted(rng.choice(len(case.ctx), size=n_pick, replace=False).tolist())
    total, outs = 0.0, {}
    for b in pick:
        n = int(case.ctx[b])
        nblk = -(-n // 16)
        blocks = case.block_tables[b, :nblk].long()
        q, kb, vb = (case.q[b].cpu(), case.k_cache.index_select(0, blocks).cpu(),
                     case.v_cache.index_select(0, blocks).cpu())
        tbl = torch.arange(nblk, dtype=torch.int32)
        total += median_time(lambda: outs.__setitem__(b, decode_one(q, kb, vb, tbl, n,
                                                                    case.scale)))
    tokens = int(sum(int(case.ctx[b]) for b in pick))
    nbytes = tokens * case.row_bytes()
    what = "all" if n_pick == len(case.ctx) else f"a seeded sample of {n_pick} of the"
    return {
        "value": float(f"{nbytes / total / 1e9:.4g}"),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "sample": (f"{what} {len(case.ctx)} {case.name} sequences ({tokens} of "
                   f"{int(case.ctx.sum())} context tokens), oracle/attention.py decode_one "
                   f"(torch fp32 CPU) per sequence, median of 3 after 1 warm-up, summed: "
                   f"{total * 1e3:.1f} ms for {nbytes / 1e6:.1f} MB of K+V (a rate, so the "
                   f"sample's bytes over the sample's time); cpu={cpu_model()}"),
    }, outs


def cpu_decode_batched(case):
    """The batched torch oracle (oracle/attention.py paged_attention_torch, the
    reference's paged_attention_torch) over the whole case in one call, as the
    reference computes it on the CPU; returns (baseline dict, output)."""
    import torch

    from oracle.attention import paged_attention_torch

    torch.set_num_threads(host_threads())
    args = [t.cpu() for t in (case.q, case.k_cache, case.v_cache, case.block_tables,
                              case.context_lens)]
    res = {}
    t = median_time(lambda: res.__setitem__("out", paged_attention_torch(*args, case.scale)))
    nbytes = case.decode_bytes()
    return {
        "value": float(f"{nbytes / t / 1e9:.4g}"), "unit": "GB/s", "cores": torch.get_num_threads(),
        "kind": "port", "us_per_step": round(t * 1e6, 1),
        "sample": (f"the whole {case.name} batch ({len(case.ctx)} sequences) in one call of "
                   f"oracle/attention.py paged_attention_torch (torch fp32 CPU), median of 3 "
                   f"after 1 warm-up: {t * 1e3:.2f} ms for {nbytes / 1e6:.2f} MB of K+V; "
                   f"cpu={cpu_model()}"),
    }, res["out"]


def cpu_prefill_baseline(case, heads: int = 0):
    """The prefill oracle (oracle/attention.py prefill_one, the reference's
    paged_attention_prefill_torch per sequence) over every sequence of the
    case for `heads` of its heads (all of them when 0); useful causal FLOPs of
    that sample over the summed median times.  Returns (baseline dict,
    {sequence: oracle output [S_b, heads, D]})."""
    import torch

    from oracle.attention import prefill_one

    torch.set_num_threads(host_threads())
    D = case.head_dim
    heads = heads or case.n_heads
    cu = case.cu_seqlens.cpu().tolist()
    total, flops, outs = 0.0, 0, {}
    for b in range(len(case.ctx)):
        n, S = int(case.ctx[b]), cu[b + 1] - cu[b]
        nblk = -(-n // 16)
        blocks = case.block_tables[b, :nblk].long()
        q = case.q[cu[b]:cu[b + 1], :heads].cpu()
        kb = case.k_cache.index_select(0, blocks)[:, :, :heads].cpu()
        vb = case.v_cache.index_select(0, blocks)[:, :, :heads].cpu()
        tbl = torch.arange(nblk, dtype=torch.int32)
        total += median_time(lambda: outs.__setitem__(b, prefill_one(q, kb, vb, tbl, n,
                                                                     case.scale)))
        P = n - S
        flops += 4 * heads * D * (S * P + S * (S + 1) // 2)
    return {
        "value": float(f"{flops / total / 1e12:.4g}"), "unit": "TFLOP/s",   # 4 significant digits
        "cores": torch.get_num_threads(), "kind": "port",
        "sample": (f"all {len(case.ctx)} {case.name} sequences, {heads} of {case.n_heads} heads, "
                   f"oracle/attention.py prefill_one (torch fp32 CPU), median of 3 after 1 "
                   f"warm-up, summed: {total * 1e3:.1f} ms for {flops / 1e9:.2f} useful GFLOP; "
                   f"cpu={cpu_model()}"),
    }, outs


def max_err_decode(got, outs: dict) -> float:
    return max((got[b].detach().cpu() - w).abs().max().item() for b, w in outs.items())


def max_err_prefill(case, got, outs: dict, heads: int = 0) -> float:
    cu = case.cu_seqlens.cpu().tolist()
    heads = heads or case.n_heads
    return max((got[cu[b]:cu[b + 1], :heads].detach().cpu() - w).abs().max().item()
               for b, w in outs.items())


# ---------------------------------------------------------------------------


def decode_config(case, partition: int) -> dict:
    kv_dtype = str(case.k_cache.dtype).replace("torch.", "")
    cfg = {
        "workload": f"{case.name} paged decode, one layer",
        "batch": len(case.ctx), "heads": case.n_heads, "kv_heads": case.kv_heads,
        "head_dim": case.head_dim, "block_size": 16, "kv_dtype": kv_dtype,
        "sum_context": int(case.ctx.sum()), "max_context": int(case.ctx.max()),
        "num_blocks": int(case.k_cache.shape[0]),
        # (C1, a grid too small to fill the CUs, takes the small-grid form)
        "decomposition": (f"fixed partitions of {partition} tokens + LSE merge"
                          if partition else
                          "library default: one workgroup per (row, head), keys split over "
                          "its waves, no merge"
                          if case.name == "C1" else
                          "library default: even split (all pages cut into one equal range "
                          "per resident workgroup, then an LSE merge of the rows cut)"),
        "parallelism": "none (one GPU)",
    }
    if case.meta.get("shared_blocks"):
        cfg["unique_bytes"] = case.unique_decode_bytes()
    return cfg


def secondary_decode(name: str, kernel: str, steps: int, warmup: int, with_cpu: bool,
                     batched_cpu: bool = False, n_seq: int = 0) -> dict:
    """One more decode configuration: step time, roofline of its partition
    kernel, CPU baseline and parity against the oracle outputs."""
    import torch

    from hsbench import cases

    case = cases.CONFIGS[name]("cuda:0")
    # the previous leg ended with seconds of CPU baseline: warm the clocks up
    # (C1's 5-us steps are bound by the host's launch rate, not the clocks)
    dec = decode_leg(case, steps, warmup, warm_ms=0.0 if name == "C1" else 50.0)
    res = {"us_per_step": round(dec["step_ms"] * 1e3, 2), "gbs": round(dec["step_gbs"], 1),
           "hbm_frac": round(dec["step_gbs"] / HBM_PEAK_GBS, 4),
           "config": decode_config(case, 0),
           "roofline": roofline("hbm", kernel, dec["bytes"], dec["kernel_ms"],
                                leg_traffic(name))}
    log(f"{name} decode: step {dec['step_ms'] * 1e3:.1f} us ({dec['step_gbs']:.0f} GB/s), "
        f"kernel {dec['kernel_ms'] * 1e3:.1f} us ({dec['kernel_gbs']:.0f} GB/s)")
    if with_cpu:
        if batched_cpu:
            cpu, want = cpu_decode_batched(case)
            err = (dec["out"].cpu() - want).abs().max().item()
            res["parity_sample"] = "every sequence"
        else:
            cpu, outs = cpu_decode_baseline(case, n_seq=n_seq)
            err = max_err_decode(dec["out"], outs)
            res["parity_sample"] = (f"{len(outs)} of {len(case.ctx)} sequences (the CPU "
                                    "baseline's sample)")
        res["cpu_baseline"] = cpu
        res["max_abs_err"] = err
        log(f"{name} cpu baseline: {cpu['value']} GB/s; max abs err {err:.2e}")
    del case, dec
    torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C2", choices=["C1", "C2", "C2-gqa", "C3", "B64-4k", "C5-decode"],
                    help="decode configuration of the headline line")
    ap.add_argument("--partition", type=int, default=0,
                    help="decode partition tokens (0 = library default)")
    ap.add_argument("--no-secondary", action="store_true", help="skip the secondary legs")
    ap.add_argument("--no-cpu", action="store_true",
                    help="skip the CPU baselines (and with them the parity checks of the "
                         "attention legs)")
    args = ap.parse_args()

    if args.gpus != 1:
        log(f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
            "(the paged-attention path has no multi-GPU decomposition on this box).")
        return 2

    import torch

    from heteroserve import _hip
    from hsbench import cases

    if not _hip.ready():
        log(f"libhsattn unavailable: {_hip.error()}")
        return 1
    dev = "cuda:0"
    log(f"device: {torch.cuda.get_device_name(0)}; host: {cpu_model()}, "
        f"{host_threads()} threads")
    with_cpu = not args.no_cpu
    errors = {}          # leg -> max abs error (attention legs)
    exact = {}           # leg -> bit-exact (copy legs)

    # the decode legs' pools, one case at a time, in one buffer reserved as
    # the process's first large allocation (as an engine allocates its KV
    # pool once); the largest is C2's and B64-4k's 65536-block pool
    arena = torch.empty(65536 * 2 * 16 * 32 * 128 * 2, dtype=torch.uint8, device=dev)
    cases.set_pool_arena(arena)
    case = cases.CONFIGS[args.config](dev)
    log(f"{case.name}: B={len(case.ctx)} sum(ctx)={int(case.ctx.sum())} "
        f"bytes={case.decode_bytes() / 1e9:.3f} GB")
    dec = decode_leg(case, args.steps, args.warmup, args.partition)
    log(f"decode: step {dec['step_ms'] * 1e3:.1f} us ({dec['step_gbs']:.0f} GB/s), "
        f"main kernel {dec['kernel_ms'] * 1e3:.1f} us ({dec['kernel_gbs']:.0f} GB/s)")
    cpu = None
    if with_cpu:
        cpu, outs = cpu_decode_baseline(case)
        errors[case.name] = max_err_decode(dec["out"], outs)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads; "
            f"max abs err {errors[case.name]:.2e}")
        if not args.no_secondary and args.config == "C2":
            c2_entries = c2_entry_points(case, outs, max(10, args.steps // 2))
            for k, v in c2_entries.items():
                errors[f"C2_{k}"] = v["max_abs_err"]
        del outs
    config = decode_config(case, args.partition)
    headline_name = case.name
    del case
    torch.cuda.empty_cache()

    secondary = {}
    if not args.no_secondary and with_cpu and args.config == "C2":
        secondary["C2_entry_points"] = c2_entries
    if not args.no_secondary:
        legs = [("C1", "row_attn_wg_kernel<_Float16, 64, true, 1, 16>", True, 0),
                ("C2-gqa", "splitmm_even_kernel<Bf16Ops, 128, true, 4>", False, 16),
                ("C3", "row_attn_part_kernel<Bf16, 128, true, 1>", False, 4),
                ("B64-4k", "row_attn_part_kernel<Bf16, 128, true, 1>", False, 8)]
        for name, kernel, batched, n_seq in legs:
            if name == headline_name:
                continue
            r = secondary_decode(name, kernel, args.steps, args.warmup, with_cpu,
                                 batched_cpu=batched, n_seq=n_seq)
            secondary[f"{name}_decode"] = r
            if "max_abs_err" in r:
                errors[name] = r["max_abs_err"]
    # the other legs hold several cases at once: their own allocations
    cases.set_pool_arena(None)
    del arena
    torch.cuda.empty_cache()
    if not args.no_secondary:
        pc = cases.c4_prefill(dev)
        # >= 60 warm-up launches (~20 ms): after the memory-bound decode legs
        # the clock takes tens of milliseconds of MFMA work to ramp up
        pre = prefill_leg(pc, max(20, args.steps // 5), max(60, args.warmup))
        secondary["C4_prefill"] = {
            "us_per_step": round(pre["step_ms"] * 1e3, 2),
            "tflops": round(pre["step_tflops"], 2),
            "kernel_tflops": round(pre["kernel_tflops"], 2),
            "mfma_frac": round(pre["kernel_tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
            "useful_flops": pre["flops"],
            "roofline": roofline("mfma", "prefill_stream_kernel<Bf16, 128>", pre["flops"],
                                 pre["kernel_ms"], leg_traffic("C4")),
        }
        log(f"C4 prefill: {pre['step_ms'] * 1e3:.1f} us, {pre['kernel_tflops']:.1f} TFLOP/s")
        if with_cpu:
            pcpu, pouts = cpu_prefill_baseline(pc)
            secondary["C4_prefill"]["cpu_baseline"] = pcpu
            errors["C4"] = max_err_prefill(pc, pre["out"], pouts)
            secondary["C4_prefill"]["max_abs_err"] = errors["C4"]
            secondary["C4_prefill"]["parity_sample"] = "every row of every sequence, all heads"
            log(f"C4 prefill cpu baseline: {pcpu['value']} TFLOP/s; "
                f"max abs err {errors['C4']:.2e}")
            # the scalar entry point (paged_attention_prefill's fp32 row
            # kernel) on the same batch, against the same oracle outputs
            from heteroserve import _hip as _h
            sargs = (pc.q, pc.cu_seqlens, int(pc.q_lens.max()), pc.k_cache, pc.v_cache,
                     pc.block_tables, pc.context_lens, pc.scale, False)
            sout = _h.prefill_varlen(*sargs)
            serr = max_err_prefill(pc, sout, pouts)
            host_us, dev_us = _timed_calls(lambda: _h.prefill_varlen(*sargs), 5)
            secondary["C4_prefill_scalar"] = {
                "us_per_call": round(host_us, 2), "device_us_per_call": round(dev_us, 2),
                "tflops": round(pre["flops"] / (dev_us * 1e-6) / 1e12, 3),
                "max_abs_err": float(f"{serr:.3e}"),
                "path": "hs_prefill_varlen(use_mfma=0): the fp32 row kernel of "
                        "paged_attention_prefill"}
            errors["C4_scalar"] = serr
            log(f"C4 scalar prefill: {dev_us:.1f} us, err {serr:.2e}")
            del pouts, sout
        del pc, pre
        torch.cuda.empty_cache()

        mig = migration_legs(max(5, args.steps // 5), 2, with_cpu)
        secondary["C5_pack"] = mig["pack"]
        secondary["C5_unpack"] = mig["unpack"]
        secondary["copy_ceiling"] = mig["copy_ceiling"]
        exact["C5_pack"] = mig["pack"]["bit_exact"]
        exact["C5_unpack"] = mig["unpack"]["bit_exact"]

        kw = kv_write_leg(max(20, args.steps // 5), 10)
        secondary["C5_kv_write"] = {
            "us_per_step": round(kw["step_ms"] * 1e3, 2), "gbs": round(kw["kernel_gbs"], 1),
            "hbm_frac": round(kw["kernel_gbs"] / HBM_PEAK_GBS, 4), "bit_exact": kw["bit_exact"],
            "bytes_moved": kw["bytes"], "torch_index_put_us": round(kw["ref_ms"] * 1e3, 2),
        }
        exact["C5_kv_write"] = kw["bit_exact"]
        log(f"C5 KV write (1024-token chunk): {kw['kernel_ms'] * 1e3:.1f} us, "
            f"{kw['kernel_gbs']:.0f} GB/s, torch fk[slots]=k: {kw['ref_ms'] * 1e3:.1f} us, "
            f"exact={kw['bit_exact']}")
        tb = tables_leg(max(10, args.steps // 5))
        secondary["C5_tables"] = tb
        exact["C5_tables"] = tb["bit_exact"]
        log(f"C5 tables + slots + KV write (B=255): {tb['us_per_step']:.1f} us, reference torch "
            f"path {tb['reference_torch_us']:.1f} us, exact={tb['bit_exact']}")
        if with_cpu:
            rh = reference_harness_leg(with_cpu)
            secondary["reference_harness"] = rh
            for shape, r in rh.items():
                for label, row in list(r["rows"].items()) + list(
                        r.get("v3_split_sweep", {}).items()):
                    errors[f"{shape}: {label}"] = row["max_abs_err"]
            g1 = gqa_one_partition_leg()
            secondary["gqa_one_partition"] = g1
            for label, row in g1.items():
                errors[f"gqa_one_partition: {label}"] = row["max_abs_err"]
        st = c5_step_leg(max(10, args.steps // 5), 10, with_cpu)
        secondary["C5_step"] = st
        for part, key in (("prefill", "C5_step_prefill"), ("decode", "C5_step_decode")):
            if "max_abs_err" in st["parts"][part]:
                errors[key] = st["parts"][part]["max_abs_err"]
        log("C5 step: " + f"{st['us_per_step']:.1f} us = " + ", ".join(
            f"{k} {v['us']:.1f} us" for k, v in st["parts"].items())
            + f" (plain hs_decode: {st['decode_plain_us']:.1f} us)")

    ok = all(e <= TOL for e in errors.values()) and all(exact.values())
    line = {
        "metric": METRIC,
        "value": round(dec["step_gbs"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["step_ms"], 5),
        "us_per_step": round(dec["step_ms"] * 1e3, 2),
        "hbm_frac": round(dec["step_gbs"] / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,1) KV and queries, seeded block tables)",
        "config": config,
        "roofline": roofline(
            "hbm",
            LEG_KERNELS[args.config][0].replace("hs::", "") if args.config in LEG_KERNELS
            else "row_attn_part_kernel",
            dec["bytes"], dec["kernel_ms"],
            leg_traffic(args.config)
            if args.config in LEG_KERNELS and args.config != "C2-gqa" and not args.partition
            else None),
        "cpu_baseline": cpu,
        "max_abs_err": errors.get(headline_name),
        "parity": ("pass" if ok else "fail") if (errors or exact) else "not checked (--no-cpu)",
        "parity_tolerance": TOL,
        "parity_errors": {k: float(f"{v:.3e}") for k, v in errors.items()},
        "parity_exact": exact,
        "host": {"cpu": cpu_model(), "threads": host_threads()},
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    if not ok:
        log(f"parity check failed: errors {errors} (tolerance {TOL}), exact {exact}")
        return 1
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
