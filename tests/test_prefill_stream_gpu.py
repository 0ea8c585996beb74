"""GPU parity of the persistent MFMA prefill (prefill_stream_kernel).

Large grids of 256-row query tiles (two or more per CU, whole XCDs of heads)
run one workgroup per CU that takes query tiles from a per-XCD queue and
streams the K/V tiles of consecutive ones.  Its per-tile arithmetic is the
grid kernel's, so on every shape here its output must equal the grid
kernel's bit for bit (HETEROSERVE_PREFILL_GRID=1 forces the grid kernel),
and both must match the oracle (paged_attention_prefill_torch semantics,
heteroserve/model/paged_attn_prefill.py:281-322) within the north-star 2e-3.

The persistent path is the one the library plans when
hs_prefill_workspace_bytes asks for its 256-byte queue workspace; each test
checks that it does, so a change of plan cannot turn these into grid tests.
"""

from __future__ import annotations

import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from hsbench import cases  # noqa: E402
from oracle.attention import prefill_one  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
STREAM_WS = 256   # the queue workspace of the persistent plan


def _case(prefix, chunk, H, Hkv, D, dtype, seed, cut=None):
    prefix = np.asarray(prefix)
    chunk = np.asarray(chunk)
    need = int(sum(-(-int(p + s) // 16) for p, s in zip(prefix, chunk)))
    case = cases.build_prefill("stream", prefix, chunk, H, Hkv, D, 2 * need + 16, dtype, DEV,
                               seed)
    if cut is not None:   # shorter contexts: leading rows at negative positions are zero
        ctx = np.maximum(case.ctx - np.asarray(cut), 0)
        case.ctx = ctx
        case.context_lens = torch.from_numpy(ctx.astype(np.int32)).to(DEV)
    return case


def _run(case, grid: bool):
    from heteroserve import _hip

    old = os.environ.get("HETEROSERVE_PREFILL_GRID")
    os.environ["HETEROSERVE_PREFILL_GRID"] = "1" if grid else "0"
    try:
        out = _hip.prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()),
                                  case.k_cache, case.v_cache, case.block_tables,
                                  case.context_lens, case.scale, use_mfma=True)
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["HETEROSERVE_PREFILL_GRID"]
        else:
            os.environ["HETEROSERVE_PREFILL_GRID"] = old
    return out


def _plans_stream(case) -> bool:
    from heteroserve import _hip

    T, H, D = case.q.shape
    B = case.block_tables.shape[0]
    os.environ.pop("HETEROSERVE_PREFILL_GRID", None)
    return _hip.lib().hs_prefill_workspace_bytes(B, int(case.q_lens.max()), H, D, 1) == STREAM_WS


def _oracle_err(case, out, seqs) -> float:
    cu = case.cu_seqlens.cpu().numpy()
    kc, vc = case.k_cache.cpu(), case.v_cache.cpu()
    err = 0.0
    for b in seqs:
        want = prefill_one(case.q[cu[b]:cu[b + 1]].cpu(), kc, vc, case.block_tables[b].cpu(),
                           int(case.ctx[b]), case.scale)
        err = max(err, (out[cu[b]:cu[b + 1]].cpu() - want).abs().max().item())
    return err


SHAPES = {
    # D 64, fp16 cache
    "d64-f16": dict(prefix=[1046, 23, 711, 1499, 380, 0, 951, 402, 1200, 77, 640, 1333, 5,
                            888, 260, 999],
                    chunk=[512, 833, 200, 650, 399, 256, 700, 431, 612, 257, 300, 880, 201,
                           555, 640, 777],
                    H=32, Hkv=32, D=64, dtype=torch.float16, seed=1),
    # grouped-query heads (4 query heads per KV head), bf16
    "gqa": dict(prefix=[1800, 0, 640, 1200, 333, 1999, 64, 900, 1500, 10, 700, 1111],
                chunk=[1400, 300, 1024, 555, 1499, 301, 900, 777, 640, 1300, 256, 999],
                H=16, Hkv=4, D=128, dtype=torch.bfloat16, seed=2),
    # one long chunk: 32 query tiles per head
    "one-long": dict(prefix=[1000], chunk=[8000], H=32, Hkv=32, D=128, dtype=torch.bfloat16,
                     seed=3),
    # contexts shorter than the chunk: rows at negative positions (zero), some
    # query tiles without any key (items with no tiles in the stream)
    "negative-rows": dict(prefix=[0] * 16, chunk=[600] * 16, H=32, Hkv=32, D=128,
                          dtype=torch.bfloat16, seed=5,
                          cut=[0, 100, 300, 600, 700, 0, 256, 257, 512, 599, 1, 0, 0, 0, 0,
                               600]),
    # many query tiles of 1..7 key tiles: the stream reaches the end of the
    # published items and restarts
    "tiny-items": dict(prefix=[3, 90, 0, 41, 77, 12, 60, 99, 5, 31, 88, 2, 70, 15, 46, 0, 81,
                               23, 54, 9, 66, 37, 94, 18, 72, 1, 49, 85, 28, 63, 11, 97, 44,
                               20, 58, 6, 79, 33, 91, 26],
                       chunk=[1, 299, 17, 150, 256, 257, 64, 200, 33, 128, 90, 275, 5, 180,
                              222, 48, 111, 300, 7, 160, 245, 70, 19, 290, 135, 240, 56, 12,
                              201, 99, 260, 150, 38, 177, 288, 3, 120, 215, 66, 254],
                       H=32, Hkv=8, D=128, dtype=torch.bfloat16, seed=4),
    # 64 heads (8 per XCD), 8 query heads per KV head, fp16 cache at head dim 128
    "h64-f16": dict(prefix=[700, 2900, 0, 1500, 64, 333, 2048, 10],
                    chunk=[900, 300, 1100, 257, 640, 1000, 128, 700],
                    H=64, Hkv=8, D=128, dtype=torch.float16, seed=7),
    # 200 sequences (near the 256 the ranking holds), short chunks, head dim 64
    "many-seqs": dict(prefix=[int(x) for x in np.random.default_rng(8).integers(0, 3000, 200)],
                      chunk=[int(x) for x in np.random.default_rng(9).integers(1, 600, 200)],
                      H=16, Hkv=16, D=64, dtype=torch.bfloat16, seed=8),
}


@pytest.mark.parametrize("name", list(SHAPES))
def test_stream_equals_grid_and_oracle(name):
    kw = dict(SHAPES[name])
    case = _case(**kw)
    assert _plans_stream(case), "shape no longer planned for the persistent kernel"
    grid = _run(case, grid=True)
    got = _run(case, grid=False)
    assert torch.isfinite(got).all()
    assert torch.equal(got, grid), f"{name}: persistent and grid kernels differ"
    B = case.block_tables.shape[0]
    seqs = range(B) if B <= 16 else range(0, B, 3)
    err = _oracle_err(case, got, seqs)
    assert err <= 2e-3, f"{name}: max abs err {err:.2e}"


def test_stream_c4_equals_grid():
    """The C4 configuration itself (the benchmark's prefill leg); its oracle
    check over every row is test_prefill_gpu.py::test_prefill_configs."""
    case = cases.c4_prefill(DEV)
    assert _plans_stream(case)
    assert torch.equal(_run(case, grid=False), _run(case, grid=True))


def test_stream_range_fallback():
    """A bf16 K value fp16 cannot hold (1e6) in one sequence's first page.
    The workgroup that meets it leaves the matrix-core loop and computes that
    query tile and its remaining ones in fp32 (the grid kernel falls back per
    query tile instead, so only the oracle is compared)."""
    case = _case(prefix=[1046, 23, 711, 1499, 380, 0, 951, 402, 1200, 77, 640, 1333, 5, 888,
                         260, 999],
                 chunk=[512, 833, 200, 650, 399, 256, 700, 431, 612, 257, 300, 880, 201, 555,
                        640, 777],
                 H=32, Hkv=32, D=128, dtype=torch.bfloat16, seed=6)
    blk = int(case.block_tables[3, 0])
    case.pool[0, 0, blk, 5, 7, 11] = 1.0e6
    assert _plans_stream(case)
    got = _run(case, grid=False)
    assert torch.isfinite(got).all()
    err = _oracle_err(case, got, range(case.block_tables.shape[0]))
    assert err <= 2e-3, f"max abs err {err:.2e}"


def test_stream_workspace_must_hold_the_queue():
    """A workspace smaller than the queue's 256 bytes is refused before any
    launch (HS_EWORKSPACE), like a split whose partials do not fit."""
    from heteroserve import _hip

    case = cases.c4_prefill(DEV)
    T, H, D = case.q.shape
    kc = case.k_cache
    NB, BS, Hkv, _ = kc.shape
    B, MB = case.block_tables.shape
    ws = torch.empty(64, dtype=torch.uint8, device=DEV)
    out = torch.zeros((T, H, D), device=DEV)
    lib = _hip.lib()
    os.environ.pop("HETEROSERVE_PREFILL_GRID", None)
    rc = lib.hs_prefill_varlen(case.q.data_ptr(), case.cu_seqlens.data_ptr(),
                               int(case.q_lens.max()), kc.data_ptr(), case.v_cache.data_ptr(),
                               _hip.dtype_code(kc.dtype), NB, case.block_tables.data_ptr(),
                               case.context_lens.data_ptr(), out.data_ptr(), B, H, Hkv, D, BS, MB,
                               float(case.scale), 1, ws.data_ptr(), 64,
                               torch.cuda.current_stream().cuda_stream)
    assert rc == -4
    assert b"workspace" in lib.hs_last_error()
    torch.cuda.synchronize()
    assert not out.any()


def test_stream_under_graph_capture():
    """The persistent prefill captured in a HIP graph: its queue reset is a
    kernel (no memset node), so each replay starts from zeroed counters.
    Three replays, with eager work between them, equal the eager call bit for
    bit."""
    case = _case(**SHAPES["gqa"])
    assert _plans_stream(case)
    want = _run(case, grid=False)

    from heteroserve import _hip

    def call():
        return _hip.prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()),
                                   case.k_cache, case.v_cache, case.block_tables,
                                   case.context_lens, case.scale, use_mfma=True)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for i in range(3):
        out.fill_(float("nan"))
        _run(case, grid=True)   # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"
