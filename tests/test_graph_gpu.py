"""The attention and pack calls under HIP graph capture.

Serving loops capture their decode step to cut launch overhead.  Nothing on
these paths allocates with hipMalloc, fills memory or synchronises with the
host, so the calls capture as they are (outputs and workspaces come from
torch's allocator, which serves a capture from the graph's pool).  Each graph
is replayed several times, with eager work and synchronisations between the
replays, and every replay must equal the eager result bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _capture(fn):
    """Warm up on a side stream (default priority), then capture fn()."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = fn()
    return graph, out


def _replays_match(graph, outs, wants, n=3):
    for i in range(n):
        for o in outs:
            o.fill_(float("nan") if o.is_floating_point() else -1)   # eager work between
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for o, w in zip(outs, wants):
            assert torch.equal(o, w), f"replay {i}"


def test_decode_prefill_and_pack_replay_bit_exact():
    from heteroserve import _hip
    from heteroserve.model import paged_attn, paged_attn_wmma
    from hsbench.cases import build_decode, build_prefill

    assert _hip.ready(), _hip.error()
    dec = build_decode("g", np.array([1, 300, 1100, 4000, 17]), 8, 8, 128, 800,
                       torch.bfloat16, DEV, seed=12)
    dec_args = (dec.q, dec.k_cache, dec.v_cache, dec.block_tables, dec.context_lens, dec.scale)
    # grouped-query decode of a bf16 and of an fp16 cache: the split-operand
    # matrix-core kernel (with its power-of-two query scaling for fp16)
    gqa = build_decode("g", np.array([5, 700, 2500, 16]), 32, 8, 128, 300,
                       torch.bfloat16, DEV, seed=14)
    gqa_args = (gqa.q, gqa.k_cache, gqa.v_cache, gqa.block_tables, gqa.context_lens, gqa.scale)
    g16 = build_decode("g", np.array([900, 3, 1800]), 16, 8, 64, 200, torch.float16, DEV,
                       seed=15)
    g16_args = (g16.q, g16.k_cache, g16.v_cache, g16.block_tables, g16.context_lens, g16.scale)
    # a single chunk: a small grid, so the MFMA prefill splits the key range
    # and runs its merge kernel too
    pre = build_prefill("g", np.array([700]), np.array([300]), 8, 8, 128, 80,
                        torch.bfloat16, DEV, seed=13)
    q4 = pre.q.unsqueeze(0)
    pre_args = (q4, pre.k_cache, pre.v_cache, pre.block_tables, pre.context_lens, pre.scale)
    pool = dec.pool
    ids = torch.tensor([5, 0, 799, 42, 42, 7], dtype=torch.int64, device=DEV)
    packed = torch.empty((ids.numel(),) + tuple(pool.shape[:2]) + tuple(pool.shape[3:]),
                         dtype=pool.dtype, device=DEV)

    want_dec = paged_attn.paged_attention(*dec_args)
    want_gqa = paged_attn.paged_attention(*gqa_args)
    want_g16 = paged_attn.paged_attention(*g16_args)
    want_pre = paged_attn_wmma.paged_attention_prefill_wmma(*pre_args)
    _hip.kv_pack(pool, ids, packed)
    want_pack = packed.clone()
    torch.cuda.synchronize()

    def step():
        d = paged_attn.paged_attention(*dec_args)
        g = paged_attn.paged_attention(*gqa_args)
        h = paged_attn.paged_attention(*g16_args)
        p = paged_attn_wmma.paged_attention_prefill_wmma(*pre_args)
        _hip.kv_pack(pool, ids, packed)
        return d, g, h, p

    graph, (d, g, h, p) = _capture(step)
    _replays_match(graph, [d, g, h, p, packed],
                   [want_dec, want_gqa, want_g16, want_pre, want_pack])


@pytest.mark.parametrize("Hkv", [8, 32])
def test_even_split_decode_replays_bit_exact(Hkv):
    """The decode's even split (4 query heads per KV head on the matrix
    cores, or plain multi-head attention on the VALU walk; a batch whose
    fixed partitions would overflow one round of the device): the even-split
    kernel and its merge, captured and replayed bit for bit, and equal to
    the oracle-checked eager call."""
    from heteroserve import _hip
    from heteroserve.model import paged_attn
    from hsbench.cases import build_decode

    assert _hip.ready(), _hip.error()
    lens = np.random.default_rng(31).integers(64, 4000, 64)
    need = int(sum(-(-int(n) // 16) for n in lens))
    case = build_decode("e", lens, 32, Hkv, 128, need + 64, torch.bfloat16, DEV, seed=31)
    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens, case.scale)
    want = paged_attn.paged_attention(*args)
    fixed = _hip.decode(*args, 0, partition_tokens=768)
    assert (want - fixed).abs().max().item() <= 5e-5   # agrees with the fixed partitions
    torch.cuda.synchronize()
    graph, out = _capture(lambda: paged_attn.paged_attention(*args))
    _replays_match(graph, [out], [want])
