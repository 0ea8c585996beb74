"""GPU parity of writing new K/V rows into the paged cache, and of building
the block-table tensor the kernels walk.

hs_kv_scatter / hs_kv_append against the oracle's restatement of the
engine's ``fk[slots] = k.to(dtype)`` (torch_engine.py:239-240, :306-308) and
of TorchBlockAllocator.write_kv (torch_blocks.py:89-106): bit-exact for every
non-NaN value (torch's own NaN encodings differ between its code paths, so a
NaN only has to stay NaN), untouched slots unchanged.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle.kvpack as kvp  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DTYPES = [torch.float32, torch.float16, torch.bfloat16]
BITS = {torch.float32: torch.int32, torch.float16: torch.int16, torch.bfloat16: torch.int16}


def _pack():
    from heteroserve import _hip
    from heteroserve.kv import pack

    assert _hip.ready(), _hip.error()
    return pack


def _assert_same(got, want):
    """Bitwise equality, except that NaN only has to match NaN."""
    got, want = got.detach().cpu(), want.detach().cpu()
    assert got.dtype == want.dtype and got.shape == want.shape
    nan = torch.isnan(want.float())
    assert torch.equal(torch.isnan(got.float()), nan)
    g = got.view(BITS[got.dtype])[~nan]
    w = want.view(BITS[want.dtype])[~nan]
    bad = (g != w).nonzero()
    assert bad.numel() == 0, f"{bad.shape[0]} elements differ, first at {bad[:3].tolist()}"


def _rows(n, h, d, dtype, seed, special=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(n, h, d, generator=g) * 3
    if special and n > 1:
        x[0, 0, :8] = torch.tensor([float("nan"), float("inf"), -float("inf"), 65520.0, 65519.0,
                                    1e-8, -3e-5, 1.0 + 2 ** -8])
        x[1, 0, 0] = -0.0
    return x.to(dtype)


@pytest.mark.parametrize("cache_dt", DTYPES)
@pytest.mark.parametrize("src_dt", DTYPES)
def test_scatter_matches_oracle(src_dt, cache_dt):
    """Every source/cache dtype pair, random distinct slots, one launch."""
    pk = _pack()
    nb, bs, h, d = 37, 16, 4, 64
    rng = np.random.default_rng(7)
    cache_k = torch.randn(nb, bs, h, d, generator=torch.Generator().manual_seed(1)).to(cache_dt)
    cache_v = torch.randn(nb, bs, h, d, generator=torch.Generator().manual_seed(2)).to(cache_dt)
    k = _rows(45, h, d, src_dt, 3)
    v = _rows(45, h, d, src_dt, 4)
    slots = rng.permutation(nb * bs)[:45]
    want_k, want_v = cache_k.clone(), cache_v.clone()
    kvp.scatter_rows(want_k, slots, k)
    kvp.scatter_rows(want_v, slots, v)
    gk, gv = cache_k.to(DEV), cache_v.to(DEV)
    pk.scatter_kv(gk, gv, torch.as_tensor(slots, device=DEV), k.to(DEV), v.to(DEV))
    _assert_same(gk, want_k)
    _assert_same(gv, want_v)


@pytest.mark.parametrize("extra", [0, 3, 8])
def test_scatter_from_strided_qkv_rows(extra):
    """K and V as slices of the fused QKV output (torch_engine.py:233-235):
    row stride 3 * Hkv * D (+ extra columns); `extra = 3` gives rows that are
    not 16-byte aligned and takes the element-wise kernel."""
    pk = _pack()
    nb, bs, h, d = 20, 16, 2, 32
    kvd = h * d
    qkv = torch.randn(24, 3 * kvd + extra, generator=torch.Generator().manual_seed(9))
    k = qkv[:, kvd:2 * kvd].view(24, h, d)
    v = qkv[:, 2 * kvd:3 * kvd].view(24, h, d)
    slots = torch.arange(24) * 7 % (nb * bs)
    want_k = torch.zeros(nb, bs, h, d, dtype=torch.bfloat16)
    want_v = torch.zeros_like(want_k)
    kvp.scatter_rows(want_k, slots, k)
    kvp.scatter_rows(want_v, slots, v)
    gk, gv = torch.zeros_like(want_k, device=DEV), torch.zeros_like(want_v, device=DEV)
    q_dev = qkv.to(DEV)
    pk.scatter_kv(gk, gv, slots.to(DEV), q_dev[:, kvd:2 * kvd].view(24, h, d),
                  q_dev[:, 2 * kvd:3 * kvd].view(24, h, d))
    _assert_same(gk, want_k)
    _assert_same(gv, want_v)


def test_append_decode_step():
    """One new token per sequence at position ctx_b (torch_engine.py:215-240):
    slots from the block tables on the GPU equal slots_for's."""
    pk = _pack()
    rng = np.random.default_rng(11)
    nb, bs, h, d, B = 64, 16, 4, 128, 9
    ids = rng.permutation(nb)
    tables, pos, start = [], [], 0
    for b in range(B):
        need = int(rng.integers(1, 6))
        tables.append(ids[start:start + need].tolist())
        start += need
        pos.append(int(rng.integers(0, need * bs)))
    MB = max(len(t) for t in tables)
    bt = torch.full((B, MB), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.as_tensor(t)
    k = _rows(B, h, d, torch.float32, 12, special=False)
    v = _rows(B, h, d, torch.float32, 13, special=False)
    want_k = torch.zeros(nb, bs, h, d, dtype=torch.bfloat16)
    want_v = torch.zeros_like(want_k)
    slots = [int(kvp.slots_for(tables[b], [pos[b]], bs)[0]) for b in range(B)]
    kvp.scatter_rows(want_k, slots, k)
    kvp.scatter_rows(want_v, slots, v)
    gk, gv = torch.zeros_like(want_k, device=DEV), torch.zeros_like(want_v, device=DEV)
    pk.append_kv(gk, gv, bt.to(DEV), torch.tensor(pos, dtype=torch.int32, device=DEV),
                 k.to(DEV), v.to(DEV))
    _assert_same(gk, want_k)
    _assert_same(gv, want_v)


def test_append_prefill_chunk_and_invalid_rows():
    """A chunk of T tokens of one sequence (seq_ids all 0, positions
    start .. start+T-1, torch_engine.py:294-308); rows past the table or on a
    padding entry are not written."""
    pk = _pack()
    nb, bs, h, d = 32, 16, 2, 64
    table = [7, 30, 2, 19, -1]
    start, T = 5, 40                       # positions 5..44 use blocks 0..2
    bt = torch.tensor([table], dtype=torch.int32)
    pos = torch.arange(start, start + T, dtype=torch.int32)
    pos_bad = torch.cat([pos, torch.tensor([70, 100, -1], dtype=torch.int32)])  # pad, past, negative
    k = _rows(T + 3, h, d, torch.float16, 21)
    v = _rows(T + 3, h, d, torch.float16, 22)
    want_k = torch.zeros(nb, bs, h, d, dtype=torch.float16)
    want_v = torch.zeros_like(want_k)
    slots = kvp.slots_for(table[:3], range(start, start + T), bs)
    kvp.scatter_rows(want_k, slots, k[:T])
    kvp.scatter_rows(want_v, slots, v[:T])
    gk, gv = torch.zeros_like(want_k, device=DEV), torch.zeros_like(want_v, device=DEV)
    pk.append_kv(gk, gv, bt.to(DEV), pos_bad.to(DEV), k.to(DEV), v.to(DEV),
                 seq_ids=torch.zeros(T + 3, dtype=torch.int32, device=DEV))
    _assert_same(gk, want_k)
    _assert_same(gv, want_v)


def test_append_skips_sequence_ids_outside_the_tables():
    """Rows whose sequence id is negative or >= the number of table rows are
    skipped: the kernel reads no table row past B (here the row after the
    table's last holds a valid block id in the same allocation, which a
    missing bound would follow) and the cache is bit-identical apart from
    the valid rows."""
    pk = _pack()
    nb, bs, h, d = 16, 16, 2, 64
    big = torch.tensor([[3, 5], [8, 1], [11, 12]], dtype=torch.int32, device=DEV)
    bt = big[:2]                                   # B = 2 tables; row 2 lies beyond
    k = _rows(5, h, d, torch.float32, 40, special=False)
    v = _rows(5, h, d, torch.float32, 41, special=False)
    seq = torch.tensor([0, 2, 1, -1, 7], dtype=torch.int32, device=DEV)
    pos = torch.tensor([3, 4, 20, 1, 0], dtype=torch.int32, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(42)
    gk = torch.randn(nb, bs, h, d, generator=gen, device=DEV).to(torch.bfloat16)
    gv = torch.randn(nb, bs, h, d, generator=gen, device=DEV).to(torch.bfloat16)
    want_k, want_v = gk.cpu().clone(), gv.cpu().clone()
    slots = [int(kvp.slots_for([3, 5], [3], bs)[0]), int(kvp.slots_for([8, 1], [20], bs)[0])]
    kvp.scatter_rows(want_k, slots, k[[0, 2]])
    kvp.scatter_rows(want_v, slots, v[[0, 2]])
    pk.append_kv(gk, gv, bt, pos, k.to(DEV), v.to(DEV), seq_ids=seq)
    _assert_same(gk, want_k)
    _assert_same(gv, want_v)


def test_write_kv_matches_reference_allocator():
    """HipKVMixin.write_kv == TorchBlockAllocator.write_kv (torch_blocks.py:
    89-106) for the tiny model's shape, then read back by the GPU gather."""
    pk = _pack()
    L, nb, bs, h, d = 4, 24, 16, 4, 64
    table = [17, 3, 9, 21]
    k = torch.randn(L, h, 50, d, generator=torch.Generator().manual_seed(30))
    v = torch.randn(L, h, 50, d, generator=torch.Generator().manual_seed(31))
    want = torch.zeros(L, 2, nb, bs, h, d, dtype=torch.float16)
    kvp.write_kv(want, table, 7, k, v)
    pool = torch.zeros_like(want, device=DEV)
    pk.write_kv(pool, table, 7, k.to(DEV), v.to(DEV))
    _assert_same(pool, want)
    gk, gv = pk.gather_kv_batch(pool, [table], 57, layer=2)
    assert torch.equal(gk[0, 7:].cpu(), k[2].permute(1, 0, 2).to(torch.float16))


def test_host_slots_are_checked_and_empty_writes_are_noops():
    pk = _pack()
    gk = torch.zeros(4, 16, 2, 32, dtype=torch.bfloat16, device=DEV)
    gv = torch.zeros_like(gk)
    rows = torch.ones(2, 2, 32, device=DEV)
    with pytest.raises(IndexError):
        pk.scatter_kv(gk, gv, [3, 64], rows, rows)
    pk.scatter_kv(gk, gv, [-1, 0], rows, rows)          # torch indexing: -1 is the last slot
    assert gk.view(-1, 2, 32)[63].float().eq(1).all() and gk.view(-1, 2, 32)[0].float().eq(1).all()
    pk.scatter_kv(gk, gv, torch.empty(0, dtype=torch.long), rows[:0], rows[:0])
    with pytest.raises(RuntimeError):
        pk.scatter_kv(gk, gv, [1, 2], torch.ones(2, 3, 32, device=DEV), rows)


def test_block_table_tensor_matches_reference():
    """block_table_tensor (torch_blocks.py:75-85) built on the GPU from one
    upload: C5's 255 sequences, explicit widths (padding and truncation) and
    empty tables, equal to the reference's loop of per-sequence copies."""
    pk = _pack()
    rng = np.random.default_rng(50)
    tables = [rng.permutation(65536)[: int(n)].tolist() for n in rng.integers(16, 257, size=255)]
    tables[3] = []
    for pad_to in (None, 300, 100):
        got = pk.block_table_tensor(tables, pad_to, DEV)
        want = kvp.block_table_tensor(tables, pad_to)
        assert torch.equal(got.cpu(), want)
    for tbl in ([], [[], []], [[5]], [[1, 2], [3]]):
        assert torch.equal(pk.block_table_tensor(tbl, None, DEV).cpu(), kvp.block_table_tensor(tbl))
