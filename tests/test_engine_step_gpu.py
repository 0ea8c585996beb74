"""The engine's calling pattern: write the step's new K/V into the paged pool,
then attend over it.

hetero-serve's engine does, per layer and step:

* decode (heteroserve/model/torch_engine.py:215-245): the slot of each
  sequence's new token at position ctx_b through its own block table
  (slots_for), ``fk[slots] = k.to(dtype)`` for K and V, then
  ``paged_attention(q, pool[l, 0], pool[l, 1], tables, ctx + 1, scale)``;
* prefill (torch_engine.py:294-313): the chunk's slots at positions
  start .. start + T - 1, the same write, then the WMMA prefill (or the
  scalar one when ``supports`` says no) with B = 1 and ctx = start + T.

The reference checks that sequence end to end against its gather path
(tests/test_torch_engine.py:221-249).  Here the same sequence runs through
this library (hs_kv_append for the write, then the attention entry points),
several steps in a row on one pool, and each step is compared with the
oracle applied to a host copy of the pool that the reference's own write
(``oracle/kvpack.py`` scatter_rows: ``cache[slots] = rows.to(dtype)``) keeps
up to date.  The device pool must equal that host pool bit for bit after
every write, and the attention output must match the oracle on it.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle.kvpack as kvp  # noqa: E402
from oracle.attention import paged_attention_prefill_torch, paged_attention_torch  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BS = 16


def _mods():
    from heteroserve.kv import pack
    from heteroserve.model import paged_attn, paged_attn_prefill, paged_attn_wmma

    assert paged_attn.which_backend() == "cuda", paged_attn.build_error()
    return pack, paged_attn, paged_attn_prefill, paged_attn_wmma


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _table_tensor(tables):
    return kvp.block_table_tensor(tables)


class Pool:
    """A two-layer pool on the GPU and its host mirror; writes go to the
    device through the library and to the host through the reference's
    expression."""

    def __init__(self, nb, hkv, d, dtype, seed):
        g = torch.Generator().manual_seed(seed)
        # garbage everywhere: a slot the engine has not written must never be read
        host = (torch.randn(2, 2, nb, BS, hkv, d, generator=g) * 4).to(dtype)
        self.host = host
        self.dev = host.to(DEV)
        self.layer = 1    # the engine passes pool[l, 0] / pool[l, 1] views

    def views(self):
        return self.dev[self.layer, 0], self.dev[self.layer, 1]

    def host_views(self):
        return self.host[self.layer, 0], self.host[self.layer, 1]

    def write(self, pack, tables_dev, tables, positions, seq_ids, k, v):
        """k, v: [n, Hkv, D] fp32 device rows (slices of one fused QKV tensor)."""
        kc, vc = self.views()
        pack.append_kv(kc, vc, tables_dev,
                       torch.as_tensor(positions, dtype=torch.int32, device=DEV), k, v,
                       seq_ids=None if seq_ids is None else
                       torch.as_tensor(seq_ids, dtype=torch.int32, device=DEV))
        hk, hv = self.host_views()
        sids = range(len(positions)) if seq_ids is None else seq_ids
        slots = np.array([int(kvp.slots_for(tables[s], [p], BS)[0])
                          for s, p in zip(sids, positions)], dtype=np.int64)
        kvp.scatter_rows(hk, slots, k.cpu())
        kvp.scatter_rows(hv, slots, v.cpu())

    def assert_synced(self):
        torch.cuda.synchronize()
        assert torch.equal(_bits(self.dev.cpu()), _bits(self.host)), "pool differs from the host"


def _qkv(n, h, hkv, d, gen):
    """One fused QKV projection output [n, (H + 2 Hkv) * D] and its q, k, v
    views, as torch_engine.py:230-235 slices them."""
    e, kvd = h * d, hkv * d
    qkv = torch.randn(n, e + 2 * kvd, generator=gen).to(DEV)
    return (qkv[:, :e].view(n, h, d), qkv[:, e:e + kvd].view(n, hkv, d),
            qkv[:, e + kvd:].view(n, hkv, d))


@pytest.mark.parametrize("H,Hkv,D,dtype", [
    (8, 8, 128, torch.bfloat16),     # MHA, the VALU decode
    (8, 2, 128, torch.bfloat16),     # 4 query heads per KV head: matrix-core decode
    (12, 12, 64, torch.float16),     # the reference benchmark's GPT-2 geometry
    (16, 2, 64, torch.float16),      # 8 query heads per KV head
])
def test_decode_steps_write_then_attend(H, Hkv, D, dtype):
    """Four decode steps of a ragged batch: before each, sequence b holds n_b
    tokens; its new token goes to position n_b (crossing into a fresh page
    for n_b % 16 == 0), then attention runs with context n_b + 1.  Lengths
    include one-token and page-boundary cases and a row past one default
    partition."""
    pack, m1, _, _ = _mods()
    lens = [1, 15, 16, 31, 100, 700, 1300]
    steps = 4
    nb = 4 * sum(-(-(n + steps) // BS) for n in lens)
    pool = Pool(nb, Hkv, D, dtype, seed=71)
    rng = np.random.default_rng(72)
    perm = rng.permutation(nb).tolist()
    tables, start = [], 0
    for n in lens:   # the allocator reserves the steps' pages up front
        need = -(-(n + steps) // BS)
        tables.append(perm[start:start + need])
        start += need
    bt = _table_tensor(tables).to(DEV)
    gen = torch.Generator().manual_seed(73)
    # the cached past of every sequence, written as one prefill would
    for b, n in enumerate(lens):
        _, k, v = _qkv(n, H, Hkv, D, gen)
        pool.write(pack, bt, tables, list(range(n)), [b] * n, k, v)
    pool.assert_synced()
    scale = 1.0 / math.sqrt(D)
    n_now = list(lens)
    for step in range(steps):
        q, k, v = _qkv(len(lens), H, Hkv, D, gen)
        pool.write(pack, bt, tables, n_now, None, k, v)          # fk[slots] = k
        pool.assert_synced()
        ctx = torch.tensor([n + 1 for n in n_now], dtype=torch.int32, device=DEV)
        kc, vc = pool.views()
        got = m1.paged_attention(q, kc, vc, bt, ctx, scale)
        hk, hv = pool.host_views()
        want = paged_attention_torch(q.cpu(), hk, hv, bt.cpu(), ctx.cpu(), scale)
        err = (got.cpu() - want).abs().max().item()
        assert err <= 1e-4, (step, err)
        n_now = [n + 1 for n in n_now]


@pytest.mark.parametrize("D,dtype", [(128, torch.bfloat16), (64, torch.float16)])
def test_chunked_prefill_then_decode(D, dtype):
    """One sequence through the engine's prefill path chunk by chunk (each
    chunk written, then attended with B = 1 and ctx = start + T, on the
    matrix cores and on the scalar kernel), then two decode steps on the
    same pool.  Chunks of 1, 50, 300 and 37 tokens: a one-row chunk, chunks
    that start and end mid-page, one longer than a 256-row query tile."""
    pack, m1, mpf, mw = _mods()
    H, Hkv = 8, 4
    assert mw.supports(BS, D, dtype)
    chunks = [1, 50, 300, 37]
    total = sum(chunks) + 2
    nb = 3 * -(-total // BS)
    pool = Pool(nb, Hkv, D, dtype, seed=81)
    table = np.random.default_rng(82).permutation(nb)[: -(-total // BS)].tolist()
    bt = _table_tensor([table]).to(DEV)
    gen = torch.Generator().manual_seed(83)
    scale = 1.0 / math.sqrt(D)
    start = 0
    for T in chunks:
        q, k, v = _qkv(T, H, Hkv, D, gen)
        pool.write(pack, bt, [table], list(range(start, start + T)), [0] * T, k, v)
        pool.assert_synced()
        ctx = torch.tensor([start + T], dtype=torch.int32, device=DEV)
        kc, vc = pool.views()
        qb = q.reshape(1, T, H, D)
        hk, hv = pool.host_views()
        want = paged_attention_prefill_torch(qb.cpu(), hk, hv, bt.cpu(), ctx.cpu(), scale)
        got_mfma = mw.paged_attention_prefill_wmma(qb, kc, vc, bt, ctx, scale)
        got_scalar = mpf.paged_attention_prefill(qb, kc, vc, bt, ctx, scale)
        assert (got_mfma.cpu() - want).abs().max().item() <= 2e-3, T
        assert (got_scalar.cpu() - want).abs().max().item() <= 1e-3, T
        start += T
    for _ in range(2):
        q, k, v = _qkv(1, H, Hkv, D, gen)
        pool.write(pack, bt, [table], [start], None, k, v)
        pool.assert_synced()
        ctx = torch.tensor([start + 1], dtype=torch.int32, device=DEV)
        kc, vc = pool.views()
        got = m1.paged_attention(q, kc, vc, bt, ctx, scale)
        hk, hv = pool.host_views()
        want = paged_attention_torch(q.cpu(), hk, hv, bt.cpu(), ctx.cpu(), scale)
        assert (got.cpu() - want).abs().max().item() <= 1e-4
        start += 1
