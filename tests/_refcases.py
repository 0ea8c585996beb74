"""Inputs of the reference test suite's paged cases, rebuilt without its allocator.

The reference builds its cases through TorchBlockAllocator
(tests/test_torch_engine.py:158-176, :496-515, test_model.py:106-124).  A fresh
allocator hands out block ids lowest-first (heteroserve/kv/blocks.py:83 keeps
the free list so that pop() returns the lowest id), and write_kv scatters
[L, H, T, D] K/V into [L, 2, NB, BS, H, D] (blocks.py:234-255).  This module
replays the same numpy RNG calls in the same order, so the inputs are the
reference tests' inputs bit for bit.

The "tiny" model of those tests (heteroserve/config.py:73-84) has 4 layers,
4 query heads and head_dim 64.
"""

from __future__ import annotations

import numpy as np

TINY_LAYERS, TINY_HEADS, TINY_DIM = 4, 4, 64


def lay_out(seqs, block_size: int, num_blocks: int, kv_heads: int, dtype, first_block=0):
    """Write per-sequence (k, v) [L, Hkv, n, D] into a fresh pool.

    Returns (pool [L, 2, NB, BS, Hkv, D], tables): sequence i takes the next
    ceil(n / BS) block ids in ascending order, as allocate() does on a fresh
    allocator with no prefix hits.
    """
    L = TINY_LAYERS if not seqs else seqs[0][0].shape[0]
    D = TINY_DIM if not seqs else seqs[0][0].shape[3]
    pool = np.zeros((L, 2, num_blocks, block_size, kv_heads, D), dtype=dtype)
    nxt = first_block
    tables = []
    for k, v in seqs:
        n = k.shape[2]
        need = -(-n // block_size)
        ids = list(range(nxt, nxt + need))
        nxt += need
        pos = np.arange(n)
        blk = np.asarray(ids, dtype=np.int64)[pos // block_size]
        off = pos % block_size
        pool[:, 0][:, blk, off] = k.transpose(0, 2, 1, 3)
        pool[:, 1][:, blk, off] = v.transpose(0, 2, 1, 3)
        tables.append(ids)
    return pool, tables


def table_array(tables, width=None) -> np.ndarray:
    width = width or max(len(t) for t in tables)
    bt = np.full((len(tables), width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t[:width]
    return bt


def build_paged_case(seed=5, lens=(9, 31, 16)):
    """tests/test_torch_engine.py:158-176: BS 8, 64 blocks, fp32 KV."""
    rng = np.random.default_rng(seed)
    seqs = []
    for n in lens:
        rng.integers(1, 4000, size=n)                       # prompt token ids
        k = rng.standard_normal((TINY_LAYERS, TINY_HEADS, n, TINY_DIM)).astype(np.float32)
        v = rng.standard_normal((TINY_LAYERS, TINY_HEADS, n, TINY_DIM)).astype(np.float32)
        seqs.append((k, v))
    q = rng.standard_normal((len(lens), TINY_HEADS, TINY_DIM)).astype(np.float32)
    pool, tables = lay_out(seqs, 8, 64, TINY_HEADS, np.float32)
    return dict(pool=pool, tables=tables, lens=list(lens), q=q, seqs=seqs,
                scale=1.0 / np.sqrt(TINY_DIM))


def prefill_case(lens, S, n_kv_head=None, seed=0):
    """tests/test_torch_engine.py:496-515: BS 16, 96 blocks, fp32 KV."""
    hkv = n_kv_head or TINY_HEADS
    rng = np.random.default_rng(seed)
    seqs = []
    for n in lens:
        rng.integers(1, 4000, size=n)
        k = rng.standard_normal((TINY_LAYERS, hkv, n, TINY_DIM)).astype(np.float32)
        v = rng.standard_normal((TINY_LAYERS, hkv, n, TINY_DIM)).astype(np.float32)
        seqs.append((k, v))
    q = rng.standard_normal((len(lens), S, TINY_HEADS, TINY_DIM)).astype(np.float32)
    pool, tables = lay_out(seqs, 16, 96, hkv, np.float32)
    return dict(pool=pool, tables=tables, lens=list(lens), q=q, seqs=seqs, S=S,
                scale=1.0 / np.sqrt(TINY_DIM))


def cpu_fuzz_trials(n_trials=40, seed=1234):
    """tests/test_torch_engine.py:359-402: random batches, BS in {4, 8, 16}."""
    rng = np.random.default_rng(seed)
    for trial in range(n_trials):
        n_seqs = int(rng.integers(1, 6))
        bs = int(rng.choice([4, 8, 16]))
        lens = [int(rng.integers(1, 200)) for _ in range(n_seqs)]
        need = sum(-(-n // bs) for n in lens) + 8
        seqs = []
        for n in lens:
            rng.integers(1, 4000, size=n)
            k = rng.standard_normal((TINY_LAYERS, TINY_HEADS, n, TINY_DIM)).astype(np.float32)
            v = rng.standard_normal((TINY_LAYERS, TINY_HEADS, n, TINY_DIM)).astype(np.float32)
            seqs.append((k, v))
        q = rng.standard_normal((n_seqs, TINY_HEADS, TINY_DIM)).astype(np.float32)
        pool, tables = lay_out(seqs, bs, max(16, need), TINY_HEADS, np.float32)
        yield dict(trial=trial, pool=pool, tables=tables, lens=lens, q=q, seqs=seqs, bs=bs,
                   scale=1.0 / np.sqrt(TINY_DIM))


def pack_case():
    """tests/test_model.py:106-124: BS 4, 16 blocks, fp16, one 16-token sequence."""
    k = np.random.default_rng(2).standard_normal(
        (TINY_LAYERS, TINY_HEADS, 16, TINY_DIM)).astype(np.float16)
    v = np.random.default_rng(3).standard_normal(
        (TINY_LAYERS, TINY_HEADS, 16, TINY_DIM)).astype(np.float16)
    pool, tables = lay_out([(k, v)], 4, 16, TINY_HEADS, np.float16)
    return dict(pool=pool, ids=tables[0], k=k, v=v)


WMMA_TILING_CASES = [  # tests/test_torch_engine.py:610-619 (ctx, S, D)
    (64, 32, 64), (64, 19, 64), (57, 16, 64), (91, 23, 64),
    (48, 48, 64), (80, 1, 64), (100, 40, 128), (512, 16, 64),
]

PREFILL_CASES = [  # tests/test_torch_engine.py:518-526 (lens, S, n_kv_head)
    ([64], 64, None), ([64], 16, None), ([37, 64, 19], 16, None),
    ([64], 32, 2), ([48], 48, 1), ([80], 1, None),
]

ONLINE_CASES = [(1, 1.0), (37, 1.0), (512, 1.0), (200, 25.0)]  # :257

SPLIT_CASES = [  # :327-335 (n, splits, amp)
    (37, 1, 1.0), (37, 4, 1.0), (512, 8, 1.0), (512, 32, 1.0),
    (5, 8, 1.0), (200, 7, 25.0), (1, 4, 1.0),
]


def single_head_case(ctx, S, D):
    """tests/test_torch_engine.py:631-635."""
    rng = np.random.default_rng(ctx * 31 + S)
    return (rng.standard_normal((S, D)), rng.standard_normal((ctx, D)),
            rng.standard_normal((ctx, D)))


def recurrence_case(seed, n, amp):
    """tests/test_torch_engine.py:266-271 and :346-351 (H 4, D 64)."""
    rng = np.random.default_rng(seed)
    q = (rng.standard_normal((4, 64)) * amp).astype(np.float32)
    k = (rng.standard_normal((n, 4, 64)) * amp).astype(np.float32)
    v = rng.standard_normal((n, 4, 64)).astype(np.float32)
    return q, k, v
