"""Seeded synthetic inputs for the five benchmark configurations (C1..C5).

The configurations are the reference path's headline workloads, restated:

  C1  decode, B 8, 12 heads, D 64, fp16 KV, ctx U[16, 512], 1024-block pool;
      Q/K/V ~ N(0, 1) / sqrt(D)
  C2  ragged decode, B 64, 32 heads, D 128, bf16, ctx lognormal(median 2048,
      sigma 0.8) clipped to [64, 8192], 65536-block pool
  C2-gqa  C2's batch at Llama-3-8B's geometry: 32 query heads on 8 KV heads
  C3  long-context decode, B 16, 32 heads, D 128, bf16, ctx U[8192, 32768]
  B64-4k  the north-star decode target's shape: C2's geometry with every one
      of the 64 sequences at a 4096-token context
  C4  chunked causal prefill, 8 sequences with a cached prefix U[0, 4096] and a
      new chunk U[128, 2048], 32 heads, D 128, bf16
  C5  mixed step: a 1024-token chunk on a 2048-token prefix, 255 decode
      sequences with ctx U[256, 4096] of which half share a 1024-token prefix
      (identical block-table entries), and a pack of 4096 random blocks

Every configuration uses block_size 16 and one layer.  Pools are
[1, 2, NB, 16, Hkv, D] like hetero-serve's (heteroserve/kv/blocks.py:72-81),
filled from N(0, 1); block tables are cut from a seeded permutation of the
pool's blocks, so pages of one sequence are scattered, padded with -1.
Host-side randomness is numpy PCG64 and device-side a torch generator, both
seeded with the configuration number.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

BLOCK_SIZE = 16


@dataclass
class PagedCase:
    """One layer's paged KV plus the queries of one step."""

    name: str
    pool: "object"                 # torch [1, 2, NB, BS, Hkv, D]
    q: "object"                    # decode [B, H, D]; prefill [T, H, D] (packed rows)
    block_tables: "object"         # torch int32 [B, MB], -1 padded
    context_lens: "object"         # torch int32 [B]
    ctx: np.ndarray                # host copy of context_lens
    tables: list                   # host block lists
    n_heads: int
    scale: float
    q_lens: Optional[np.ndarray] = None       # prefill: rows per sequence
    cu_seqlens: Optional["object"] = None     # prefill: torch int32 [B + 1]
    meta: dict = field(default_factory=dict)

    @property
    def k_cache(self):
        return self.pool[0, 0]

    @property
    def v_cache(self):
        return self.pool[0, 1]

    @property
    def itemsize(self) -> int:
        return self.pool.element_size()

    @property
    def kv_heads(self) -> int:
        return self.pool.shape[4]

    @property
    def head_dim(self) -> int:
        return self.pool.shape[5]

    def row_bytes(self) -> int:
        """K + V bytes of one token of one layer."""
        return 2 * self.kv_heads * self.head_dim * self.itemsize

    def decode_bytes(self) -> int:
        """Algorithmic decode traffic: every context token's K and V once."""
        return int(self.ctx.astype(np.int64).sum()) * self.row_bytes()

    def unique_decode_bytes(self) -> int:
        """Decode traffic counting each shared (block, offset) slot once."""
        seen = set()
        for t, n in zip(self.tables, self.ctx):
            for j in range(int(n)):
                seen.add((t[j // BLOCK_SIZE], j % BLOCK_SIZE))
        return len(seen) * self.row_bytes()

    def prefill_flops(self) -> int:
        """Useful causal FLOPs: 4 * H * D * sum(S*P + S*(S+1)/2)."""
        S = self.q_lens.astype(np.int64)
        P = self.ctx.astype(np.int64) - S
        return int(4 * self.n_heads * self.head_dim * (S * P + S * (S + 1) // 2).sum())


def _torch():
    import torch

    return torch


def _fill_pool(pool, gen, scale: float = 1.0) -> None:
    """N(0, 1) * scale into the pool, one slab at a time (bounded temporaries)."""
    torch = _torch()
    flat = pool.view(-1, *pool.shape[3:])
    step = max(1, (1 << 28) // max(1, flat[0].numel()))
    for i in range(0, flat.shape[0], step):
        part = flat[i:i + step]
        tmp = torch.randn(part.shape, generator=gen, device=pool.device, dtype=torch.float32)
        if scale != 1.0:
            tmp.mul_(scale)
        part.copy_(tmp)


def _tables(rng, ctx: np.ndarray, num_blocks: int, shared: Optional[list] = None,
            share: Optional[np.ndarray] = None) -> list:
    """Per-sequence block lists cut from one seeded permutation of the pool.

    Sequences flagged in `share` start with the block ids in `shared` (a
    refcounted common prefix), then continue with fresh blocks.
    """
    perm = iter(rng.permutation(num_blocks).tolist())
    shared_set = set(shared or [])
    out = []
    for b, n in enumerate(ctx):
        need = -(-int(n) // BLOCK_SIZE)
        if shared and share is not None and share[b]:
            lst = list(shared[:need])
        else:
            lst = []
        while len(lst) < need:
            blk = next(perm)
            if blk not in shared_set:
                lst.append(blk)
        out.append(lst)
    return out


def _table_tensor(tables: list, device):
    torch = _torch()
    width = max(1, max(len(t) for t in tables))
    bt = np.full((len(tables), width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    return torch.from_numpy(bt).to(device)


# A device buffer that decode pools are carved from, or None (each pool its
# own allocation).  bench.py reserves it as the process's first large
# allocation and builds its decode legs' pools in it one case at a time, as a
# serving engine allocates its KV pool once: measured on MI355X, C2-gqa's
# decode ran 109.7 us on a process's first pool and 112.4 us on any pool
# allocated after a large one had been freed.
_POOL_ARENA = None


def set_pool_arena(buf) -> None:
    """Carve the pools of decode cases built from now on from `buf` (a uint8
    device tensor; None: allocate each pool).  Every build starts at the
    buffer's beginning, so a case built from it must be deleted before the
    next one is built."""
    global _POOL_ARENA
    _POOL_ARENA = buf


def _new_pool(shape, dtype, device):
    torch = _torch()
    n = int(np.prod(shape)) * torch.empty((), dtype=dtype).element_size()
    a = _POOL_ARENA
    if a is not None and a.device == torch.device(device) and n <= a.numel():
        return a[:n].view(dtype).view(shape)
    return torch.empty(shape, dtype=dtype, device=device)


def build_decode(name: str, ctx: np.ndarray, n_heads: int, kv_heads: int, head_dim: int,
                 num_blocks: int, dtype, device, seed: int, input_scale: float = 1.0,
                 rng=None, shared: Optional[list] = None,
                 share: Optional[np.ndarray] = None) -> PagedCase:
    torch = _torch()
    rng = rng if rng is not None else np.random.default_rng(seed)
    tables = _tables(rng, ctx, num_blocks, shared, share)
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = _new_pool((1, 2, num_blocks, BLOCK_SIZE, kv_heads, head_dim), dtype, device)
    _fill_pool(pool, gen, input_scale)
    q = torch.randn((len(ctx), n_heads, head_dim), generator=gen, device=device,
                    dtype=torch.float32)
    if input_scale != 1.0:
        q.mul_(input_scale)
    return PagedCase(name=name, pool=pool, q=q, block_tables=_table_tensor(tables, device),
                     context_lens=torch.from_numpy(ctx.astype(np.int32)).to(device),
                     ctx=ctx.astype(np.int64), tables=tables, n_heads=n_heads,
                     scale=1.0 / math.sqrt(head_dim))


def build_prefill(name: str, prefix: np.ndarray, chunk: np.ndarray, n_heads: int,
                  kv_heads: int, head_dim: int, num_blocks: int, dtype, device,
                  seed: int, rng=None) -> PagedCase:
    """Ragged chunked prefill: sequence b has prefix[b] cached tokens and a
    chunk of chunk[b] new tokens (already written to the pool)."""
    torch = _torch()
    rng = rng if rng is not None else np.random.default_rng(seed)
    ctx = (prefix + chunk).astype(np.int64)
    tables = _tables(rng, ctx, num_blocks)
    gen = torch.Generator(device=device).manual_seed(seed)
    pool = torch.empty((1, 2, num_blocks, BLOCK_SIZE, kv_heads, head_dim), dtype=dtype,
                       device=device)
    _fill_pool(pool, gen)
    total = int(chunk.sum())
    q = torch.randn((total, n_heads, head_dim), generator=gen, device=device,
                    dtype=torch.float32)
    cu = np.concatenate([[0], np.cumsum(chunk)]).astype(np.int32)
    return PagedCase(name=name, pool=pool, q=q, block_tables=_table_tensor(tables, device),
                     context_lens=torch.from_numpy(ctx.astype(np.int32)).to(device),
                     ctx=ctx, tables=tables, n_heads=n_heads,
                     scale=1.0 / math.sqrt(head_dim), q_lens=chunk.astype(np.int64),
                     cu_seqlens=torch.from_numpy(cu).to(device))


# ---------------------------------------------------------------------------
# the five configurations
# ---------------------------------------------------------------------------


def c1_decode(device, dtype=None) -> PagedCase:
    torch = _torch()
    rng = np.random.default_rng(0)
    ctx = rng.integers(16, 512, size=8, endpoint=True)
    return build_decode("C1", ctx, 12, 12, 64, 1024, dtype or torch.float16, device, 0,
                        input_scale=1.0 / math.sqrt(64), rng=rng)


def c2_ctx(rng) -> np.ndarray:
    ctx = np.rint(rng.lognormal(mean=math.log(2048), sigma=0.8, size=64))
    return np.clip(ctx, 64, 8192).astype(np.int64)


def c2_decode(device, dtype=None) -> PagedCase:
    torch = _torch()
    rng = np.random.default_rng(1)
    return build_decode("C2", c2_ctx(rng), 32, 32, 128, 65536, dtype or torch.bfloat16,
                        device, 1, rng=rng)


def c2_gqa_decode(device, dtype=None) -> PagedCase:
    """C2's batch and contexts at Llama-3-8B's attention geometry
    (ModelConfig.llama3_8b_shape, heteroserve/config.py:85-93): 32 query heads
    sharing 8 KV heads, so each KV page serves a group of 4."""
    torch = _torch()
    rng = np.random.default_rng(1)
    return build_decode("C2-gqa", c2_ctx(rng), 32, 8, 128, 65536, dtype or torch.bfloat16,
                        device, 1, rng=rng)


def c3_decode(device, dtype=None) -> PagedCase:
    torch = _torch()
    rng = np.random.default_rng(2)
    ctx = rng.integers(8192, 32768, size=16, endpoint=True)
    need = int(sum(-(-int(n) // BLOCK_SIZE) for n in ctx))
    return build_decode("C3", ctx, 32, 32, 128, 2 * need, dtype or torch.bfloat16, device, 2,
                        rng=rng)


def b64_4k_decode(device, dtype=None) -> PagedCase:
    """Batch 64 at a 4k context (the decode target's "batch 64 / 4k
    context"): C2's geometry, 32 heads MHA, D 128, bf16, every context 4096
    tokens, pages scattered over a 65536-block pool."""
    torch = _torch()
    rng = np.random.default_rng(6)
    ctx = np.full(64, 4096, dtype=np.int64)
    return build_decode("B64-4k", ctx, 32, 32, 128, 65536, dtype or torch.bfloat16, device, 6,
                        rng=rng)


def c4_prefill(device, dtype=None) -> PagedCase:
    torch = _torch()
    rng = np.random.default_rng(3)
    prefix = rng.integers(0, 4096, size=8, endpoint=True)
    chunk = rng.integers(128, 2048, size=8, endpoint=True)
    need = int(sum(-(-int(p + s) // BLOCK_SIZE) for p, s in zip(prefix, chunk)))
    return build_prefill("C4", prefix, chunk, 32, 32, 128, 2 * need, dtype or torch.bfloat16,
                         device, 3, rng=rng)


C5_POOL_BLOCKS = 65536


def c5_decode(device, dtype=None) -> PagedCase:
    """255 decode sequences; the even-indexed half share a 1024-token prefix."""
    torch = _torch()
    rng = np.random.default_rng(4)
    ctx = rng.integers(256, 4096, size=255, endpoint=True)
    shared = rng.choice(C5_POOL_BLOCKS, size=1024 // BLOCK_SIZE, replace=False).tolist()
    share = np.arange(255) % 2 == 0
    case = build_decode("C5-decode", ctx, 32, 32, 128, C5_POOL_BLOCKS,
                        dtype or torch.bfloat16, device, 4, rng=rng, shared=shared,
                        share=share)
    case.meta["shared_blocks"] = shared
    return case


def c5_decode_tables():
    """C5's decode batch without its pool: (context lengths, block lists),
    the same seeded values c5_decode builds."""
    rng = np.random.default_rng(4)
    ctx = rng.integers(256, 4096, size=255, endpoint=True)
    shared = rng.choice(C5_POOL_BLOCKS, size=1024 // BLOCK_SIZE, replace=False).tolist()
    share = np.arange(255) % 2 == 0
    return ctx, _tables(rng, ctx, C5_POOL_BLOCKS, shared, share)


def c5_prefill(device, dtype=None) -> PagedCase:
    torch = _torch()
    rng = np.random.default_rng(40)
    return build_prefill("C5-prefill", np.array([2048]), np.array([1024]), 32, 32, 128,
                         8192, dtype or torch.bfloat16, device, 40, rng=rng)


def c5_pack_ids(num_blocks: int = C5_POOL_BLOCKS, n: int = 4096) -> list:
    """4096 distinct random block ids of the C5 pool, seeded."""
    rng = np.random.default_rng(41)
    return rng.choice(num_blocks, size=n, replace=False).tolist()


CONFIGS = {
    "C1": c1_decode,
    "C2": c2_decode,
    "C2-gqa": c2_gqa_decode,
    "C3": c3_decode,
    "B64-4k": b64_4k_decode,
    "C4": c4_prefill,
    "C5-decode": c5_decode,
    "C5-prefill": c5_prefill,
}
