"""numpy oracle of KV-block migration pack/unpack and the contiguous gather.

Test infrastructure: see oracle/__init__.py.  All three are bitwise copies;
the GPU results must equal these byte for byte.
"""

from __future__ import annotations

import numpy as np


def export_blocks(pool: np.ndarray, block_ids) -> np.ndarray:
    """out[i, l, c] = pool[l, c, block_ids[i]]: [n, L, 2, BS, H, D].

    heteroserve/kv/blocks.py:281-285 and heteroserve/kv/torch_blocks.py:137-148
    (pool[:, :, idx].permute(2, 0, 1, 3, 4, 5)); negative ids wrap as numpy
    and torch indexing do.
    """
    idx = np.asarray(list(block_ids), dtype=np.int64)
    return np.ascontiguousarray(np.moveaxis(pool[:, :, idx], 2, 0))


def write_blocks(pool: np.ndarray, block_ids, payload: np.ndarray) -> None:
    """pool[:, :, block_ids[i]] = payload[i], in order (a later id wins).

    heteroserve/kv/blocks.py:306-317, heteroserve/kv/torch_blocks.py:150-154.
    """
    for i, blk in enumerate(block_ids):
        pool[:, :, blk] = payload[i]


def export_blocks_torch(pool, block_ids):
    """The same payload with torch on a CPU pool tensor, in the reference's
    own expression: pool[:, :, idx].permute(2, 0, 1, 3, 4, 5).contiguous().

    heteroserve/kv/torch_blocks.py:137-148 (export_blocks_device).  The
    benchmark times this as the pack's CPU baseline.
    """
    import torch

    idx = torch.as_tensor(list(block_ids), dtype=torch.long)
    return pool[:, :, idx].permute(2, 0, 1, 3, 4, 5).contiguous()


def write_blocks_torch(pool, block_ids, payload) -> None:
    """pool[:, :, blk] = payload[i] for each (i, blk), in order, with torch on
    CPU tensors: the reference's per-block loop.

    heteroserve/kv/torch_blocks.py:150-154 (write_blocks_device).
    """
    for i, blk in enumerate(block_ids):
        pool[:, :, int(blk)] = payload[i]


def gather_kv_batch(pool: np.ndarray, tables, length: int, layer: int):
    """([B, length, H, D], same for V) through each sequence's block list.

    heteroserve/kv/torch_blocks.py:125-135 with slots from slots_for
    (:68-73): slot = table[pos // BS] * BS + pos % BS.
    """
    _, _, nb, bs, h, d = pool.shape
    pos = np.arange(length)
    ks, vs = [], []
    for t in tables:
        tbl = np.asarray(list(t), dtype=np.int64)
        slots = tbl[pos // bs] * bs + pos % bs
        ks.append(pool[layer, 0].reshape(nb * bs, h, d)[slots])
        vs.append(pool[layer, 1].reshape(nb * bs, h, d)[slots])
    shape = (0, length, h, d)
    return (np.stack(ks) if ks else np.zeros(shape, pool.dtype),
            np.stack(vs) if vs else np.zeros(shape, pool.dtype))


# ---------------------------------------------------------------------------
# writing new K/V rows (the step before attention)
# ---------------------------------------------------------------------------

def slots_for(block_ids, positions, block_size: int) -> np.ndarray:
    """Flat slots of absolute positions through one block table, int64.

    heteroserve/kv/torch_blocks.py:68-73: tbl[pos // BS] * BS + pos % BS.
    """
    tbl = np.asarray(list(block_ids), dtype=np.int64)
    pos = np.asarray(list(positions), dtype=np.int64)
    return tbl[pos // block_size] * block_size + pos % block_size


def scatter_rows(cache, slots, rows) -> None:
    """cache.view(-1, H, D)[slots] = rows.to(cache dtype), on CPU torch.

    The engine's write of one step's new K (or V), heteroserve/model/
    torch_engine.py:239-240 (decode) and :306-308 (a prefill chunk): `cache`
    is one layer's [NB, BS, H, D] pool view, `rows` is [n, H, D].  torch's
    `.to()` supplies the rounding (round to nearest even).
    """
    import torch

    flat = cache.reshape(-1, cache.shape[2], cache.shape[3])
    flat[torch.as_tensor(slots, dtype=torch.long)] = torch.as_tensor(rows).to(cache.dtype)


def write_kv(pool, block_ids, start_pos: int, k, v) -> None:
    """TorchBlockAllocator.write_kv, heteroserve/kv/torch_blocks.py:89-106.

    pool [L, 2, NB, BS, H, D] (CPU torch); k, v [L, H, T, D] of one sequence
    written at positions start_pos .. start_pos + T - 1 of every layer.
    """
    import torch

    k = torch.as_tensor(k)
    v = torch.as_tensor(v)
    T = int(k.shape[2])
    if T == 0:
        return
    bs = pool.shape[3]
    slots = slots_for(block_ids, range(start_pos, start_pos + T), bs)
    kt = k.permute(0, 2, 1, 3).contiguous()
    vt = v.permute(0, 2, 1, 3).contiguous()
    for layer in range(pool.shape[0]):
        scatter_rows(pool[layer, 0], slots, kt[layer])
        scatter_rows(pool[layer, 1], slots, vt[layer])


def block_table_tensor(tables, pad_to=None):
    """TorchBlockAllocator.block_table_tensor, heteroserve/kv/torch_blocks.py:75-85,
    on CPU torch: [len(tables), width] int32, -1 padded, rows truncated to width."""
    import torch

    width = pad_to or max((len(t) for t in tables), default=1)
    out = torch.full((len(tables), width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        if t:
            out[i, : len(t)] = torch.as_tensor(list(t)[:width], dtype=torch.int32)
    return out
