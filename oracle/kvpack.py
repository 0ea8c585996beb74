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
