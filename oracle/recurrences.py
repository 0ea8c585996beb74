"""numpy oracle of the kernels' own recurrences (online softmax, split/merge,
the tile loop of the matrix-core prefill).

Test infrastructure: see oracle/__init__.py.  These are fp64 scalar or
tile-level loops that mirror what a kernel does step by step, so that an
algorithmic mistake shows on the CPU against dense attention.
"""

from __future__ import annotations

import numpy as np

NEG_BIG = -3.0e38   # heteroserve/model/paged_attn_wmma.py:399


def _online_state(q, k, v, scale, lo: int, hi: int):
    """Running (m, l, acc) over keys [lo, hi) for every head, in fp64.

    The recurrence of heteroserve/model/paged_attn_v2.py:296-311: per key,
    m' = max(m, s); l = l * e^(m - m') + e^(s - m'); acc likewise; the first
    key has no previous state (correction 0).
    """
    H, D = q.shape
    qd = q.astype(np.float64)
    m = np.full(H, -np.inf)
    l = np.zeros(H)
    acc = np.zeros((H, D))
    for j in range(lo, hi):
        s = (qd * k[j].astype(np.float64)).sum(axis=-1) * scale
        m_new = np.maximum(m, s)
        corr = np.where(np.isfinite(m), np.exp(m - m_new), 0.0)
        p = np.exp(s - m_new)
        l = l * corr + p
        acc = acc * corr[:, None] + p[:, None] * v[j].astype(np.float64)
        m = m_new
    return m, l, acc


def online_softmax_reference(q, k, v, scale):
    """One streaming pass: q [H, D], k, v [n, H, D] -> [H, D] fp32.

    heteroserve/model/paged_attn_v2.py:284-313.
    """
    _, l, acc = _online_state(q, k, v, scale, 0, k.shape[0])
    return (acc / l[:, None]).astype(np.float32)


def split_merge_reference(q, k, v, scale, num_splits: int):
    """Context cut into num_splits slices of ceil(n / num_splits) keys, one
    online pass per slice, then the log-sum-exp merge.

    heteroserve/model/paged_attn_v3.py:370-408; an empty slice has m = -inf
    and weight 0.
    """
    H, D = q.shape
    n = k.shape[0]
    chunk = -(-n // num_splits)
    states = [_online_state(q, k, v, scale, s * chunk, min((s + 1) * chunk, n))
              for s in range(num_splits)]
    m_g = np.max(np.stack([m for m, _, _ in states]), axis=0)
    l_g = np.zeros(H)
    out = np.zeros((H, D))
    for m, l, acc in states:
        w = np.where(np.isfinite(m), np.exp(m - m_g), 0.0)
        l_g += l * w
        out += acc * w[:, None]
    return (out / l_g[:, None]).astype(np.float32)


def tiled_prefill_reference(q, k, v, scale, ctx_len, tile: int = 16):
    """The matrix-core prefill's tile loop for one head, in fp64.

    heteroserve/model/paged_attn_wmma.py:402-458: q [S, D] are the trailing S
    positions of a context of ctx_len keys k, v [N, D].  Query tiles of `tile`
    rows walk key tiles of `tile` keys up to the tile's last causal position;
    masked scores take the finite sentinel NEG_BIG (so a fully masked tile
    never computes exp(-inf + inf)) and get probability 0; a row with l = 0
    outputs 0.
    """
    S, D = q.shape
    out = np.zeros((S, D))
    for q0 in range(0, S, tile):
        rows = min(tile, S - q0)
        qt = np.zeros((tile, D))
        qt[:rows] = q[q0:q0 + rows]
        pos0 = ctx_len - S + q0                   # position of the tile's first row
        m = np.full(tile, NEG_BIG)
        l = np.zeros(tile)
        o = np.zeros((tile, D))
        key_end = min(ctx_len, pos0 + tile)       # one past the last row's position
        n_kt = max(0, -(-key_end // tile))
        for kt in range(n_kt):
            k0 = kt * tile
            kk = np.zeros((tile, D))
            vv = np.zeros((tile, D))
            take = max(0, min(tile, len(k) - k0))
            kk[:take] = k[k0:k0 + take]
            vv[:take] = v[k0:k0 + take]
            sc = (qt @ kk.T) * scale
            r = np.arange(tile)[:, None]
            c = np.arange(tile)[None, :]
            qpos = pos0 + r
            keep = ((q0 + r) < S) & (qpos >= 0) & (k0 + c <= qpos) & (k0 + c < ctx_len)
            sc = np.where(keep, sc, NEG_BIG)
            m_new = np.maximum(m, sc.max(axis=1))
            corr = np.exp(m - m_new)
            p = np.where(sc <= NEG_BIG, 0.0, np.exp(sc - m_new[:, None]))
            l = l * corr + p.sum(axis=1)
            o = o * corr[:, None] + p @ vv
            m = m_new
        for i in range(rows):
            out[q0 + i] = o[i] / l[i] if l[i] > 0 else 0.0
    return out.astype(np.float32)
