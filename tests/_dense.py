"""fp64 dense attention by brute force: the mathematical definition the paged
kernels and the oracle must both agree with.

These loops never touch a block table, a mask tensor or a partition, so a
mistake in any of those (a wrong slot, an off-by-one causal bound, a GQA head
mapping, a dropped scale) separates the paged result from this one.
"""

from __future__ import annotations

import numpy as np


def dense_decode(q, k, v, scale):
    """q [H, D]; k, v [n, Hkv, D] -> [H, D]: softmax over all n keys."""
    H = q.shape[0]
    hkv = k.shape[1]
    out = np.zeros((H, q.shape[1]))
    for h in range(H):
        kh = h // (H // hkv)
        s = np.array([float(np.dot(q[h].astype(np.float64), k[j, kh].astype(np.float64)))
                      for j in range(k.shape[0])]) * scale
        w = np.exp(s - s.max())
        out[h] = (w[:, None] * v[:, kh].astype(np.float64)).sum(0) / w.sum()
    return out


def dense_causal(q, k, v, scale, q_start):
    """q [S, H, D] at positions q_start + s; k, v [N, Hkv, D] -> [S, H, D].

    Row s attends to keys [0, q_start + s]; a row with no key is 0.
    """
    S, H, D = q.shape
    out = np.zeros((S, H, D))
    for s in range(S):
        end = q_start + s + 1
        if end <= 0:
            continue
        out[s] = dense_decode(q[s], k[:end], v[:end], scale)
    return out
