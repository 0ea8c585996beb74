"""Integer oracle of the v3 split-count heuristic.

Test infrastructure: see oracle/__init__.py.
"""

from __future__ import annotations


def choose_num_splits(num_seqs: int, num_heads: int, max_context: int, cus: int) -> int:
    """heteroserve/model/paged_attn_v3.py:212-232 with `cus` compute units:
    clamp(max(max_context // 32, ceil(cus * 8 / (num_seqs * num_heads))), 1, 64),
    each term at least 1.
    """
    have = max(num_seqs * num_heads, 1)
    by_chain = max(max_context // 32, 1)
    to_fill = max((cus * 8 + have - 1) // have, 1)
    return max(1, min(max(by_chain, to_fill), 64))
