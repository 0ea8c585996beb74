"""Paged decode attention, v3 entry point: context split plus log-sum-exp merge.

Interface of heteroserve/model/paged_attn_v3.py (is_available :342,
build_error :347, choose_num_splits :352-356, paged_attention_v3 :359-367).

``num_splits > 0`` keeps the reference's decomposition: every sequence's
context is cut into ``num_splits`` slices of ceil(ctx / num_splits) tokens,
each slice runs an independent online softmax, and a merge kernel combines
the partial states.  ``num_splits <= 0`` lets the library choose; on MI355X it
uses fixed 512-token partitions, which balance a ragged batch across the 256
CUs better than a per-batch split count.  Results do not depend on the
decomposition (the reference asserts this, test_torch_engine.py:405-429).
"""

from __future__ import annotations

from typing import Optional

from .. import _hip


def is_available() -> bool:
    return _hip.ready()


def build_error() -> Optional[str]:
    return _hip.error()


def choose_num_splits(num_seqs: int, num_heads: int, max_context: int) -> int:
    """The reference's split heuristic with the device's CU count."""
    return _hip.choose_num_splits(num_seqs, num_heads, max_context)


def paged_attention_v3(q, k_cache, v_cache, block_tables, context_lens, scale,
                       num_splits: int = 0):
    """num_splits <= 0 lets the library pick the context decomposition."""
    _hip.lib("v3 kernel")
    return _hip.decode(q, k_cache, v_cache, block_tables, context_lens, scale,
                       num_splits=max(int(num_splits), 0))
