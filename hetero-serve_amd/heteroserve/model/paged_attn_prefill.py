"""Causal chunked prefill over the paged cache, fp32 VALU entry point.

Interface of heteroserve/model/paged_attn_prefill.py (is_available :253,
build_error :258, paged_attention_prefill :263-278).

    q               [B, S, H, D] float32; query s of sequence b sits at
                    position context_lens[b] - S + s and attends to keys
                    [0, context_lens[b] - S + s]; rows at negative positions
                    (padding) are zero
    ->              [B, S, H, D] float32

Runs libhsattn's row kernel (one online-softmax pass per query row and head,
fp32 arithmetic, any KV dtype).  Difference from the reference: no torch
fallback -- RuntimeError when the library is unavailable.  The binding that
goes into the reference tree keeps the reference's torch branch
(``paged_attention_prefill_torch``) for hosts without the library, which the
worker reaches under HETEROSERVE_FORCE_PAGED (worker.py:209-211).
"""

from __future__ import annotations

from typing import Optional

from .. import _hip


def is_available() -> bool:
    return _hip.ready()


def build_error() -> Optional[str]:
    return _hip.error()


def paged_attention_prefill(q, k_cache, v_cache, block_tables, context_lens, scale):
    _hip.lib("prefill kernel")
    return _hip.prefill(q, k_cache, v_cache, block_tables, context_lens, scale, use_mfma=False)


def paged_attention_prefill_varlen(q, cu_seqlens_q, max_seqlen_q, k_cache, v_cache,
                                   block_tables, context_lens, scale, use_mfma: bool = True):
    """Several ragged chunks in one launch (no reference counterpart).

    q [total, H, D]; sequence b owns rows cu_seqlens_q[b]:cu_seqlens_q[b+1],
    which are the trailing tokens of its context.  use_mfma selects the
    matrix-core kernel (fp16/bf16 KV, block_size 16) or the fp32 row kernel.
    """
    _hip.lib("prefill kernel")
    return _hip.prefill_varlen(q, cu_seqlens_q, max_seqlen_q, k_cache, v_cache,
                               block_tables, context_lens, scale, use_mfma)
