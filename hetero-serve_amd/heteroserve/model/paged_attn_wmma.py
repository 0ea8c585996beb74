"""Causal chunked prefill on the matrix cores (the reference's WMMA path).

Interface of heteroserve/model/paged_attn_wmma.py (is_available :362,
build_error :367, supports :372-387, paged_attention_prefill_wmma :390-396,
NEG_BIG :399).  The reference runs 16x16x16 WMMA fragments on fp16 caches;
here the kernel is a FlashAttention-style loop on gfx950 MFMA with fp16
operands and fp32 accumulation, reading 16-token KV pages through the block
table.  It takes fp16 or bf16 caches (bf16 pages are widened to fp16
operands, exact for |x| < 65504).

``supports`` keeps the reference's geometry gate -- block_size 16 and
head_dim in {32, 64, 128} -- and widens the dtype gate to {fp16, bf16}.
"""

from __future__ import annotations

from typing import Optional

from .. import _hip

NEG_BIG = -3.0e38


def is_available() -> bool:
    return _hip.ready()


def build_error() -> Optional[str]:
    return _hip.error()


def supports(block_size: int, head_dim: int, kv_dtype) -> bool:
    """Whether the matrix-core kernel can serve this cache geometry."""
    import torch

    return (
        is_available()
        and block_size == 16
        and head_dim % 16 == 0
        and head_dim in (32, 64, 128)
        and kv_dtype in (torch.float16, torch.bfloat16)
    )


def paged_attention_prefill_wmma(q, k_cache, v_cache, block_tables, context_lens, scale):
    _hip.lib("MFMA prefill kernel")
    return _hip.prefill(q, k_cache, v_cache, block_tables, context_lens, scale, use_mfma=True)
