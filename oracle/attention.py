"""Torch (CPU) oracle of paged decode and causal prefill attention.

Test infrastructure: see oracle/__init__.py.
"""

from __future__ import annotations

import torch


def _slot_positions(block_tables: torch.Tensor, block_size: int) -> torch.Tensor:
    """Flat pool row of every logical position: [B, MB * BS] int64.

    heteroserve/model/paged_attn.py:274-278 -- a position j lives in block
    block_tables[b][j // BS] (entries clamped to >= 0) at offset j % BS.
    """
    blocks = block_tables.to(torch.int64).clamp(min=0)
    offs = torch.arange(block_size, dtype=torch.int64, device=blocks.device)
    return (blocks[:, :, None] * block_size + offs).flatten(1)


def _gather_heads(cache: torch.Tensor, slots: torch.Tensor, n_heads: int) -> torch.Tensor:
    """[B, K, H, D] fp32 rows of `cache` at `slots`, KV heads expanded for GQA.

    heteroserve/model/paged_attn.py:280-291 (query head h reads KV head
    h // (H / Hkv)).
    """
    nb, bs, hkv, d = cache.shape
    rows = cache.reshape(nb * bs, hkv, d).index_select(0, slots.reshape(-1))
    rows = rows.reshape(*slots.shape, hkv, d).to(torch.float32)
    if n_heads != hkv:
        rows = rows.repeat_interleave(n_heads // hkv, dim=2)
    return rows


def paged_attention_torch(q, k_cache, v_cache, block_tables, context_lens, scale):
    """Decode attention through the block table, masked to the context.

    heteroserve/model/paged_attn.py:255-298: q [B, H, D] fp32, caches
    [NB, BS, Hkv, D], block_tables [B, MB], context_lens [B] -> [B, H, D] fp32.
    Positions >= context_lens[b] are masked with -inf before the softmax, so a
    sequence with no context yields NaN, as in the reference.
    """
    B, H, _ = q.shape
    bs = k_cache.shape[1]
    slots = _slot_positions(block_tables, bs)
    k = _gather_heads(k_cache, slots, H)
    v = _gather_heads(v_cache, slots, H)
    scores = torch.einsum("bhd,bkhd->bhk", q.to(torch.float32), k) * scale
    pos = torch.arange(slots.shape[1], device=q.device)
    live = pos[None, :] < context_lens.to(pos.dtype)[:, None]
    scores = scores.masked_fill(~live[:, None, :], float("-inf"))
    return torch.einsum("bhk,bkhd->bhd", torch.softmax(scores, dim=-1), v)


def paged_attention_prefill_torch(q, k_cache, v_cache, block_tables, context_lens, scale):
    """Causal chunked prefill through the block table.

    heteroserve/model/paged_attn_prefill.py:281-322: q [B, S, H, D]; query s of
    sequence b sits at position ctx_b - S + s and may see keys k with
    k <= that position and k < ctx_b; fully masked rows (negative positions)
    are 0 (nan_to_num).
    """
    B, S, H, _ = q.shape
    bs = k_cache.shape[1]
    slots = _slot_positions(block_tables, bs)
    k = _gather_heads(k_cache, slots, H)
    v = _gather_heads(v_cache, slots, H)
    scores = torch.einsum("bshd,bkhd->bshk", q.to(torch.float32), k) * scale
    ctx = context_lens.to(torch.int64)
    key = torch.arange(slots.shape[1], device=q.device)
    qpos = ctx[:, None] - S + torch.arange(S, device=q.device)[None, :]
    live = (key[None, None, :] <= qpos[:, :, None]) & (key[None, None, :] < ctx[:, None, None])
    scores = scores.masked_fill(~live[:, :, None, :], float("-inf"))
    probs = torch.nan_to_num(torch.softmax(scores, dim=-1), nan=0.0)
    return torch.einsum("bshk,bkhd->bshd", probs, v)


# ---------------------------------------------------------------------------
# per-sequence forms: same function, without padding the batch to MB * BS
# ---------------------------------------------------------------------------


def _sequence_kv(k_cache, v_cache, table_row, n: int, n_heads: int):
    """[n, H, D] fp32 K and V of the first n positions of one sequence."""
    bs = k_cache.shape[1]
    nblk = -(-n // bs)
    blocks = table_row[:nblk].to(torch.int64).clamp(min=0)
    k = k_cache.index_select(0, blocks).reshape(nblk * bs, *k_cache.shape[2:])[:n]
    v = v_cache.index_select(0, blocks).reshape(nblk * bs, *v_cache.shape[2:])[:n]
    k, v = k.to(torch.float32), v.to(torch.float32)
    if n_heads != k.shape[1]:
        g = n_heads // k.shape[1]
        k, v = k.repeat_interleave(g, dim=1), v.repeat_interleave(g, dim=1)
    return k, v


def decode_one(q_b, k_cache, v_cache, table_row, ctx_b: int, scale):
    """paged_attention_torch for a single sequence: q_b [H, D] -> [H, D].

    Identical function (heteroserve/model/paged_attn.py:255-298); masked
    positions contribute exp(-inf) = 0 there, so dropping them is exact.
    """
    H = q_b.shape[0]
    n = min(int(ctx_b), table_row.shape[0] * k_cache.shape[1])
    if n <= 0:
        return torch.full_like(q_b, float("nan"), dtype=torch.float32)
    k, v = _sequence_kv(k_cache, v_cache, table_row, n, H)
    s = torch.einsum("hd,nhd->hn", q_b.to(torch.float32), k) * scale
    return torch.einsum("hn,nhd->hd", torch.softmax(s, dim=-1), v)


def prefill_one(q_b, k_cache, v_cache, table_row, ctx_b: int, scale):
    """paged_attention_prefill_torch for a single sequence: q_b [S, H, D].

    heteroserve/model/paged_attn_prefill.py:281-322 with B = 1, the shape the
    engine uses (heteroserve/model/torch_engine.py:292-294).
    """
    S, H, _ = q_b.shape
    n = min(int(ctx_b), table_row.shape[0] * k_cache.shape[1])
    out = torch.zeros(S, H, q_b.shape[2], dtype=torch.float32)
    if n <= 0:
        return out
    k, v = _sequence_kv(k_cache, v_cache, table_row, n, H)
    s = torch.einsum("shd,nhd->shn", q_b.to(torch.float32), k) * scale
    qpos = int(ctx_b) - S + torch.arange(S)
    live = torch.arange(n)[None, :] <= qpos[:, None]
    s = s.masked_fill(~live[:, None, :], float("-inf"))
    p = torch.nan_to_num(torch.softmax(s, dim=-1), nan=0.0)
    return torch.einsum("shn,nhd->shd", p, v)
