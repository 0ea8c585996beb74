"""Paged decode attention, v1 entry point: hetero-serve's engine calls this one.

Interface of heteroserve/model/paged_attn.py (which_backend :244,
build_error :249, paged_attention :301-308); the engine's decode step calls
``paged_attention`` once per layer (heteroserve/model/torch_engine.py:242-245).

Layout, as in the reference:

    q                   [B, H, D]            float32
    k_cache / v_cache   [num_blocks, block_size, n_kv_heads, head_dim]
                        (views pool[layer, 0] / pool[layer, 1]); fp32, fp16 or bf16
    block_tables        [B, max_blocks]      int32, -1 for unused slots
    context_lens        [B]                  int32
    ->                  [B, H, D]            float32

The reference's v1 kernel keeps every score in shared memory; here the call
runs libhsattn's partitioned online-softmax decode (fixed 512-token
partitions plus a log-sum-exp merge), which computes the same function.

Difference from the reference: when the HIP library is unavailable the
reference silently computes with torch; this module raises RuntimeError
instead, so a caller can never get a CPU result it did not ask for.  The
worker calls ``paged_attention`` when ``which_backend() == "cuda"`` and also,
with no GPU kernel at all, when HETEROSERVE_FORCE_PAGED is set
(worker.py:209-211; the reference's CPU test test_distributed.py:326-371 runs
that way).  So the binding that goes into the reference tree keeps the
reference's own torch branch for that case (the module's
``paged_attention_torch``, which stays there); this repository ships no CPU
path.
"""

from __future__ import annotations

from typing import Optional

from .. import _hip


def which_backend() -> str:
    """'cuda' when libhsattn.so is loaded on a HIP device, else 'torch'.

    PyTorch-ROCm keeps CUDA's device names, and the worker takes the fused
    path only on the literal 'cuda', so that is what a working HIP library
    reports.  'none' means torch itself is missing.
    """
    try:
        import torch  # noqa: F401
    except ImportError:
        return "none"
    return "cuda" if _hip.ready() else "torch"


def build_error() -> Optional[str]:
    """Why the HIP library is unavailable, or None."""
    return _hip.error()


def paged_attention(q, k_cache, v_cache, block_tables, context_lens, scale,
                    shared_pages: bool = False):
    """Decode attention over the paged pool on the GPU (raises when unavailable).

    shared_pages (not in the reference's signature, default off): for batches
    whose sequences share cached prefix pages, read a partition that several
    sequences hold once for all of them (hs_decode_shared; same function,
    matrix-core products with split 16-bit operands on the shared partitions,
    fp32-grade results)."""
    return _hip.decode(q, k_cache, v_cache, block_tables, context_lens, scale, num_splits=0,
                       shared_pages=shared_pages)
