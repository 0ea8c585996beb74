"""Paged decode attention, v2 entry point: one online-softmax pass per (sequence, head).

Interface of heteroserve/model/paged_attn_v2.py (is_available :265,
build_error :270, paged_attention_v2 :275-281, bytes_moved :321-327,
peak_bandwidth_gbs :330-345).  ``paged_attention_v2`` runs libhsattn's decode
kernel with a single partition per (sequence, head), i.e. the reference's
single-pass algorithm; it raises RuntimeError when the library is unavailable,
as the reference does.
"""

from __future__ import annotations

from typing import Optional

from .. import _hip

# Published HBM3E peak of MI355X (gfx950), GB/s.
_PEAK_GBS_BY_ARCH = {"gfx950": 8000.0}


def is_available() -> bool:
    return _hip.ready()


def build_error() -> Optional[str]:
    return _hip.error()


def paged_attention_v2(q, k_cache, v_cache, block_tables, context_lens, scale):
    _hip.lib("v2 kernel")
    return _hip.decode(q, k_cache, v_cache, block_tables, context_lens, scale, num_splits=1)


def bytes_moved(batch: int, context: int, n_heads: int, head_dim: int, itemsize: int) -> int:
    """Minimum bytes a decode attention must read: K and V once each (MHA)."""
    return 2 * batch * context * n_heads * head_dim * itemsize


def peak_bandwidth_gbs() -> Optional[float]:
    """Peak HBM bandwidth of the current device in GB/s, or None if unknown.

    For gfx950 this is the published 8000 GB/s; for other devices the
    clock * bus-width estimate the reference uses, when torch exposes it.
    """
    try:
        import torch

        if not torch.cuda.is_available():
            return None
        p = torch.cuda.get_device_properties(0)
        arch = getattr(p, "gcnArchName", "").split(":")[0]
        if arch in _PEAK_GBS_BY_ARCH:
            return _PEAK_GBS_BY_ARCH[arch]
        clock_khz = getattr(p, "memory_clock_rate", None)
        bus_bits = getattr(p, "memory_bus_width", None)
        if not clock_khz or not bus_bits:
            return None
        return (clock_khz * 1e3 * 2 * (bus_bits / 8)) / 1e9
    except Exception:  # noqa: BLE001 - a probe, never fatal
        return None
