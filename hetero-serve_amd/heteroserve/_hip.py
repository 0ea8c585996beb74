"""Loader and tensor marshalling for libhsattn.so (the gfx950 C-ABI library).

This module is the only place that touches ctypes.  It keeps the reference's
module-state contract (heteroserve/model/paged_attn.py:197-252): the library is
loaded once, on first use, and a failure is recorded with a reason rather than
raised at import.  Unlike the reference there is no compute fallback: an entry
point called while the library is unavailable raises RuntimeError.

Environment:
  HETEROSERVE_DISABLE_CUDA_KERNEL  treat the library as unavailable (reference flag)
  HETEROSERVE_HIP_LIB              path of libhsattn.so (default: next to this file)
  HETEROSERVE_PREFILL_GRID=1       keep the MFMA prefill on its grid kernel (one workgroup
                                   per query tile) where the persistent one would run;
                                   read at each call, for comparisons

PyTorch provides device memory and the current stream; every kernel launches
on ``torch.cuda.current_stream(device)`` of the input's device.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Optional

ABI_VERSION = 5
DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None
_state = "unloaded"          # "unloaded" | "ready" | "unavailable"
_error: Optional[str] = None

_c_int, _c_i64, _c_size, _c_float, _c_vp = (
    ctypes.c_int, ctypes.c_int64, ctypes.c_size_t, ctypes.c_float, ctypes.c_void_p)

# name -> (restype, argtypes); must match include/hsattn.h
_SIGNATURES = {
    "hs_abi_version": (_c_int, []),
    "hs_last_error": (ctypes.c_char_p, []),
    "hs_profile_next_launch": (_c_int, [_c_vp, _c_vp]),
    "hs_device_cu_count": (_c_int, [_c_int]),
    "hs_choose_num_splits": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "hs_decode_workspace_bytes": (_c_size, [_c_int] * 8),
    "hs_decode": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                           _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
                           _c_int, _c_int, _c_vp, _c_size, _c_vp]),
    "hs_decode_noalloc": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                                   _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
                                   _c_int, _c_int, _c_vp]),
    "hs_decode_shared_workspace_bytes": (_c_size, [_c_int] * 7),
    "hs_decode_shared": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                                  _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_float,
                                  _c_int, _c_vp, _c_size, _c_vp]),
    "hs_prefill_workspace_bytes": (_c_size, [_c_int] * 5),
    "hs_prefill": (_c_int, [_c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_vp, _c_vp, _c_vp,
                            _c_int, _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                            _c_float, _c_int, _c_vp, _c_size, _c_vp]),
    "hs_prefill_varlen": (_c_int, [_c_vp, _c_vp, _c_int, _c_vp, _c_vp, _c_int, _c_int,
                                   _c_vp, _c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int,
                                   _c_int, _c_int, _c_float, _c_int, _c_vp, _c_size, _c_vp]),
    "hs_kv_pack": (_c_int, [_c_vp, _c_int, _c_int, _c_i64, _c_vp, _c_int, _c_vp, _c_vp]),
    "hs_kv_unpack": (_c_int, [_c_vp, _c_int, _c_int, _c_i64, _c_vp, _c_int, _c_vp, _c_vp]),
    "hs_kv_gather": (_c_int, [_c_vp, _c_int, _c_int, _c_i64, _c_vp, _c_int, _c_int, _c_int,
                              _c_vp, _c_vp]),
    "hs_block_tables": (_c_int, [_c_vp, _c_int, _c_int, _c_vp, _c_vp]),
    "hs_kv_scatter": (_c_int, [_c_vp, _c_vp, _c_int, _c_i64, _c_int, _c_int, _c_vp, _c_i64,
                               _c_vp, _c_vp, _c_int, _c_i64, _c_vp]),
    "hs_kv_append": (_c_int, [_c_vp, _c_vp, _c_int, _c_int, _c_int, _c_int, _c_int, _c_vp,
                              _c_int, _c_int, _c_vp, _c_vp, _c_i64, _c_vp, _c_vp, _c_int, _c_i64,
                              _c_vp]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def lib_path() -> Path:
    env = os.environ.get("HETEROSERVE_HIP_LIB")
    return Path(env) if env else Path(__file__).resolve().parent / "libhsattn.so"


def open_library(path: Optional[Path] = None) -> ctypes.CDLL:
    """dlopen libhsattn.so and bind its signatures.  Needs no GPU."""
    lib = ctypes.CDLL(str(path or lib_path()))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    got = lib.hs_abi_version()
    if got != ABI_VERSION:
        raise OSError(f"libhsattn ABI version {got}, expected {ABI_VERSION}")
    return lib


def _load() -> None:
    global _lib, _state, _error
    if _state != "unloaded":
        return
    with _lock:
        if _state != "unloaded":
            return
        if os.environ.get("HETEROSERVE_DISABLE_CUDA_KERNEL"):
            _state, _error = "unavailable", "disabled by HETEROSERVE_DISABLE_CUDA_KERNEL"
            return
        try:
            import torch
        except ImportError as exc:
            _state, _error = "unavailable", f"torch unavailable: {exc}"
            return
        if not torch.cuda.is_available():
            _state, _error = "unavailable", "no HIP device"
            return
        arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "").split(":")[0]
        if arch != "gfx950":
            _state, _error = "unavailable", (
                f"libhsattn.so is built for gfx950 only; device 0 is {arch or 'unknown'}")
            return
        path = lib_path()
        if not path.exists():
            _state, _error = "unavailable", (
                f"{path} is missing -- build it with python hetero-serve_amd/build.py")
            return
        try:
            _lib = open_library(path)
        except OSError as exc:
            _state, _error = "unavailable", f"OSError: {str(exc)[:200]}"
            return
        _state = "ready"


def ready() -> bool:
    _load()
    return _state == "ready"


def error() -> Optional[str]:
    _load()
    return _error


def lib(what: str = "paged attention HIP kernel") -> ctypes.CDLL:
    """The loaded library, or RuntimeError naming why it is unavailable."""
    _load()
    if _state != "ready":
        raise RuntimeError(f"{what} unavailable: {_error}")
    return _lib


def check(rc: int) -> None:
    if rc != 0:
        raise RuntimeError(_lib.hs_last_error().decode(errors="replace"))


# ---------------------------------------------------------------------------
# marshalling helpers
# ---------------------------------------------------------------------------

def dtype_code(dt) -> int:
    import torch

    codes = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}
    if dt not in codes:
        raise RuntimeError(f"unsupported KV cache dtype {dt} (float32, float16 or bfloat16)")
    return codes[dt]


def stream_of(device) -> int:
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def _int32_on(t, device):
    import torch

    if not torch.is_tensor(t):
        t = torch.as_tensor(t)
    return t.to(device=device, dtype=torch.int32).contiguous()


def _check_device(q, k_cache, v_cache) -> None:
    if not q.is_cuda:
        raise RuntimeError("q must be on CUDA")
    if not (k_cache.is_cuda and v_cache.is_cuda):
        raise RuntimeError("kv cache must be on CUDA")
    if k_cache.device != q.device or v_cache.device != q.device:
        raise RuntimeError("q and the kv cache must be on the same device")


def _check_q(q):
    import torch

    if q.dtype != torch.float32:
        raise RuntimeError(f"q must be float32, got {q.dtype}")
    return q.contiguous()


def _check_kv(k_cache, v_cache, D):
    if k_cache.dim() != 4:
        raise RuntimeError("k_cache must be [NB, BS, H, D]")
    if v_cache.shape != k_cache.shape:
        raise RuntimeError("v_cache must have the shape of k_cache")
    if k_cache.dtype != v_cache.dtype:
        raise RuntimeError("k_cache and v_cache must have the same dtype")
    if k_cache.shape[3] != D:
        raise RuntimeError(f"head_dim mismatch: q has {D}, cache has {k_cache.shape[3]}")
    return k_cache.contiguous(), v_cache.contiguous()


class _DeviceGuard:
    """Make `device` current for the duration of a library call."""

    def __init__(self, device):
        import torch

        self._torch = torch
        self._dev = device.index if device.index is not None else torch.cuda.current_device()
        self._prev = None

    def __enter__(self):
        cur = self._torch.cuda.current_device()
        if cur != self._dev:
            self._prev = cur
            self._torch.cuda.set_device(self._dev)

    def __exit__(self, *exc):
        if self._prev is not None:
            self._torch.cuda.set_device(self._prev)


def decode(q, k_cache, v_cache, block_tables, context_lens, scale: float,
           num_splits: int, partition_tokens: int = 0, shared_pages: bool = False):
    """out[B, H, D] fp32 = paged decode attention via hs_decode.

    shared_pages=True (fixed partitions only, num_splits == 0) runs
    hs_decode_shared: partitions whose block ids several sequences share are
    read once for all of them."""
    import torch

    L = lib()
    _check_device(q, k_cache, v_cache)
    if q.dim() != 3:
        raise RuntimeError("q must be [B, H, D]")
    q = _check_q(q)
    B, H, D = q.shape
    k_cache, v_cache = _check_kv(k_cache, v_cache, D)
    NB, BS, Hkv, _ = k_cache.shape
    bt = _int32_on(block_tables, q.device)
    ctx = _int32_on(context_lens, q.device)
    if bt.dim() != 2 or bt.shape[0] != B:
        raise RuntimeError("block_tables must be [B, max_blocks]")
    if ctx.numel() != B:
        raise RuntimeError("context_lens must have one entry per sequence")
    MB = bt.shape[1]
    out = torch.empty((B, H, D), dtype=torch.float32, device=q.device)
    if B == 0:
        return out
    if shared_pages and int(num_splits) != 0:
        raise RuntimeError("shared_pages needs fixed partitions (num_splits == 0)")
    if shared_pages:
        ws_bytes = L.hs_decode_shared_workspace_bytes(B, H, Hkv, D, BS, max(MB, 1),
                                                      int(partition_tokens))
    else:
        ws_bytes = L.hs_decode_workspace_bytes(B, H, Hkv, D, BS, max(MB, 1), int(num_splits),
                                               int(partition_tokens))
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    wsp = ws.data_ptr() if ws is not None else None
    with _DeviceGuard(q.device):
        if shared_pages:
            check(L.hs_decode_shared(
                q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), dtype_code(k_cache.dtype),
                NB, bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), B, H, Hkv, D, BS, MB,
                float(scale), int(partition_tokens), wsp, ws_bytes, stream_of(q.device)))
        else:
            check(L.hs_decode(
                q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), dtype_code(k_cache.dtype),
                NB, bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), B, H, Hkv, D, BS, MB,
                float(scale), int(num_splits), int(partition_tokens), wsp, ws_bytes,
                stream_of(q.device)))
    return out


def _prefill_workspace(L, B: int, rows: int, H: int, D: int, use_mfma: bool, split: bool,
                       device):
    """(tensor or None, bytes): the key-range split's scratch, when it applies."""
    import torch

    nbytes = L.hs_prefill_workspace_bytes(B, rows, H, D, int(bool(use_mfma))) if split else 0
    if not nbytes:
        return None, 0
    return torch.empty(nbytes, dtype=torch.uint8, device=device), nbytes


def prefill(q, k_cache, v_cache, block_tables, context_lens, scale: float, use_mfma: bool,
            split: bool = True):
    """out[B, S, H, D] fp32 = causal chunked prefill via hs_prefill.

    split=False passes no workspace, so the matrix-core kernel runs without
    the key-range split (for tests of that launch shape)."""
    import torch

    L = lib()
    _check_device(q, k_cache, v_cache)
    if q.dim() != 4:
        raise RuntimeError("q must be [B, S, H, D]")
    q = _check_q(q)
    B, S, H, D = q.shape
    k_cache, v_cache = _check_kv(k_cache, v_cache, D)
    NB, BS, Hkv, _ = k_cache.shape
    bt = _int32_on(block_tables, q.device)
    ctx = _int32_on(context_lens, q.device)
    if bt.dim() != 2 or bt.shape[0] != B:
        raise RuntimeError("block_tables must be [B, max_blocks]")
    if ctx.numel() != B:
        raise RuntimeError("context_lens must have one entry per sequence")
    out = torch.empty((B, S, H, D), dtype=torch.float32, device=q.device)
    if B == 0 or S == 0:
        return out
    with _DeviceGuard(q.device):
        ws, ws_bytes = _prefill_workspace(L, B, S, H, D, use_mfma, split, q.device)
        check(L.hs_prefill(
            q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), dtype_code(k_cache.dtype),
            NB, bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), B, S, H, Hkv, D, BS,
            bt.shape[1], float(scale), int(bool(use_mfma)),
            ws.data_ptr() if ws is not None else None, ws_bytes, stream_of(q.device)))
    return out


def prefill_varlen(q, cu_seqlens_q, max_seqlen_q: int, k_cache, v_cache, block_tables,
                   context_lens, scale: float, use_mfma: bool, split: bool = True):
    """out[T, H, D] fp32 for ragged chunks via hs_prefill_varlen (split as for
    prefill)."""
    import torch

    L = lib()
    _check_device(q, k_cache, v_cache)
    if q.dim() != 3:
        raise RuntimeError("q must be [total_tokens, H, D]")
    q = _check_q(q)
    T, H, D = q.shape
    k_cache, v_cache = _check_kv(k_cache, v_cache, D)
    NB, BS, Hkv, _ = k_cache.shape
    bt = _int32_on(block_tables, q.device)
    ctx = _int32_on(context_lens, q.device)
    cu = _int32_on(cu_seqlens_q, q.device)
    B = bt.shape[0]
    if cu.numel() != B + 1 or ctx.numel() != B:
        raise RuntimeError("cu_seqlens_q must be [B + 1] and context_lens [B]")
    out = torch.empty((T, H, D), dtype=torch.float32, device=q.device)
    if B == 0 or T == 0:
        return out
    with _DeviceGuard(q.device):
        ws, ws_bytes = _prefill_workspace(L, B, int(max_seqlen_q), H, D, use_mfma, split,
                                          q.device)
        check(L.hs_prefill_varlen(
            q.data_ptr(), cu.data_ptr(), int(max_seqlen_q), k_cache.data_ptr(),
            v_cache.data_ptr(), dtype_code(k_cache.dtype), NB, bt.data_ptr(), ctx.data_ptr(),
            out.data_ptr(), B, H, Hkv, D, BS, bt.shape[1], float(scale),
            int(bool(use_mfma)), ws.data_ptr() if ws is not None else None, ws_bytes,
            stream_of(q.device)))
    return out


def choose_num_splits(num_seqs: int, num_heads: int, max_context: int) -> int:
    L = lib("v3 kernel")
    s = L.hs_choose_num_splits(int(num_seqs), int(num_heads), int(max_context))
    if s < 0:
        raise RuntimeError(L.hs_last_error().decode(errors="replace"))
    return int(s)


def kv_pack(pool, ids_dev, out) -> None:
    """out[n, L, 2, page] = pool[L, 2, NB, page][:, :, ids]  (bitwise)."""
    L = lib("KV pack HIP kernel")
    Ls, _, NB = pool.shape[:3]
    page = pool[0, 0, 0].numel() * pool.element_size()
    with _DeviceGuard(pool.device):
        check(L.hs_kv_pack(pool.data_ptr(), Ls, NB, page, ids_dev.data_ptr(), ids_dev.numel(),
                           out.data_ptr(), stream_of(pool.device)))


def kv_unpack(pool, ids_dev, src) -> None:
    """pool[:, :, ids[i]] = src[i]  (bitwise; ids must not repeat)."""
    L = lib("KV unpack HIP kernel")
    Ls, _, NB = pool.shape[:3]
    page = pool[0, 0, 0].numel() * pool.element_size()
    with _DeviceGuard(pool.device):
        check(L.hs_kv_unpack(pool.data_ptr(), Ls, NB, page, ids_dev.data_ptr(),
                             ids_dev.numel(), src.data_ptr(), stream_of(pool.device)))


def kv_gather(cache, block_tables_dev, length: int, out) -> None:
    """out[B, length, Hkv, D] = cache[NB, BS, Hkv, D] gathered through the tables."""
    L = lib("KV gather HIP kernel")
    NB, BS = cache.shape[:2]
    row = cache[0, 0].numel() * cache.element_size()
    B, MB = block_tables_dev.shape
    with _DeviceGuard(cache.device):
        check(L.hs_kv_gather(cache.data_ptr(), NB, BS, row, block_tables_dev.data_ptr(), MB,
                             B, int(length), out.data_ptr(), stream_of(cache.device)))


def _rows(x, Hkv: int, D: int):
    """(tensor, row stride in elements) of new K or V rows [n, Hkv, D].

    Accepts [n, Hkv, D] or [n, Hkv * D]; the rows may be strided (a slice of
    the fused QKV output) but each row's Hkv * D elements must be contiguous.
    """
    if x.dim() == 3:
        if tuple(x.shape[1:]) != (Hkv, D):
            raise RuntimeError(f"K/V rows must be [n, {Hkv}, {D}], got {tuple(x.shape)}")
        row_ok = x.stride(2) == 1 and x.stride(1) == D
    elif x.dim() == 2:
        if x.shape[1] != Hkv * D:
            raise RuntimeError(f"K/V rows must be [n, {Hkv * D}], got {tuple(x.shape)}")
        row_ok = x.stride(1) == 1
    else:
        raise RuntimeError(f"K/V rows must be [n, Hkv, D], got {tuple(x.shape)}")
    if not row_ok:
        x = x.contiguous()
    stride = x.stride(0) if x.shape[0] > 1 else Hkv * D
    return x, stride


def _check_write(k_cache, v_cache, k, v):
    """The caches are written in place: CUDA, contiguous, same shape/dtype."""
    if k_cache.dim() != 4:
        raise RuntimeError("k_cache must be [NB, BS, Hkv, D]")
    if v_cache.shape != k_cache.shape or v_cache.dtype != k_cache.dtype:
        raise RuntimeError("k_cache and v_cache must have the same shape and dtype")
    if not (k_cache.is_cuda and v_cache.is_cuda and k.is_cuda and v.is_cuda):
        raise RuntimeError("kv cache and new rows must be on CUDA")
    if len({k_cache.device, v_cache.device, k.device, v.device}) != 1:
        raise RuntimeError("kv cache and new rows must be on the same device")
    if not (k_cache.is_contiguous() and v_cache.is_contiguous()):
        raise RuntimeError("kv cache must be contiguous (it is written in place)")


def _same_rows(k, v, Hkv: int, D: int):
    k, ks = _rows(k, Hkv, D)
    v, vs = _rows(v, Hkv, D)
    if k.shape[0] != v.shape[0] or k.dtype != v.dtype:
        raise RuntimeError("k and v rows must have the same count and dtype")
    if ks != vs:
        k, v = k.contiguous(), v.contiguous()
        ks = vs = Hkv * D
    return k, v, ks


def kv_scatter(k_cache, v_cache, slots, k, v) -> None:
    """k_cache.view(-1, Hkv, D)[slots] = k.to(cache dtype); same for v."""
    L = lib("KV scatter HIP kernel")
    _check_write(k_cache, v_cache, k, v)
    NB, BS, Hkv, D = k_cache.shape
    k, v, stride = _same_rows(k, v, Hkv, D)
    n = k.shape[0]
    if slots.numel() != n:
        raise RuntimeError(f"{slots.numel()} slots for {n} rows")
    import torch

    slots = torch.as_tensor(slots).to(device=k_cache.device, dtype=torch.int64).contiguous()
    with _DeviceGuard(k_cache.device):
        check(L.hs_kv_scatter(k_cache.data_ptr(), v_cache.data_ptr(), dtype_code(k_cache.dtype),
                              NB * BS, Hkv, D, slots.data_ptr(), n, k.data_ptr(), v.data_ptr(),
                              dtype_code(k.dtype), stride, stream_of(k_cache.device)))


def kv_append(k_cache, v_cache, block_tables, positions, k, v, seq_ids=None) -> None:
    """Row i -> slot block_tables[s][pos // BS] * BS + pos % BS of sequence
    s = seq_ids[i] (or i), pos = positions[i]; cast as kv_scatter."""
    L = lib("KV append HIP kernel")
    _check_write(k_cache, v_cache, k, v)
    NB, BS, Hkv, D = k_cache.shape
    k, v, stride = _same_rows(k, v, Hkv, D)
    n = k.shape[0]
    dev = k_cache.device
    bt = _int32_on(block_tables, dev)
    pos = _int32_on(positions, dev)
    if pos.numel() != n:
        raise RuntimeError(f"{pos.numel()} positions for {n} rows")
    sid = None if seq_ids is None else _int32_on(seq_ids, dev)
    if sid is not None and sid.numel() != n:
        raise RuntimeError(f"{sid.numel()} sequence ids for {n} rows")
    if sid is None and n > bt.shape[0]:
        raise RuntimeError("without seq_ids, row i uses table row i: more rows than tables")
    with _DeviceGuard(dev):
        check(L.hs_kv_append(k_cache.data_ptr(), v_cache.data_ptr(), dtype_code(k_cache.dtype), NB,
                             BS, Hkv, D, bt.data_ptr(), bt.shape[0], bt.shape[1], pos.data_ptr(),
                             None if sid is None else sid.data_ptr(), n, k.data_ptr(),
                             v.data_ptr(), dtype_code(k.dtype), stride, stream_of(dev)))


def block_tables(packed_dev, B: int, width: int, out) -> None:
    """out[B, width] int32 from the packed [off[0..B], ids...] device buffer."""
    L = lib("block table HIP kernel")
    with _DeviceGuard(out.device):
        check(L.hs_block_tables(packed_dev.data_ptr(), B, width, out.data_ptr(),
                                stream_of(out.device)))
