"""KV-block migration pack/unpack and contiguous gather on the GPU.

The pool is hetero-serve's device KV tensor ``[L, 2, num_blocks, block_size,
n_kv_heads, head_dim]`` (heteroserve/kv/torch_blocks.py:48, layout from
heteroserve/kv/blocks.py:72-81).  A migration payload is
``[n, L, 2, block_size, n_kv_heads, head_dim]`` in the pool dtype, the wire
format both of the reference's transports carry.

    export_blocks_device  pool -> payload   torch_blocks.py:137-148
    write_blocks_device   payload -> pool   torch_blocks.py:150-154
    gather_kv_batch       pool layer -> [B, length, Hkv, D]   torch_blocks.py:125-135
    scatter_kv            new K/V rows -> their slots   torch_engine.py:239-240, :306-308
    append_kv             new K/V rows -> slots from block tables and positions
    write_kv              [L, H, T, D] K/V -> pool   torch_blocks.py:89-106
    block_table_tensor    tables -> [B, width] int32   torch_blocks.py:75-85

Each is one libhsattn launch (a bitwise page copy) instead of the reference's
advanced-index gather plus permute-copy, or its Python loop of one copy per
block.  Block ids follow torch indexing rules: negative ids count from the
end of the pool, and an id outside [-num_blocks, num_blocks) raises
IndexError before anything is launched.

``HipKVMixin`` carries these as methods, so the reference allocator picks them
up by inheritance:

    class TorchBlockAllocator(HipKVMixin, _ReferenceTorchBlockAllocator): ...
"""

from __future__ import annotations

from .. import _hip


def _normalise_ids(block_ids, num_blocks: int):
    """Block ids as an int64 numpy array, negatives wrapped as torch indexing
    does; the first id outside [-num_blocks, num_blocks) raises IndexError.
    Integer lists, arrays and tensors are converted in one numpy pass; other
    elements (floats, objects, values beyond int64) go through int() one by
    one, as torch's indexing would take them."""
    import numpy as np
    import torch

    ids = None
    try:
        if torch.is_tensor(block_ids):
            if not block_ids.is_floating_point() and not block_ids.is_complex():
                ids = block_ids.detach().to("cpu").reshape(-1).to(torch.int64).numpy()
        else:
            arr = np.asarray(block_ids).reshape(-1)
            if arr.dtype.kind in "ib" or (arr.dtype.kind == "u" and arr.dtype.itemsize < 8):
                ids = arr.astype(np.int64, copy=False)
    except (TypeError, ValueError, OverflowError):
        ids = None
    if ids is None:   # element by element
        if torch.is_tensor(block_ids):
            block_ids = block_ids.detach().to("cpu").reshape(-1).tolist()
        vals = [int(raw) for raw in block_ids]
        for i in vals:
            if not -num_blocks <= i < num_blocks:
                raise IndexError(
                    f"index {i} is out of bounds for dimension 2 with size {num_blocks}")
        ids = np.array(vals, dtype=np.int64)
    bad = (ids < -num_blocks) | (ids >= num_blocks)
    if bad.any():
        i = int(ids[int(np.argmax(bad))])
        raise IndexError(f"index {i} is out of bounds for dimension 2 with size {num_blocks}")
    return np.where(ids < 0, ids + num_blocks, ids)


def _ids_tensor(ids, device):
    import numpy as np
    import torch

    return torch.from_numpy(np.ascontiguousarray(ids, dtype=np.int64)).to(device)


def _check_pool(pool) -> None:
    if pool.dim() != 6 or pool.shape[1] != 2:
        raise RuntimeError("pool must be [L, 2, num_blocks, block_size, n_kv_heads, head_dim]")
    if not pool.is_contiguous():
        raise RuntimeError("pool must be contiguous")
    if not pool.is_cuda:
        raise RuntimeError("pool must be on CUDA")


def export_blocks_device(pool, block_ids):
    """pool[:, :, ids].permute(2, 0, 1, 3, 4, 5).contiguous(), bit for bit."""
    import torch

    _hip.lib("KV pack HIP kernel")
    _check_pool(pool)
    ids = _normalise_ids(block_ids, pool.shape[2])
    L, _, _, BS, H, D = pool.shape
    out = torch.empty((len(ids), L, 2, BS, H, D), dtype=pool.dtype, device=pool.device)
    if len(ids):
        _hip.kv_pack(pool, _ids_tensor(ids, pool.device), out)
    return out


def write_blocks_device(pool, block_ids, payload) -> None:
    """pool[:, :, block_ids[i]] = payload[i] for every i, in one launch.

    The payload is converted to the pool's device and dtype first, as the
    reference's ``payload.to(device, dtype)`` does.  When an id repeats, the
    last payload entry for it wins, which is what the reference's sequential
    loop leaves behind.
    """
    import numpy as np
    import torch

    _hip.lib("KV unpack HIP kernel")
    _check_pool(pool)
    ids = _normalise_ids(block_ids, pool.shape[2])
    if not len(ids):
        return
    data = payload.to(device=pool.device, dtype=pool.dtype)
    block_shape = tuple(pool.shape[:2]) + tuple(pool.shape[3:])
    if data.dim() != 6 or tuple(data.shape[1:]) != block_shape or data.shape[0] < len(ids):
        raise RuntimeError(
            f"payload must be [n >= {len(ids)}, {', '.join(map(str, block_shape))}], "
            f"got {list(data.shape)}")
    n = len(ids)
    uniq, first_rev = np.unique(ids[::-1], return_index=True)
    if len(uniq) != n:  # duplicates: keep each block's final write, in write order
        last = np.sort(n - 1 - first_rev)
        ids = ids[last]
        data = data[torch.from_numpy(last).to(data.device)]
    data = data[: len(ids)].contiguous()
    _hip.kv_unpack(pool, _ids_tensor(ids, pool.device), data)


def gather_kv_batch(pool, tables, length: int, layer: int):
    """([B, length, Hkv, D], same for V): each sequence's first `length` tokens.

    tables is a list of per-sequence block-id lists, as the reference takes;
    every list must cover `length` tokens.
    """
    import numpy as np
    import torch

    _hip.lib("KV gather HIP kernel")
    _check_pool(pool)
    L, _, NB, BS, H, D = pool.shape
    if not 0 <= layer < L:
        raise IndexError(f"layer {layer} out of range for {L} layers")
    need = -(-int(length) // BS)
    rows = []
    for t in tables:
        ids = _normalise_ids(list(t)[:need], NB)
        if len(ids) < need:
            raise IndexError(
                f"block table of {len(ids)} blocks cannot hold {length} tokens")
        rows.append(ids)
    B = len(rows)
    k_out = torch.empty((B, length, H, D), dtype=pool.dtype, device=pool.device)
    v_out = torch.empty_like(k_out)
    if B == 0 or length == 0:
        return k_out, v_out
    bt = torch.from_numpy(np.stack(rows).astype(np.int32)).reshape(B, need).to(pool.device)
    _hip.kv_gather(pool[layer, 0], bt, length, k_out)
    _hip.kv_gather(pool[layer, 1], bt, length, v_out)
    return k_out, v_out


def slots_for(block_ids, positions, block_size: int):
    """Flat slots of absolute token positions through one block table
    (torch_blocks.py:68-73): ``table[pos // BS] * BS + pos % BS``, int64."""
    import torch

    tbl = torch.as_tensor(block_ids, dtype=torch.long)
    pos = torch.as_tensor(positions, dtype=torch.long)
    return tbl[pos // block_size] * block_size + (pos % block_size)


def scatter_kv(k_cache, v_cache, slots, k, v) -> None:
    """``fk[slots] = k.to(dtype); fv[slots] = v.to(dtype)`` for one layer's caches
    ``[NB, BS, Hkv, D]`` and new rows ``[n, Hkv, D]`` (torch_engine.py:239-240,
    :306-308), in one launch.  Rows may be a strided view such as a slice of
    the fused QKV output.  Negative slots count from the end, as in torch
    indexing.  Host slots (a list or CPU tensor) outside [-NB*BS, NB*BS) raise
    IndexError before the launch; device slots are not read back (that would
    stall the step), and a device slot out of range is not written.  Slots
    must not repeat (as in the engine: one token per slot per step).
    """
    import torch

    n_slots = k_cache.shape[0] * k_cache.shape[1]
    on_host = not (torch.is_tensor(slots) and slots.is_cuda)
    slots = torch.as_tensor(slots, dtype=torch.long)
    if on_host and slots.numel():
        lo, hi = int(slots.min()), int(slots.max())
        if lo < -n_slots or hi >= n_slots:
            bad = lo if lo < -n_slots else hi
            raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {n_slots}")
    slots = torch.where(slots < 0, slots + n_slots, slots)
    _hip.kv_scatter(k_cache, v_cache, slots, k, v)


def append_kv(k_cache, v_cache, block_tables, positions, k, v, seq_ids=None) -> None:
    """Write row i at absolute position ``positions[i]`` of sequence
    ``seq_ids[i]`` (row i of the tables when None), slots computed on the GPU
    from the int32 ``[B, MB]`` block tables.  Replaces the engine's
    per-sequence slot loop (torch_engine.py:221-227, a device-to-host copy per
    sequence) and the scatter after it.  Rows whose sequence id is outside
    ``[0, B)``, whose position is past the table or whose table entry is
    padding (-1) are not written.
    """
    _hip.kv_append(k_cache, v_cache, block_tables, positions, k, v, seq_ids)


def write_kv(pool, block_ids, start_pos: int, k, v) -> None:
    """``TorchBlockAllocator.write_kv`` (torch_blocks.py:89-106): scatter
    ``[L, Hkv, T, D]`` K/V of one sequence into every layer of the pool at
    positions ``start_pos .. start_pos + T - 1``; one launch per layer."""
    import torch

    _check_pool(pool)
    L, _, NB, BS, H, D = pool.shape
    k = torch.as_tensor(k, device=pool.device)
    v = torch.as_tensor(v, device=pool.device)
    T = int(k.shape[2])
    if T == 0:
        return
    slots = slots_for(block_ids, range(start_pos, start_pos + T), BS).to(pool.device)
    kt = k.permute(0, 2, 1, 3).contiguous()      # [L, T, H, D]: token-major rows
    vt = v.permute(0, 2, 1, 3).contiguous()
    for layer in range(L):
        scatter_kv(pool[layer, 0], pool[layer, 1], slots, kt[layer], vt[layer])


def block_table_tensor(tables, pad_to=None, device="cuda"):
    """``TorchBlockAllocator.block_table_tensor`` (torch_blocks.py:75-85): an
    int32 ``[len(tables), width]`` table, -1 padded, ``width = pad_to`` or the
    longest table (1 when there are no tables); longer tables are truncated.
    One host-to-device copy of all ids instead of one per sequence."""
    import array
    import itertools

    import numpy as np
    import torch

    if not isinstance(tables, (list, tuple)):
        tables = list(tables)
    width = pad_to or max((len(t) for t in tables), default=1)
    B = len(tables)
    out = torch.empty((B, width), dtype=torch.int32, device=device)
    if B == 0 or width == 0:
        return out
    # one conversion of all ids (the Python-int conversion is the host cost:
    # array.fromlist converts a list of ints ~3x faster than numpy does)
    lens = [min(len(t), width) for t in tables]
    ids = array.array("l" if array.array("l").itemsize == 8 else "q")
    try:
        for t in tables:
            ids.fromlist(t if type(t) is list and len(t) <= width else list(t)[:width])
        flat = np.frombuffer(ids, dtype=np.int64)
    except TypeError:   # ids that are not integers: numpy's conversion
        flat = np.array(list(itertools.chain.from_iterable(list(t)[:width] for t in tables)),
                        dtype=np.int64)
    except OverflowError:
        raise RuntimeError("value cannot be converted to type int32 without overflow") from None
    if flat.size and (flat.min() < -2 ** 31 or flat.max() >= 2 ** 31):
        raise RuntimeError("value cannot be converted to type int32 without overflow")
    off = np.zeros(B + 1, dtype=np.int64)
    np.cumsum(lens, out=off[1:])
    packed = torch.from_numpy(np.concatenate([off, flat]).astype(np.int32)).to(out.device)
    _hip.block_tables(packed, B, width, out)
    return out


class HipKVMixin:
    """GPU storage methods for hetero-serve's TorchBlockAllocator.

    Expects ``self.pool`` (the device pool), ``self.device`` and
    ``self.torch_dtype`` as TorchBlockAllocator defines them
    (torch_blocks.py:33-48).  Overrides the methods of torch_blocks.py:89-175
    that write or move KV pages.
    """

    def export_blocks_device(self, block_ids):
        return export_blocks_device(self.pool, block_ids)

    def write_blocks_device(self, block_ids, payload) -> None:
        write_blocks_device(self.pool, block_ids, payload)

    def export_blocks(self, block_ids):
        """Host copy of the payload (numpy), for the shaped-TCP transport."""
        return export_blocks_device(self.pool, block_ids).cpu().numpy()

    def write_blocks(self, block_ids, payload) -> None:
        import numpy as np
        import torch

        data = torch.as_tensor(np.ascontiguousarray(payload), dtype=self.torch_dtype,
                               device=self.device)
        write_blocks_device(self.pool, block_ids, data)

    def gather_kv_batch(self, tables, length: int, layer: int):
        return gather_kv_batch(self.pool, tables, length, layer)

    def write_kv(self, block_ids, start_pos, k, v) -> None:
        write_kv(self.pool, block_ids, start_pos, k, v)

    def block_table_tensor(self, tables, pad_to=None):
        return block_table_tensor(tables, pad_to, self.device)
