"""GPU parity of KV-block pack / unpack / gather: bit-exact against the oracle.

Restates the migration tests of the reference (tests/test_model.py:106-124,
tests/test_torch_engine.py:127-142) on libhsattn, and runs the 4096-block
pack of the C5 configuration at full size.  Every comparison is byte
equality (fp data compared through an integer view, so NaN payloads and
signed zeros count too).
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from _refcases import pack_case  # noqa: E402
from oracle.kvpack import export_blocks, gather_kv_batch, write_blocks  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    """Integer view of a tensor's bytes (host numpy)."""
    t = t.detach().contiguous().cpu()
    width = {1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()]
    return t.view(width).numpy()


def _np_bits(a: np.ndarray):
    return a.view({1: np.uint8, 2: np.int16, 4: np.int32, 8: np.int64}[a.itemsize])


def _pack():
    from heteroserve.kv import pack

    from heteroserve import _hip

    assert _hip.ready(), _hip.error()
    return pack


def test_reference_migration_roundtrip():
    """tests/test_model.py:106-124 on the GPU: export the sequence's blocks,
    import them into a second pool, gather them back: K and V unchanged."""
    pk = _pack()
    c = pack_case()
    src = torch.as_tensor(c["pool"], device=DEV)
    payload = pk.export_blocks_device(src, c["ids"])
    np.testing.assert_array_equal(_bits(payload), _np_bits(export_blocks(c["pool"], c["ids"])))

    dst = torch.zeros_like(src)
    new_ids = [5, 9, 2, 14]                  # any free blocks of the receiver
    pk.write_blocks_device(dst, new_ids, payload)
    gk, gv = pk.gather_kv_batch(dst, [new_ids], 16, layer=0)
    want_k = c["k"][0].transpose(1, 0, 2)     # [T, H, D]
    want_v = c["v"][0].transpose(1, 0, 2)
    np.testing.assert_array_equal(_bits(gk[0]), _np_bits(np.ascontiguousarray(want_k)))
    np.testing.assert_array_equal(_bits(gv[0]), _np_bits(np.ascontiguousarray(want_v)))
    for layer in range(4):
        gk, gv = pk.gather_kv_batch(dst, [new_ids], 16, layer=layer)
        np.testing.assert_array_equal(
            _bits(gk[0]), _np_bits(np.ascontiguousarray(c["k"][layer].transpose(1, 0, 2))))


@pytest.mark.parametrize("dtype,shape", [
    (torch.float16, (3, 2, 40, 16, 4, 64)),     # page 8 KiB
    (torch.bfloat16, (1, 2, 70, 16, 32, 128)),  # page 128 KiB (C5 geometry)
    (torch.float32, (2, 2, 33, 8, 4, 64)),
    (torch.uint8, (2, 2, 17, 3, 5, 7)),         # page 105 B: byte-granular kernel
])
def test_pack_unpack_match_oracle(dtype, shape):
    pk = _pack()
    gen = torch.Generator(device=DEV).manual_seed(sum(shape))
    if dtype == torch.uint8:
        pool = torch.randint(0, 256, shape, generator=gen, device=DEV, dtype=torch.uint8)
    else:
        pool = torch.randn(shape, generator=gen, device=DEV).to(dtype)
    nb = shape[2]
    rng = np.random.default_rng(nb)
    ids = rng.choice(nb, size=nb // 2, replace=False).tolist()
    ids[0] = -1                                  # negative ids wrap like torch indexing
    host = pool.cpu()
    host_np = host.view(torch.int16).numpy() if dtype == torch.bfloat16 else host.numpy()
    payload = pk.export_blocks_device(pool, ids)
    np.testing.assert_array_equal(_bits(payload), _np_bits(export_blocks(host_np, ids)))

    # unpack into other blocks, with one repeated id (the later payload wins)
    dst_ids = rng.choice(nb, size=len(ids), replace=False).tolist()
    dst_ids[-1] = dst_ids[0]
    dst = torch.zeros_like(pool)
    pk.write_blocks_device(dst, dst_ids, payload)
    want = np.zeros_like(host_np)
    write_blocks(want, dst_ids, _np_bits(export_blocks(host_np, ids)).view(want.dtype))
    np.testing.assert_array_equal(_bits(dst), _np_bits(want))


def test_gather_matches_oracle():
    pk = _pack()
    gen = torch.Generator(device=DEV).manual_seed(3)
    pool = torch.randn((2, 2, 64, 16, 4, 64), generator=gen, device=DEV).half()
    rng = np.random.default_rng(3)
    perm = rng.permutation(64).tolist()
    tables = [perm[0:10], perm[10:30], perm[30:35]]
    host = pool.cpu().numpy()
    for layer in (0, 1):
        for length in (1, 16, 77):
            if any(len(t) * 16 < length for t in tables):
                continue
            gk, gv = pk.gather_kv_batch(pool, tables, length, layer)
            wk, wv = gather_kv_batch(host, tables, length, layer)
            np.testing.assert_array_equal(_bits(gk), _np_bits(wk))
            np.testing.assert_array_equal(_bits(gv), _np_bits(wv))
    with pytest.raises(IndexError):
        pk.gather_kv_batch(pool, tables, 100, 0)


def test_bad_ids_raise_before_launch():
    pk = _pack()
    pool = torch.zeros((1, 2, 8, 16, 2, 64), device=DEV, dtype=torch.float16)
    with pytest.raises(IndexError):
        pk.export_blocks_device(pool, [0, 8])
    with pytest.raises(IndexError):
        pk.write_blocks_device(pool, [-9], torch.zeros((1, 1, 2, 16, 2, 64), device=DEV))
    assert pk.export_blocks_device(pool, []).shape == (0, 1, 2, 16, 2, 64)


def test_c5_pack_4096_blocks_bit_exact():
    """C5's migration pack: 4096 random blocks of a 65536-block bf16 pool
    (1 GiB payload) against torch's own gather + permute on the device, then
    unpacked into a second pool region and packed again (a round trip)."""
    from hsbench import cases

    pk = _pack()
    nb = cases.C5_POOL_BLOCKS
    pool = torch.empty((1, 2, nb, 16, 32, 128), dtype=torch.bfloat16, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(41)
    cases._fill_pool(pool, gen)
    ids = cases.c5_pack_ids(nb)
    payload = pk.export_blocks_device(pool, ids)
    idx = torch.as_tensor(ids, device=DEV)
    want = pool[:, :, idx].permute(2, 0, 1, 3, 4, 5).contiguous()
    assert torch.equal(payload.view(torch.int16), want.view(torch.int16))
    del want
    # spot check against the numpy oracle on a few blocks
    for i in (0, 1234, 4095):
        blk = pool[:, :, ids[i]].cpu().view(torch.int16).numpy()
        np.testing.assert_array_equal(_bits(payload[i]), blk)
    # round trip through other blocks
    rng = np.random.default_rng(42)
    others = rng.choice(nb, size=4096, replace=False).tolist()
    pk.write_blocks_device(pool, others, payload)
    again = pk.export_blocks_device(pool, others)
    assert torch.equal(again.view(torch.int16), payload.view(torch.int16))
