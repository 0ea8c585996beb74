"""Operands beyond fp16 range on the matrix-core paths.

The MFMA prefill feeds fp16 operands to the matrix cores.  A bf16 cache can
hold values fp16 cannot (|x| >= 65536 rounds to inf), and a large query
overflows fp16 once scaled.  The reference never meets this: its WMMA path
admits fp16 caches only (paged_attn_wmma.py:266-267, :372-387) and its torch
oracle computes in fp32 (paged_attn.py:255-298, paged_attn_prefill.py:281-322).
Here the prefill checks the operands it converts and recomputes an affected
unit in fp32, so the result must match the fp32 oracle.  The grouped-query
and shared-page decodes (split operands of the cache's own type, the query
scaled into range for fp16 caches) convert nothing and need no fallback;
their tests here check exactly that.

Tolerance, per element: 2e-3 * max(1, |oracle|) -- the north-star 2e-3
max-abs where outputs are O(1), 2e-3 relative where a planted V value makes
them large.  Planted values are placed so that no two large values meet in
one (sequence, head, dim), which would make the comparison one of
cancellation rather than of the kernels.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from oracle.attention import decode_one, prefill_one  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
BS = 16

BIG = [1e5, -1e5, 1e30, -1e30]


def _assert_close(got, want, what):
    got = got.detach().float().cpu()
    want = want.float()
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    err = (got - want).abs()
    tol = 2e-3 * torch.clamp(want.abs(), min=1.0)
    worst = (err / tol).max().item()
    assert worst <= 1.0, f"{what}: error {err.max().item():.3e} ({worst:.2f} x tolerance)"


def _tables(rng, lens, nb):
    perm = iter(rng.permutation(nb).tolist())
    return [[next(perm) for _ in range(-(-int(n) // BS))] for n in lens]


def _table_tensor(tables):
    width = max(len(t) for t in tables)
    bt = torch.full((len(tables), width), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return bt.to(DEV)


def _plant(cache, tables, lens, rng, n, seqs=None):
    """n values of BIG at distinct (sequence, KV head, dim) places inside the
    contexts of `seqs` (default: all sequences); returns the sequences hit."""
    hkv, d = cache.shape[2], cache.shape[3]
    seqs = list(range(len(lens))) if seqs is None else list(seqs)
    used, hit = set(), set()
    while len(used) < n:
        b = int(rng.choice(seqs))
        h, e = int(rng.integers(hkv)), int(rng.integers(d))
        if (b, h, e) in used:
            continue
        used.add((b, h, e))
        t = int(rng.integers(lens[b]))
        cache[tables[b][t // BS], t % BS, h, e] = BIG[len(used) % len(BIG)]
        hit.add(b)
    return hit


# ---------------------------------------------------------------------------
# prefill (prefill_mfma_kernel)
# ---------------------------------------------------------------------------


def _prefill_case(prefix, chunk, H, Hkv, D, dtype, seed):
    rng = np.random.default_rng(seed)
    lens = [int(p + s) for p, s in zip(prefix, chunk)]
    nb = sum(-(-n // BS) for n in lens) + 8
    tables = _tables(rng, lens, nb)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(dtype)
    vc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((sum(chunk), H, D), generator=gen, device=DEV)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(chunk)]), dtype=torch.int32, device=DEV)
    return rng, lens, tables, kc, vc, q, cu


def _prefill(q, cu, chunk, kc, vc, bt, ctx, scale, split):
    from heteroserve import _hip

    return _hip.prefill_varlen(q, cu, max(chunk), kc, vc, bt, ctx, scale, use_mfma=True,
                               split=split)


@pytest.mark.parametrize("target", ["K", "V", "KV", "Q"])
@pytest.mark.parametrize("D,split", [(128, False), (128, True), (64, False)])
def test_prefill_operands_beyond_fp16(target, D, split):
    """Planted bf16 values of 1e5 and 1e30 in K and/or V, or a query of 1e6,
    through the MFMA prefill with and without the key-range split: finite,
    and within tolerance of the fp32 oracle for every sequence."""
    prefix, chunk = [0, 300, 1000], [200, 77, 300]
    rng, lens, tables, kc, vc, q, cu = _prefill_case(prefix, chunk, 8, 4, D, torch.bfloat16,
                                                     seed=D + len(target))
    if "K" in target:
        _plant(kc, tables, lens, rng, 6)
    if "V" in target:
        _plant(vc, tables, lens, rng, 6)
    if target == "Q":
        for row in (0, 150, 260, 400):
            q[row, int(rng.integers(8)), int(rng.integers(D))] = 1e6
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = D ** -0.5
    got = _prefill(q, cu, chunk, kc, vc, bt, ctx, scale, split)
    c = cu.cpu().numpy()
    for b in range(len(lens)):
        want = prefill_one(q[c[b]:c[b + 1]].cpu(), kc.cpu(), vc.cpu(), bt[b].cpu(), lens[b],
                           scale)
        _assert_close(got[c[b]:c[b + 1]], want, f"{target} D{D} split={split} seq {b}")


def test_prefill_fp16_cache_with_large_query():
    """An fp16 cache cannot overflow, but a query can once scaled by
    scale * log2(e): the query check alone must catch it."""
    prefix, chunk = [100, 0], [90, 257]
    rng, lens, tables, kc, vc, q, cu = _prefill_case(prefix, chunk, 4, 4, 128, torch.float16, 3)
    q[5, 1, 7] = 2e6
    q[200, 3, 100] = -2e6
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    got = _prefill(q, cu, chunk, kc, vc, bt, ctx, 128 ** -0.5, False)
    c = cu.cpu().numpy()
    for b in range(2):
        want = prefill_one(q[c[b]:c[b + 1]].cpu(), kc.cpu(), vc.cpu(), bt[b].cpu(), lens[b],
                           128 ** -0.5)
        _assert_close(got[c[b]:c[b + 1]], want, f"seq {b}")


def test_prefill_range_fallback_is_local():
    """Only the workgroups that meet a large value recompute: a sequence with
    no planted value gives the same bits as on the clean cache, and values
    fp16 can hold (|x| <= 60000 in V) stay on the matrix-core path."""
    prefix, chunk = [0, 500], [300, 300]
    rng, lens, tables, kc, vc, q, cu = _prefill_case(prefix, chunk, 8, 8, 128, torch.bfloat16, 5)
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 128 ** -0.5
    clean = _prefill(q, cu, chunk, kc, vc, bt, ctx, scale, False)
    _plant(kc, tables, lens, rng, 4, seqs=[1])
    got = _prefill(q, cu, chunk, kc, vc, bt, ctx, scale, False)
    c = cu.cpu().numpy()
    assert torch.equal(got[c[0]:c[1]], clean[c[0]:c[1]])
    want = prefill_one(q[c[1]:c[2]].cpu(), kc.cpu(), vc.cpu(), bt[1].cpu(), lens[1], scale)
    _assert_close(got[c[1]:c[2]], want, "planted sequence")
    # in-range large V values: fast path, relative tolerance
    vc2 = vc.clone()
    vc2[tables[0][3], 5, 2, 17] = 60000.0
    got2 = _prefill(q, cu, chunk, kc, vc2, bt, ctx, scale, False)
    want0 = prefill_one(q[c[0]:c[1]].cpu(), kc.cpu(), vc2.cpu(), bt[0].cpu(), lens[0], scale)
    _assert_close(got2[c[0]:c[1]], want0, "in-range V")


def test_prefill_garbage_beyond_the_context():
    """Huge values in pool slots past a sequence's context (the tail of its
    last page) are read by the tile loop and masked: the output is the clean
    one's within tolerance (the check may send the unit to the fp32 path)."""
    prefix, chunk = [0], [100]           # 100 keys: slots 100..111 of page 6 unused
    rng, lens, tables, kc, vc, q, cu = _prefill_case(prefix, chunk, 4, 4, 64, torch.bfloat16, 6)
    kc[tables[0][6], 10, 1, 3] = 1e30
    vc[tables[0][6], 12, 2, 9] = -1e30
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    got = _prefill(q, cu, chunk, kc, vc, bt, ctx, 0.125, False)
    want = prefill_one(q.cpu(), kc.cpu(), vc.cpu(), bt[0].cpu(), lens[0], 0.125)
    _assert_close(got, want, "garbage past ctx")


# ---------------------------------------------------------------------------
# grouped-query decode on the matrix cores (splitmm_part_kernel)
# ---------------------------------------------------------------------------


def _decode_case(lens, H, Hkv, D, dtype, seed):
    rng = np.random.default_rng(seed)
    nb = sum(-(-n // BS) for n in lens) + 8
    tables = _tables(rng, lens, nb)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(dtype)
    vc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((len(lens), H, D), generator=gen, device=DEV)
    return rng, tables, kc, vc, q


def _decode_oracle(q, kc, vc, bt, lens, scale, b):
    return decode_one(q[b].cpu(), kc.cpu(), vc.cpu(), bt[b].cpu(), lens[b], scale)


@pytest.mark.parametrize("target", ["K", "V", "KV", "Q"])
@pytest.mark.parametrize("H,Hkv,D", [(32, 4, 128), (32, 1, 128), (16, 2, 64), (16, 2, 32)])
def test_gqa_decode_operands_beyond_fp16(target, H, Hkv, D):
    """8 to 32 query heads per KV head (the matrix-core decode, head dims 32,
    64 and 128) with planted bf16 values or a 1e6 query: every sequence within
    tolerance of the fp32 oracle, for one-partition rows (direct output) and
    multi-partition rows (partition states and the merge)."""
    from heteroserve.model import paged_attn

    lens = [40, 511, 700, 1500, 3000]
    rng, tables, kc, vc, q = _decode_case(lens, H, Hkv, D, torch.bfloat16, seed=H + D)
    if "K" in target:
        _plant(kc, tables, lens, rng, 6)
    if "V" in target:
        _plant(vc, tables, lens, rng, 6)
    if target == "Q":
        for b in (0, 2, 4):
            q[b, int(rng.integers(H)), int(rng.integers(D))] = 1e6
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = D ** -0.5
    got = paged_attn.paged_attention(q, kc, vc, bt, ctx, scale)
    for b in range(len(lens)):
        _assert_close(got[b], _decode_oracle(q, kc, vc, bt, lens, scale, b),
                      f"{target} H{H}/{Hkv} D{D} seq {b}")


# ---------------------------------------------------------------------------
# split-operand matrix-core decode (splitmm_part_kernel)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H,Hkv,D", [(8, 4, 128), (32, 4, 128), (48, 2, 64)])
def test_split_decode_query_and_cache_range(H, Hkv, D, dtype):
    """2 to 24 query heads per KV head on 16-bit caches (the split-operand
    decode, no fallback): heads scaled by 1e-30 .. 1e20 -- far outside fp16
    either way once multiplied by scale * log2(e) -- side by side in one KV
    group, and cache values up to 6e4 in K and V.  For fp16 each head's query
    is brought into range by a power of two before it is split, so every
    sequence must match the fp32 oracle to 2e-5 * max(1, |oracle|) (fp16) or
    5e-5 (bf16), far inside the 2e-3 of the paths above.

    The factors give either near-uniform or one-hot attention.  In between
    (a factor of 300 puts scores near 400, and two tokens can share the
    weight) any fp32 evaluation is off by some 1e-5: measured on such a head,
    the fp32 oracle was 4.1e-5 from an fp64 evaluation and this kernel
    2.2e-5, so such heads would test the oracle's rounding, not the kernel."""
    from heteroserve import _hip
    from heteroserve.model import paged_attn

    lens = [40, 511, 700, 1500, 3000]
    rng, tables, kc, vc, q = _decode_case(lens, H, Hkv, D, dtype, seed=H + D + 7)
    factors = [1.0, 1e6, 1e-7, 1e-30, 1e20, 0.01]
    for h in range(H):
        q[:, h] *= factors[h % len(factors)]
    for cache in (kc, vc):
        for b, t in [(1, 77), (3, 1000), (4, 2999)]:
            cache[tables[b][t // BS], t % BS, int(rng.integers(Hkv)), int(rng.integers(D))] = \
                float(rng.choice([6e4, -6e4]))
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = D ** -0.5
    tol = 2e-5 if dtype == torch.float16 else 5e-5
    for pt in (0, 16, 1024):
        got = _hip.decode(q, kc, vc, bt, ctx, scale, 0, partition_tokens=pt).cpu()
        assert torch.isfinite(got).all()
        for b in range(len(lens)):
            want = _decode_oracle(q, kc, vc, bt, lens, scale, b)
            err = (got[b] - want).abs() / torch.clamp(want.abs(), min=1.0)
            assert err.max().item() <= tol, (dtype, H, Hkv, D, pt, b, err.max().item())
    assert torch.isfinite(paged_attn.paged_attention(q, kc, vc, bt, ctx, scale)).all()


# ---------------------------------------------------------------------------
# shared pages (shared_pages_kernel)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("H,Hkv,D", [(8, 8, 128), (32, 4, 128), (16, 4, 64)])
def test_shared_pages_operands_beyond_fp16(H, Hkv, D):
    """A shared prefix page holding 1e30 goes through the shared-page kernel's
    split-operand products as stored (bf16 operands, fp32 accumulation);
    every sequence against the fp32 oracle.  A large value in a private page
    goes through the partition kernel's own path."""
    from heteroserve import _hip

    rng = np.random.default_rng(H + Hkv + D)
    lens = [1100 + 37 * i for i in range(10)] + [600, 2500]
    nb = sum(-(-n // BS) for n in lens) + 16
    perm = iter(rng.permutation(nb).tolist())
    prefix = [next(perm) for _ in range(64)]            # 1024 shared tokens
    tables = []
    for b, n in enumerate(lens):
        t = list(prefix) if b < 10 else []
        t = t[:-(-n // BS)]
        while len(t) < -(-n // BS):
            t.append(next(perm))
        tables.append(t)
    gen = torch.Generator(device=DEV).manual_seed(H * D)
    kc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(torch.bfloat16)
    vc = torch.randn((nb, BS, Hkv, D), generator=gen, device=DEV).to(torch.bfloat16)
    q = torch.randn((len(lens), H, D), generator=gen, device=DEV)
    kc[prefix[7], 3, Hkv - 1, 5] = 1e30          # shared K
    vc[prefix[40], 9, 0, D - 1] = -1e30          # shared V
    vc[tables[11][100], 2, 0, 1] = 1e5           # private V
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = D ** -0.5
    got = _hip.decode(q, kc, vc, bt, ctx, scale, num_splits=0, shared_pages=True)
    plain = _hip.decode(q, kc, vc, bt, ctx, scale, num_splits=0)
    for b in range(len(lens)):
        want = _decode_oracle(q, kc, vc, bt, lens, scale, b)
        _assert_close(got[b], want, f"shared H{H}/{Hkv} D{D} seq {b}")
        _assert_close(plain[b], want, f"plain H{H}/{Hkv} D{D} seq {b}")


# ---------------------------------------------------------------------------
# the fp32 paths take large values as they are
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("G", [1, 2, 4])
def test_valu_decode_with_large_values(G):
    """The VALU decode kernel computes in fp32 from the bf16 cache: planted
    values need no fallback and match the oracle (v1, v2 and v3 entry points)."""
    from heteroserve.model import paged_attn, paged_attn_v2, paged_attn_v3

    lens = [33, 512, 1700]
    rng, tables, kc, vc, q = _decode_case(lens, 8, 8 // G, 128, torch.bfloat16, seed=G)
    _plant(kc, tables, lens, rng, 4)
    _plant(vc, tables, lens, rng, 4)
    bt = _table_tensor(tables)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    scale = 128 ** -0.5
    for got in (paged_attn.paged_attention(q, kc, vc, bt, ctx, scale),
                paged_attn_v2.paged_attention_v2(q, kc, vc, bt, ctx, scale),
                paged_attn_v3.paged_attention_v3(q, kc, vc, bt, ctx, scale, 5)):
        for b in range(len(lens)):
            _assert_close(got[b], _decode_oracle(q, kc, vc, bt, lens, scale, b), f"G{G} seq {b}")
