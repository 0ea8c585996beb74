"""Pins of the CPU oracle (oracle/) -- CPU only.

The oracle is what every GPU parity test trusts, so each of its functions is
checked here against something that does not restate it:

* fp64 dense brute force (tests/_dense.py) on the reference test suite's own
  parameter sets and RNG streams (tests/_refcases.py);
* closed forms: q = 0 gives the mean of V, a constant V gives that constant,
  a one-key context gives that key's value, a dominant score selects its
  value;
* invariances: physical block layout, padding entries past the context, GQA
  versus duplicated MHA heads, one-query prefill versus decode, split counts;
* explicit index loops for the pack permutation;
* known answers the reference records for its split heuristic (README:336,
  :346: 16 splits at B16/ctx512 and 64 at B32/ctx2048 on a 40-SM T4).

The last section plants plausible mistakes in copies of the oracle (an
off-by-one causal bound, a wrong GQA head, a dropped scale, a floor instead
of a ceiling, transposed pack axes) and asserts that these same checks catch
every one of them.
"""

from __future__ import annotations

import inspect
import types

import numpy as np
import pytest

torch = pytest.importorskip("torch")

import oracle.attention as att  # noqa: E402
import oracle.kvpack as kvp  # noqa: E402
import oracle.recurrences as rec  # noqa: E402
from _dense import dense_causal, dense_decode  # noqa: E402
from _refcases import (ONLINE_CASES, PREFILL_CASES, SPLIT_CASES, WMMA_TILING_CASES,  # noqa: E402
                       build_paged_case, cpu_fuzz_trials, pack_case, prefill_case,
                       recurrence_case, single_head_case, table_array)
from oracle.splits import choose_num_splits  # noqa: E402


def _t(x):
    return torch.as_tensor(x)


# ---------------------------------------------------------------------------
# check functions (take the implementation, so planted mutants reuse them)
# ---------------------------------------------------------------------------


def check_decode_vs_dense(decode_fn, seed=5, lens=(9, 31, 16), tol=1e-4):
    c = build_paged_case(seed=seed, lens=lens)
    pool = _t(c["pool"])
    bt = _t(table_array(c["tables"]))
    got = decode_fn(_t(c["q"]), pool[0, 0], pool[0, 1], bt,
                    torch.tensor(c["lens"], dtype=torch.int32), c["scale"]).numpy()
    for b, (k, v) in enumerate(c["seqs"]):
        want = dense_decode(c["q"][b], k[0].transpose(1, 0, 2), v[0].transpose(1, 0, 2),
                            c["scale"])
        np.testing.assert_allclose(got[b], want, rtol=tol, atol=tol)


def check_prefill_vs_dense(prefill_fn, lens, S, kvh, tol=1e-4):
    c = prefill_case(lens, S, kvh, seed=len(lens) * 7 + S)
    pool = _t(c["pool"])
    bt = _t(table_array(c["tables"]))
    got = prefill_fn(_t(c["q"]), pool[0, 0], pool[0, 1], bt,
                     torch.tensor(lens, dtype=torch.int32), c["scale"]).numpy()
    for b, (k, v) in enumerate(c["seqs"]):
        want = dense_causal(c["q"][b], k[0].transpose(1, 0, 2), v[0].transpose(1, 0, 2),
                            c["scale"], lens[b] - S)
        np.testing.assert_allclose(got[b], want, rtol=tol, atol=tol,
                                   err_msg=f"sequence {b}, len {lens[b]}, S={S}")


def check_split_vs_dense(split_fn, n, splits, amp):
    q, k, v = recurrence_case(n * 31 + splits, n, amp)
    want = dense_decode(q, k, v, 1 / 8)
    np.testing.assert_allclose(split_fn(q, k, v, 1 / 8, splits), want, rtol=1e-4, atol=1e-4)


def check_tiled_vs_dense(tiled_fn, ctx, S, D):
    q, k, v = single_head_case(ctx, S, D)
    want = dense_causal(q[:, None], k[:, None], v[:, None], D ** -0.5, ctx - S)[:, 0]
    np.testing.assert_allclose(tiled_fn(q, k, v, D ** -0.5, ctx), want, rtol=1e-5, atol=1e-5)


def check_pack_by_loops(export_fn):
    rng = np.random.default_rng(0)
    pool = rng.integers(0, 1 << 15, size=(2, 2, 7, 3, 2, 5)).astype(np.int16)
    ids = [4, 0, 6, 4, -1]
    got = export_fn(pool, ids)
    assert got.shape == (5, 2, 2, 3, 2, 5)
    for i, blk in enumerate(ids):
        for l in range(2):
            for c in range(2):
                for t in range(3):
                    for h in range(2):
                        for d in range(5):
                            assert got[i, l, c, t, h, d] == pool[l, c, blk % 7, t, h, d]


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns, round to nearest even (non-NaN inputs)."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def check_slots_by_loop(slots_fn):
    rng = np.random.default_rng(3)
    for bs in (1, 4, 16):
        table = rng.permutation(40)[:9].tolist()
        pos = rng.integers(0, 9 * bs, size=25)
        got = slots_fn(table, pos, bs)
        for i, p_ in enumerate(pos):
            assert got[i] == table[p_ // bs] * bs + p_ % bs


def check_scatter_by_loops(scatter_fn):
    """Each written row equals its source row rounded independently (numpy's
    fp16 cast, the bf16 bit formula); rows not written stay zero."""
    rng = np.random.default_rng(4)
    nb, bs, h, d = 5, 4, 3, 8
    src = (rng.standard_normal((7, h, d)) * 3).astype(np.float32)
    src[0, 0, :6] = [np.inf, -np.inf, 65520.0, 65519.0, 1e-8, -3e-5]   # fp16 edges
    src[1, 0, 0] = np.float32(1.0) + np.float32(2 ** -8)               # a bf16 tie
    slots = rng.permutation(nb * bs)[:7]
    for dt in (torch.float32, torch.float16, torch.bfloat16):
        cache = torch.zeros(nb, bs, h, d, dtype=dt)
        scatter_fn(cache, slots, torch.as_tensor(src))
        flat = cache.reshape(-1, h, d)
        written = set(int(x) for x in slots)
        for i, sl in enumerate(slots):
            row = flat[int(sl)]
            if dt == torch.float32:
                assert np.array_equal(row.numpy(), src[i])
            elif dt == torch.float16:
                with np.errstate(over="ignore"):          # 65520 rounds to inf, as intended
                    want = src[i].astype(np.float16)
                assert np.array_equal(row.numpy(), want)
            else:
                assert np.array_equal(row.view(torch.int16).numpy().view(np.uint16),
                                      bf16_bits(src[i]))
        for sl in range(nb * bs):
            if sl not in written:
                assert not flat[sl].any()


def check_write_kv_round_trip(write_fn):
    """write_kv, then a gather through the same table, returns the rows."""
    rng = np.random.default_rng(5)
    L, nb, bs, h, d = 2, 9, 4, 3, 8
    pool = torch.zeros(L, 2, nb, bs, h, d)
    table = [6, 1, 8, 3]
    k = torch.as_tensor(rng.standard_normal((L, h, 11, d)).astype(np.float32))
    v = torch.as_tensor(rng.standard_normal((L, h, 11, d)).astype(np.float32))
    write_fn(pool, table, 3, k, v)
    for layer in range(L):
        gk, gv = kvp.gather_kv_batch(pool.numpy(), [table], 14, layer)
        assert np.array_equal(gk[0, 3:], k[layer].permute(1, 0, 2).numpy())
        assert np.array_equal(gv[0, 3:], v[layer].permute(1, 0, 2).numpy())
        assert not gk[0, :3].any() and not gv[0, :3].any()


# ---------------------------------------------------------------------------
# the oracle against the mathematics
# ---------------------------------------------------------------------------


def test_decode_matches_dense_on_reference_cases():
    """tests/test_torch_engine.py:179-196 (seed 5) and :303-319 (seed 9)."""
    check_decode_vs_dense(att.paged_attention_torch, seed=5)
    check_decode_vs_dense(att.paged_attention_torch, seed=9)


def test_decode_fuzz_matches_dense():
    """tests/test_torch_engine.py:359-402: 40 random geometries, BS in {4,8,16}."""
    for c in cpu_fuzz_trials():
        pool = _t(c["pool"])
        got = att.paged_attention_torch(_t(c["q"]), pool[0, 0], pool[0, 1],
                                        _t(table_array(c["tables"])),
                                        torch.tensor(c["lens"], dtype=torch.int32),
                                        c["scale"]).numpy()
        for b, (k, v) in enumerate(c["seqs"]):
            want = dense_decode(c["q"][b], k[0].transpose(1, 0, 2), v[0].transpose(1, 0, 2),
                                c["scale"])
            np.testing.assert_allclose(got[b], want, rtol=1e-4, atol=1e-4,
                                       err_msg=f"trial {c['trial']} seq {b}")


@pytest.mark.parametrize("lens,S,kvh", PREFILL_CASES)
def test_prefill_matches_dense_causal(lens, S, kvh):
    """tests/test_torch_engine.py:518-546, including GQA, MQA and S = 1."""
    check_prefill_vs_dense(att.paged_attention_prefill_torch, lens, S, kvh)


@pytest.mark.parametrize("n,amp", ONLINE_CASES)
def test_online_softmax_matches_dense(n, amp):
    """tests/test_torch_engine.py:257-281 (amp 25 overflows a naive exp)."""
    q, k, v = recurrence_case(n, n, amp)
    np.testing.assert_allclose(rec.online_softmax_reference(q, k, v, 1 / 8),
                               dense_decode(q, k, v, 1 / 8), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("n,splits,amp", SPLIT_CASES)
def test_split_merge_matches_dense(n, splits, amp):
    """tests/test_torch_engine.py:327-356, incl. more splits than keys."""
    check_split_vs_dense(rec.split_merge_reference, n, splits, amp)


@pytest.mark.parametrize("ctx,S,D", WMMA_TILING_CASES)
def test_tiled_prefill_matches_dense(ctx, S, D):
    """tests/test_torch_engine.py:610-639: misaligned tiles, S == ctx, S = 1."""
    check_tiled_vs_dense(rec.tiled_prefill_reference, ctx, S, D)


def test_closed_forms():
    rng = np.random.default_rng(1)
    nb, bs, h, d = 12, 8, 3, 16
    pool = torch.as_tensor(rng.standard_normal((1, 2, nb, bs, h, d)).astype(np.float32))
    bt = torch.tensor([[3, 7, 1, -1], [0, 11, -1, -1]], dtype=torch.int32)
    ctx = torch.tensor([20, 9], dtype=torch.int32)
    flat_v = pool[0, 1].reshape(nb * bs, h, d)

    def seq_rows(b, n):
        return torch.stack([flat_v[int(bt[b, j // bs]) * bs + j % bs] for j in range(n)])

    # q = 0: uniform attention -> mean of V over the context
    out = att.paged_attention_torch(torch.zeros(2, h, d), pool[0, 0], pool[0, 1], bt, ctx, 0.3)
    for b in range(2):
        torch.testing.assert_close(out[b], seq_rows(b, int(ctx[b])).mean(0), rtol=1e-5, atol=1e-6)
    # constant V -> that constant, whatever q
    pool_c = pool.clone()
    pool_c[0, 1] = 2.5
    out = att.paged_attention_torch(torch.randn(2, h, d), pool_c[0, 0], pool_c[0, 1], bt, ctx, 0.3)
    torch.testing.assert_close(out, torch.full_like(out, 2.5))
    # one key -> its value
    one = torch.tensor([1, 1], dtype=torch.int32)
    out = att.paged_attention_torch(torch.randn(2, h, d), pool[0, 0], pool[0, 1], bt, one, 0.3)
    for b in range(2):
        torch.testing.assert_close(out[b], seq_rows(b, 1)[0])
    # a dominant score picks its value: q aligned with key 5 of sequence 0, huge scale
    flat_k = pool[0, 0].reshape(nb * bs, h, d)
    key5 = flat_k[int(bt[0, 0]) * bs + 5]
    out = att.paged_attention_torch(key5[None].clone(), pool[0, 0], pool[0, 1], bt[:1],
                                    ctx[:1], 1e4)
    torch.testing.assert_close(out[0], seq_rows(0, 6)[5], rtol=1e-4, atol=1e-4)
    # prefill with q = 0: row s is the mean of V over keys [0, pos_s]
    S = 4
    outp = att.paged_attention_prefill_torch(torch.zeros(2, S, h, d), pool[0, 0], pool[0, 1],
                                             bt, ctx, 0.3)
    for b in range(2):
        for s in range(S):
            pos = int(ctx[b]) - S + s
            torch.testing.assert_close(outp[b, s], seq_rows(b, pos + 1).mean(0),
                                       rtol=1e-5, atol=1e-6)


def test_layout_and_padding_invariance():
    """Physical block placement and table entries past the context do not
    change the result (bitwise: the same rows are gathered in the same order)."""
    c = build_paged_case(seed=13, lens=(5, 40, 17))
    pool = _t(c["pool"])
    bt = _t(table_array(c["tables"]))
    ctx = torch.tensor(c["lens"], dtype=torch.int32)
    q = _t(c["q"])
    base = att.paged_attention_torch(q, pool[0, 0], pool[0, 1], bt, ctx, c["scale"])
    perm = torch.randperm(pool.shape[2], generator=torch.Generator().manual_seed(0))
    inv = torch.argsort(perm)
    moved = pool[:, :, perm]                      # block x now lives at inv[x]
    bt2 = torch.where(bt >= 0, inv[bt.clamp(min=0).long()].int(), bt)
    got = att.paged_attention_torch(q, moved[0, 0], moved[0, 1], bt2, ctx, c["scale"])
    assert torch.equal(got, base)
    bt3 = bt.clone()
    bt3[bt3 < 0] = 7                              # junk past each context
    got = att.paged_attention_torch(q, pool[0, 0], pool[0, 1], bt3, ctx, c["scale"])
    assert torch.equal(got, base)


def test_gqa_equals_duplicated_mha_and_prefill_s1_equals_decode():
    c = prefill_case([40, 23], 1, n_kv_head=2, seed=3)
    pool = _t(c["pool"])
    bt = _t(table_array(c["tables"]))
    ctx = torch.tensor(c["lens"], dtype=torch.int32)
    q = _t(c["q"])                                # [B, 1, 4, D], 2 KV heads
    gqa = att.paged_attention_torch(q[:, 0], pool[0, 0], pool[0, 1], bt, ctx, c["scale"])
    dup = pool.repeat_interleave(2, dim=4)        # every KV head twice -> MHA
    mha = att.paged_attention_torch(q[:, 0], dup[0, 0], dup[0, 1], bt, ctx, c["scale"])
    torch.testing.assert_close(gqa, mha, rtol=0, atol=1e-6)
    pre = att.paged_attention_prefill_torch(q, pool[0, 0], pool[0, 1], bt, ctx, c["scale"])
    torch.testing.assert_close(pre[:, 0], gqa, rtol=1e-6, atol=1e-6)


def test_per_sequence_forms_match_batched():
    c = build_paged_case(seed=21, lens=(3, 64, 33))
    pool = _t(c["pool"])
    bt = _t(table_array(c["tables"]))
    ctx = torch.tensor(c["lens"], dtype=torch.int32)
    q = _t(c["q"])
    batched = att.paged_attention_torch(q, pool[0, 0], pool[0, 1], bt, ctx, c["scale"])
    for b in range(3):
        one = att.decode_one(q[b], pool[0, 0], pool[0, 1], bt[b], int(ctx[b]), c["scale"])
        torch.testing.assert_close(one, batched[b], rtol=1e-5, atol=1e-6)
    cp = prefill_case([37, 64, 19], 16, None, seed=2)
    pool = _t(cp["pool"])
    bt = _t(table_array(cp["tables"]))
    ctx = torch.tensor(cp["lens"], dtype=torch.int32)
    q = _t(cp["q"])
    batched = att.paged_attention_prefill_torch(q, pool[0, 0], pool[0, 1], bt, ctx, cp["scale"])
    for b in range(3):
        one = att.prefill_one(q[b], pool[0, 0], pool[0, 1], bt[b], int(ctx[b]), cp["scale"])
        torch.testing.assert_close(one, batched[b], rtol=1e-5, atol=1e-6)


def test_zero_context_and_padded_rows():
    """Reference semantics kept by the oracle: a decode row with no context is
    NaN (softmax over all -inf); prefill rows at negative positions are 0."""
    pool = torch.randn(1, 2, 4, 4, 2, 8)
    bt = torch.tensor([[0, 1]], dtype=torch.int32)
    out = att.paged_attention_torch(torch.randn(1, 2, 8), pool[0, 0], pool[0, 1], bt,
                                    torch.tensor([0], dtype=torch.int32), 0.3)
    assert torch.isnan(out).all()
    outp = att.paged_attention_prefill_torch(torch.randn(1, 6, 2, 8), pool[0, 0], pool[0, 1],
                                             bt, torch.tensor([4], dtype=torch.int32), 0.3)
    assert torch.all(outp[0, :2] == 0) and torch.isfinite(outp).all()


def test_pack_oracle():
    check_pack_by_loops(kvp.export_blocks)
    c = pack_case()                          # tests/test_model.py:106-124
    payload = kvp.export_blocks(c["pool"], c["ids"])
    dst = np.zeros_like(c["pool"])
    new_ids = [9, 2, 15, 4]
    kvp.write_blocks(dst, new_ids, payload)
    gk, gv = kvp.gather_kv_batch(dst, [new_ids], 16, 0)
    assert np.array_equal(gk[0], c["k"][0].transpose(1, 0, 2))
    assert np.array_equal(gv[0], c["v"][0].transpose(1, 0, 2))
    for layer in range(4):
        gk, _ = kvp.gather_kv_batch(dst, [new_ids], 16, layer)
        assert np.array_equal(gk[0], c["k"][layer].transpose(1, 0, 2))
    # repeated destination: the later payload entry wins
    dst = np.zeros_like(c["pool"])
    kvp.write_blocks(dst, [3, 3], payload[:2])
    assert np.array_equal(dst[:, :, 3], payload[1])


def test_pack_oracle_torch_forms():
    """The torch forms the benchmark times as CPU baselines (torch_blocks.py:
    137-154): the same explicit index loops as the numpy form, and the
    per-block unpack loop with a repeated id (a later payload entry wins)."""
    check_pack_by_loops(lambda pool, ids: kvp.export_blocks_torch(torch.from_numpy(pool),
                                                                  ids).numpy())
    rng = np.random.default_rng(4)
    pool = torch.from_numpy(rng.integers(-30000, 30000, size=(2, 2, 9, 4, 3, 6)).astype(np.int16))
    payload = torch.from_numpy(rng.integers(-30000, 30000, size=(4, 2, 2, 4, 3, 6))
                               .astype(np.int16))
    dst = pool.clone()
    ids = [7, 0, 7, 3]
    kvp.write_blocks_torch(dst, ids, payload)
    for blk in range(9):
        if blk in (0, 3, 7):
            i = max(j for j, x in enumerate(ids) if x == blk)
            assert torch.equal(dst[:, :, blk], payload[i]), blk
        else:
            assert torch.equal(dst[:, :, blk], pool[:, :, blk]), blk
    ref = pool.numpy().copy()
    kvp.write_blocks(ref, ids, payload.numpy())
    assert np.array_equal(ref, dst.numpy())


def test_kv_write_oracle():
    """slots_for, the engine's scatter and write_kv (torch_blocks.py:68-106,
    torch_engine.py:239-240)."""
    check_slots_by_loop(kvp.slots_for)
    check_scatter_by_loops(kvp.scatter_rows)
    check_write_kv_round_trip(kvp.write_kv)
    # NaN stays NaN (torch's encodings of it differ between its code paths)
    cache = torch.zeros(1, 2, 1, 2, dtype=torch.bfloat16)
    kvp.scatter_rows(cache, [1], torch.tensor([[[float("nan"), 1.0]]]))
    assert torch.isnan(cache[0, 1, 0, 0]) and cache[0, 1, 0, 1] == 1.0


def test_block_table_oracle():
    """block_table_tensor (torch_blocks.py:75-85) cell by cell: ids in order,
    -1 padding, width = pad_to or the longest table, truncation."""
    tables = [[4, 9, 1], [], [7], [3, 3, 8, 2, 6]]
    for pad_to in (None, 2, 8):
        got = kvp.block_table_tensor(tables, pad_to)
        width = pad_to or 5
        assert got.dtype == torch.int32 and tuple(got.shape) == (4, width)
        for i, t in enumerate(tables):
            for j in range(width):
                assert int(got[i, j]) == (t[j] if j < len(t) else -1)
    assert tuple(kvp.block_table_tensor([]).shape) == (0, 1)
    assert tuple(kvp.block_table_tensor([[], []]).shape) == (2, 0)


def test_split_heuristic_known_answers():
    """The reference's recorded runs on a 40-SM T4 (README:336, :346) and the
    formula's clamps."""
    assert choose_num_splits(16, 12, 512, cus=40) == 16
    assert choose_num_splits(32, 12, 2048, cus=40) == 64
    assert choose_num_splits(1, 1, 16, cus=256) == 64           # fill term clamps at 64
    assert choose_num_splits(64, 32, 8192, cus=256) == 64
    assert choose_num_splits(512, 64, 40, cus=256) == 1          # floor at 1
    assert choose_num_splits(8, 12, 64, cus=256) == 22           # ceil(2048 / 96)


# ---------------------------------------------------------------------------
# planted mistakes: each mutant of the oracle must fail one of the checks
# ---------------------------------------------------------------------------


def _mutant(module, old: str, new: str) -> types.ModuleType:
    src = inspect.getsource(module)
    assert src.count(old) == 1, f"mutation anchor not found once: {old!r}"
    mod = types.ModuleType(module.__name__ + "_mutant")
    exec(compile(src.replace(old, new), module.__file__, "exec"), mod.__dict__)
    return mod


MUTANTS = [
    ("causal bound off by one", att, "key[None, None, :] <= qpos[:, :, None]",
     "key[None, None, :] < qpos[:, :, None]", "prefill"),
    ("chunk position off by one", att, "qpos = ctx[:, None] - S + torch.arange",
     "qpos = ctx[:, None] - S + 1 + torch.arange", "prefill"),
    ("GQA head mapping", att, "rows.repeat_interleave(n_heads // hkv, dim=2)",
     "rows.repeat(1, 1, n_heads // hkv, 1)", "prefill_gqa"),
    ("slot offset", att, "(blocks[:, :, None] * block_size + offs)",
     "(blocks[:, :, None] * block_size + offs.flip(0))", "decode"),
    ("context mask", att, "live = pos[None, :] < context_lens",
     "live = pos[None, :] <= context_lens", "decode"),
    ("dropped scale", att, 'scores = torch.einsum("bhd,bkhd->bhk", q.to(torch.float32), k) * scale',
     'scores = torch.einsum("bhd,bkhd->bhk", q.to(torch.float32), k)', "decode"),
    ("split chunk floor", rec, "chunk = -(-n // num_splits)", "chunk = max(1, n // num_splits)",
     "split"),
    ("merge weight sign", rec, "np.exp(m - m_g)", "np.exp(m_g - m)", "split"),
    ("tile causal bound", rec, "(k0 + c <= qpos)", "(k0 + c < qpos)", "tiled"),
    ("tile key range from the first row", rec, "key_end = min(ctx_len, pos0 + tile)",
     "key_end = min(ctx_len, pos0 + 1)", "tiled"),
    ("pack axes", kvp, "np.moveaxis(pool[:, :, idx], 2, 0)", "np.moveaxis(pool[:, :, idx], 2, 1)",
     "pack"),
    ("slot offset within a block", kvp, "tbl[pos // block_size] * block_size + pos % block_size",
     "tbl[pos // block_size] * block_size + (pos + 1) % block_size", "slots"),
    ("rows not made token-major", kvp, "kt = k.permute(0, 2, 1, 3).contiguous()",
     "kt = k.reshape(k.shape[0], k.shape[2], k.shape[1], k.shape[3])", "write_kv"),
    ("write position from zero", kvp, "range(start_pos, start_pos + T)", "range(0, T)",
     "write_kv"),
]


def _run_check(kind, mod):
    if kind == "decode":
        check_decode_vs_dense(mod.paged_attention_torch)
    elif kind == "prefill":
        for lens, S, kvh in PREFILL_CASES:
            check_prefill_vs_dense(mod.paged_attention_prefill_torch, lens, S, kvh)
    elif kind == "prefill_gqa":
        check_prefill_vs_dense(mod.paged_attention_prefill_torch, [64], 32, 2)
    elif kind == "split":
        for n, splits, amp in SPLIT_CASES:
            check_split_vs_dense(mod.split_merge_reference, n, splits, amp)
    elif kind == "tiled":
        for ctx, S, D in WMMA_TILING_CASES:
            check_tiled_vs_dense(mod.tiled_prefill_reference, ctx, S, D)
    elif kind == "pack":
        check_pack_by_loops(mod.export_blocks)
    elif kind == "slots":
        check_slots_by_loop(mod.slots_for)
    elif kind == "write_kv":
        check_write_kv_round_trip(mod.write_kv)


@pytest.mark.parametrize("name,module,old,new,kind", MUTANTS, ids=[m[0] for m in MUTANTS])
def test_planted_mistakes_are_caught(name, module, old, new, kind):
    _run_check(kind, module)                       # the real oracle passes ...
    with pytest.raises((AssertionError, IndexError, ValueError, RuntimeError)):
        _run_check(kind, _mutant(module, old, new))   # ... the mutant does not
