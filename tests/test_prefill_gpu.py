"""GPU parity of the causal prefill kernels against the oracle.

Restates the reference's gates (tests/test_torch_engine.py:549-589 for the
scalar kernel, :656-699 for the tensor-core kernel) on libhsattn: the fp32
row kernel behind ``paged_attention_prefill`` and the MFMA kernel behind
``paged_attention_prefill_wmma``.  The north-star tolerance for fp16/bf16
caches is a 2e-3 max-abs error, tighter than the reference's 2e-2 WMMA gate.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from _refcases import lay_out, prefill_case, table_array  # noqa: E402
from oracle.attention import paged_attention_prefill_torch, prefill_one  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _maxerr(a, b) -> float:
    return (a.detach().float().cpu() - b.detach().float().cpu()).abs().max().item()


def _oracle(q, k, v, bt, ctx, scale):
    return paged_attention_prefill_torch(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), ctx.cpu(), scale)


def _ref_prefill(lens, S, kvh, seed, dtype=torch.float32):
    c = prefill_case(lens, S, kvh, seed=seed)
    pool = torch.as_tensor(c["pool"]).to(DEV, dtype)
    bt = torch.as_tensor(table_array(c["tables"]), device=DEV)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    q = torch.as_tensor(c["q"], device=DEV)
    return pool, bt, ctx, q, c["scale"]


def test_prefill_kernel_matches_reference():
    """tests/test_torch_engine.py:549-567 (fp32 KV, seed = S), 1e-3."""
    from heteroserve.model import paged_attn_prefill as pf

    assert pf.is_available(), pf.build_error()
    for lens, S, kvh in [([64], 64, None), ([37, 64, 19], 16, None), ([64], 32, 2),
                         ([48], 48, 1)]:
        pool, bt, ctx, q, scale = _ref_prefill(lens, S, kvh, seed=S)
        got = pf.paged_attention_prefill(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
        want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
        np.testing.assert_allclose(got.cpu().numpy(), want.numpy(), rtol=1e-3, atol=1e-3,
                                   err_msg=f"lens={lens} S={S} kv={kvh}")


def test_prefill_with_one_query_equals_decode():
    """tests/test_torch_engine.py:570-589: S = 1 prefill == v2 decode, 1e-3."""
    from heteroserve.model import paged_attn_prefill as pf
    from heteroserve.model import paged_attn_v2 as v2

    pool, bt, ctx, q, scale = _ref_prefill([31, 64, 17], 1, None, seed=3)
    pre = pf.paged_attention_prefill(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
    dec = v2.paged_attention_v2(q[:, 0].contiguous(), pool[0, 0], pool[0, 1], bt, ctx, scale)
    np.testing.assert_allclose(pre[:, 0].cpu().numpy(), dec.cpu().numpy(), rtol=1e-3, atol=1e-3)


def test_prefill_padded_rows_are_zero():
    """A sequence shorter than the chunk has leading rows at negative
    positions: they attend to nothing and are 0 (paged_attn_prefill.py:321)."""
    from heteroserve.model import paged_attn_prefill as pf

    pool, bt, ctx, q, scale = _ref_prefill([64, 10], 32, None, seed=5)
    got = pf.paged_attention_prefill(q, pool[0, 0], pool[0, 1], bt, ctx, scale).cpu()
    assert torch.all(got[1, :22] == 0)
    want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
    assert _maxerr(got, want) <= 1e-3


# ---------------------------------------------------------------------------
# matrix-core path
# ---------------------------------------------------------------------------


def _wmma():
    from heteroserve.model import paged_attn_wmma as wm

    assert wm.is_available(), wm.build_error()
    return wm


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mfma_matches_the_scalar_reference(dtype):
    """tests/test_torch_engine.py:656-699 with the north-star 2e-3 bound
    (the reference gates its WMMA kernel at 2e-2)."""
    wm = _wmma()
    for lens, S, kvh in [([64], 64, None), ([37, 64, 19], 16, None), ([64], 32, 2)]:
        hkv = kvh or 4
        rng = np.random.default_rng(S + len(lens))
        seqs = []
        for n in lens:
            rng.integers(1, 4000, size=n)
            k = rng.standard_normal((4, hkv, n, 64)).astype(np.float16)
            seqs.append((k, k))
        pool_np, tables = lay_out(seqs, 16, 96, hkv, np.float16)
        pool = torch.as_tensor(pool_np, device=DEV).to(dtype)
        assert wm.supports(16, 64, pool.dtype)
        gen = torch.Generator(device=DEV).manual_seed(S)
        q = torch.randn(len(lens), S, 4, 64, device=DEV, generator=gen)
        bt = torch.as_tensor(table_array(tables), device=DEV)
        ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
        got = wm.paged_attention_prefill_wmma(q, pool[0, 0], pool[0, 1], bt, ctx, 0.125)
        want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, 0.125)
        err = _maxerr(got, want)
        assert err <= 2e-3, f"lens={lens} S={S} kv={kvh} err={err:.2e}"


@pytest.mark.parametrize("ctx_len,S,D", [
    (64, 32, 64), (64, 19, 64), (57, 16, 64), (91, 23, 64), (48, 48, 64), (80, 1, 64),
    (100, 40, 128), (512, 16, 64), (300, 300, 32), (1000, 129, 128), (2048, 700, 128),
])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mfma_misaligned_shapes(ctx_len, S, D, dtype):
    """The tile-loop cases of tests/test_torch_engine.py:610-619 (plus larger
    ones) run on the GPU kernel: chunks and contexts that are not multiples of
    the tile, one query row, S == ctx, all three head dims."""
    wm = _wmma()
    rng = np.random.default_rng(ctx_len * 31 + S)
    nb = -(-ctx_len // 16) + 5
    perm = rng.permutation(nb)
    table = [int(x) for x in perm[: -(-ctx_len // 16)]]
    gen = torch.Generator(device=DEV).manual_seed(ctx_len + S + D)
    pool = torch.randn((1, 2, nb, 16, 2, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((1, S, 4, D), generator=gen, device=DEV)
    bt = torch.as_tensor(table_array([table]), device=DEV)
    ctx = torch.tensor([ctx_len], dtype=torch.int32, device=DEV)
    got = wm.paged_attention_prefill_wmma(q, pool[0, 0], pool[0, 1], bt, ctx, D ** -0.5)
    want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, D ** -0.5)
    assert _maxerr(got, want) <= 2e-3


def test_mfma_with_one_query_equals_decode():
    wm = _wmma()
    from heteroserve.model import paged_attn_v2 as v2

    pool, bt, ctx, q, scale = _ref_prefill([31, 64, 17], 1, None, seed=3, dtype=torch.float16)
    pre = wm.paged_attention_prefill_wmma(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
    dec = v2.paged_attention_v2(q[:, 0].contiguous(), pool[0, 0], pool[0, 1], bt, ctx, scale)
    assert _maxerr(pre[:, 0], dec) <= 2e-3


def test_mfma_rejects_what_it_cannot_serve():
    wm = _wmma()
    assert wm.supports(32, 64, torch.float16) is False
    assert wm.supports(16, 64, torch.float32) is False
    assert wm.supports(16, 48, torch.float16) is False
    pool = torch.zeros((1, 2, 4, 16, 4, 64), device=DEV)
    q = torch.zeros((1, 4, 4, 64), device=DEV)
    bt = torch.zeros((1, 4), dtype=torch.int32, device=DEV)
    ctx = torch.tensor([8], dtype=torch.int32, device=DEV)
    with pytest.raises(RuntimeError, match="fp16 or bf16"):
        wm.paged_attention_prefill_wmma(q, pool[0, 0], pool[0, 1], bt, ctx, 0.1)


def test_varlen_matches_per_sequence_calls():
    """One ragged launch == B = 1 calls per chunk (the engine's pattern,
    torch_engine.py:292-313), for both kernels."""
    from heteroserve.model import paged_attn_prefill as pf

    _wmma()
    from hsbench.cases import build_prefill

    case = build_prefill("t", np.array([0, 33, 500, 16]), np.array([40, 1, 129, 300]),
                         8, 4, 128, 200, torch.bfloat16, DEV, seed=8)
    cu = case.cu_seqlens.cpu().numpy()
    for mfma in (False, True):
        got = pf.paged_attention_prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()),
                                                case.k_cache, case.v_cache, case.block_tables,
                                                case.context_lens, case.scale, use_mfma=mfma)
        for b in range(4):
            qb = case.q[cu[b]:cu[b + 1]]
            want = prefill_one(qb.cpu(), case.k_cache.cpu(), case.v_cache.cpu(),
                               case.block_tables[b].cpu(), int(case.ctx[b]), case.scale)
            assert _maxerr(got[cu[b]:cu[b + 1]], want) <= 2e-3, (mfma, b)


def test_negative_context_is_empty():
    """A negative context length (invalid input; the values live on the device,
    so the host cannot reject them) gives that sequence zero rows and leaves
    its neighbours exact, through the key-range split (a small grid) as well
    as the unsplit launch."""
    from heteroserve import _hip

    _wmma()
    from hsbench.cases import build_prefill

    case = build_prefill("t", np.array([100, 300, 0]), np.array([40, 129, 64]),
                         8, 8, 128, 200, torch.bfloat16, DEV, seed=9)
    ctx = case.context_lens.clone()
    ctx[0] = -1000
    cu = case.cu_seqlens.cpu().numpy()
    for split in (True, False):
        got = _hip.prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()), case.k_cache,
                                  case.v_cache, case.block_tables, ctx, case.scale,
                                  use_mfma=True, split=split)
        assert torch.all(got[cu[0]:cu[1]] == 0), split
        for b in (1, 2):
            want = prefill_one(case.q[cu[b]:cu[b + 1]].cpu(), case.k_cache.cpu(),
                               case.v_cache.cpu(), case.block_tables[b].cpu(), int(case.ctx[b]),
                               case.scale)
            assert _maxerr(got[cu[b]:cu[b + 1]], want) <= 2e-3, (split, b)


@pytest.mark.parametrize("name", ["C4", "C5-prefill"])
def test_prefill_configs(name):
    """Full-size chunked prefill through the MFMA kernel: every row of every
    sequence, all heads, against the per-sequence oracle, 2e-3; and the C5
    chunk's engine call shape (B = 1, key-range split) against the same."""
    from heteroserve.model import paged_attn_prefill as pf
    from hsbench import cases

    _wmma()
    case = cases.CONFIGS[name](DEV)
    got = pf.paged_attention_prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()),
                                            case.k_cache, case.v_cache, case.block_tables,
                                            case.context_lens, case.scale, use_mfma=True)
    assert torch.isfinite(got).all()
    cu = case.cu_seqlens.cpu().numpy()
    for b in range(len(case.ctx)):
        n = int(case.ctx[b])
        nblk = -(-n // 16)
        blocks = case.block_tables[b, :nblk].long()
        kb = case.k_cache.index_select(0, blocks).cpu()
        vb = case.v_cache.index_select(0, blocks).cpu()
        want = prefill_one(case.q[cu[b]:cu[b + 1]].cpu(), kb, vb,
                           torch.arange(nblk, dtype=torch.int32), n, case.scale)
        err = _maxerr(got[cu[b]:cu[b + 1]], want)
        assert err <= 2e-3, f"{name} seq {b}: err {err:.2e}"


@pytest.mark.parametrize("n_seq,H,Hkv", [(300, 4, 2), (256, 12, 4), (9, 12, 3)])
def test_mfma_dispatch_orders(n_seq, H, Hkv):
    """The matrix-core kernel's two dispatch orders: longest-first ranking of
    up to 256 sequences (every XCD taking heads h % 8, here with 12 heads, so
    XCDs hold 1 or 2 heads) and the (sequence, head)-major order above 256
    sequences; ragged chunks against the per-sequence oracle."""
    from heteroserve.model import paged_attn_prefill as pf
    from hsbench.cases import build_prefill

    _wmma()
    rng = np.random.default_rng(n_seq + H)
    prefix = rng.integers(0, 200, size=n_seq)
    chunk = rng.integers(1, 60 if n_seq > 100 else 400, size=n_seq)
    need = int(sum(-(-int(p + s) // 16) for p, s in zip(prefix, chunk)))
    case = build_prefill("t", prefix, chunk, H, Hkv, 64, need + 16, torch.bfloat16, DEV,
                         seed=n_seq)
    got = pf.paged_attention_prefill_varlen(case.q, case.cu_seqlens, int(case.q_lens.max()),
                                            case.k_cache, case.v_cache, case.block_tables,
                                            case.context_lens, case.scale, use_mfma=True)
    cu = case.cu_seqlens.cpu().numpy()
    for b in sorted({0, n_seq - 1, *rng.integers(0, n_seq, size=12).tolist()}):
        qb = case.q[cu[b]:cu[b + 1]]
        want = prefill_one(qb.cpu(), case.k_cache.cpu(), case.v_cache.cpu(),
                           case.block_tables[b].cpu(), int(case.ctx[b]), case.scale)
        assert _maxerr(got[cu[b]:cu[b + 1]], want) <= 2e-3, b


@pytest.mark.parametrize("prefix,chunk,H,Hkv,D", [
    ([0], [100], 4, 4, 128),                  # 2 key tiles over 4 parts: empty parts
    ([0, 100, 700], [40, 1, 300], 8, 2, 64),  # ragged, GQA, 4 parts
    ([64, 0], [200, 130], 4, 4, 32),          # 128-row tiles at head dim 32
    ([1500], [700], 16, 4, 128),              # 48 tiles: 4 parts of 8-12 key tiles
])
def test_mfma_key_split(prefix, chunk, H, Hkv, D):
    """Grids too small to cover the CUs split each query tile's key range
    over up to 4 workgroups and merge their partial softmax states; without
    a workspace the same call runs 128-row workgroups instead.  Both against
    the per-sequence oracle, 2e-3."""
    from heteroserve import _hip
    from hsbench.cases import build_prefill

    _wmma()
    need = int(sum(-(-(p + s) // 16) for p, s in zip(prefix, chunk)))
    case = build_prefill("t", np.array(prefix), np.array(chunk), H, Hkv, D, need + 8,
                         torch.bfloat16, DEV, seed=sum(chunk) + D)
    lib = _hip.lib()
    assert lib.hs_prefill_workspace_bytes(len(prefix), max(chunk), H, D, 1) > 0
    cu = case.cu_seqlens.cpu().numpy()
    for split in (True, False):
        got = _hip.prefill_varlen(case.q, case.cu_seqlens, max(chunk), case.k_cache,
                                  case.v_cache, case.block_tables, case.context_lens,
                                  case.scale, use_mfma=True, split=split)
        for b in range(len(prefix)):
            want = prefill_one(case.q[cu[b]:cu[b + 1]].cpu(), case.k_cache.cpu(),
                               case.v_cache.cpu(), case.block_tables[b].cpu(),
                               int(case.ctx[b]), case.scale)
            err = _maxerr(got[cu[b]:cu[b + 1]], want)
            assert err <= 2e-3, (split, b, err)


def test_mfma_key_split_padded_rows():
    """The padded form through the split: rows at negative positions stay 0."""
    wm = _wmma()
    pool, bt, ctx, q, scale = _ref_prefill([64, 10], 32, None, seed=5, dtype=torch.float16)
    got = wm.paged_attention_prefill_wmma(q, pool[0, 0], pool[0, 1], bt, ctx, scale).cpu()
    assert torch.all(got[1, :22] == 0)
    assert _maxerr(got, _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale)) <= 2e-3


def test_prefill_fuzz():
    """Seeded random ragged batches through hs_prefill_varlen: 1 to 40
    sequences, prefixes up to 2500 tokens, chunks of 1 to 900 rows, head dims
    32/64/128, 1 to 8 query heads per KV head, fp16 and bf16 caches.  The
    shapes fall on every plan the matrix-core path has (the key-range split
    and narrower workgroups of small grids, the grid kernel, the persistent
    kernel of large ones); each runs with and without the workspace, and a
    few sequences of each batch are checked against the oracle, 2e-3."""
    from heteroserve import _hip
    from hsbench.cases import build_prefill

    _wmma()
    rng = np.random.default_rng(777)
    heads = [(32, 32), (32, 8), (16, 16), (16, 2), (8, 8), (24, 6), (64, 8), (8, 1)]
    plans = set()
    for case_no in range(12):
        H, Hkv = heads[case_no % len(heads)]
        D = int(rng.choice([32, 64, 128]))
        dtype = (torch.float16, torch.bfloat16)[case_no % 2]
        small = case_no % 3 == 0           # too few query tiles to cover the CUs
        B = int(rng.integers(1, 7 if small else 41))
        prefix = rng.integers(0, 2501, size=B)
        chunk = rng.integers(1, (300 if small else 900) + 1, size=B)
        need = int(sum(-(-int(p + s) // 16) for p, s in zip(prefix, chunk)))
        case = build_prefill("fuzz", prefix, chunk, H, Hkv, D, need + 16, dtype, DEV,
                             seed=900 + case_no)
        ws = _hip.lib().hs_prefill_workspace_bytes(B, int(chunk.max()), H, D, 1)
        plans.add("grid" if ws == 0 else "persistent" if ws == 256 else "key split")
        cu = case.cu_seqlens.cpu().numpy()
        kc, vc = case.k_cache.cpu(), case.v_cache.cpu()
        seqs = sorted(set(int(b) for b in rng.choice(B, size=min(B, 4), replace=False)))
        wants = {b: prefill_one(case.q[cu[b]:cu[b + 1]].cpu(), kc, vc,
                                case.block_tables[b].cpu(), int(case.ctx[b]), case.scale)
                 for b in seqs}
        for split in (True, False):
            got = _hip.prefill_varlen(case.q, case.cu_seqlens, int(chunk.max()), case.k_cache,
                                      case.v_cache, case.block_tables, case.context_lens,
                                      case.scale, use_mfma=True, split=split)
            assert torch.isfinite(got).all(), (case_no, split)
            for b in seqs:
                err = _maxerr(got[cu[b]:cu[b + 1]], wants[b])
                assert err <= 2e-3, (case_no, H, Hkv, D, dtype, B, split, b, err)
    assert plans == {"grid", "persistent", "key split"}, plans
