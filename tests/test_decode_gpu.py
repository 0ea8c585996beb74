"""GPU parity of the decode kernels (v1 / v2 / v3 entry points) against the oracle.

Restates the reference's kernel gates (tests/test_torch_engine.py:199-218,
:284-319, :405-470) on libhsattn, then adds the benchmark configurations and
the edge cases the reference leaves implicit.  Every comparison is against
the CPU oracle (oracle/attention.py) on the same inputs, copied back from the
device; tolerances are written at each assertion.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from _refcases import build_paged_case, lay_out, table_array  # noqa: E402
from oracle.attention import decode_one, paged_attention_torch  # noqa: E402

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _mods():
    from heteroserve.model import paged_attn, paged_attn_v2, paged_attn_v3

    assert paged_attn.which_backend() == "cuda", paged_attn.build_error()
    return paged_attn, paged_attn_v2, paged_attn_v3


def _ref_case(seed=5, lens=(9, 31, 16), dtype=torch.float32):
    c = build_paged_case(seed=seed, lens=lens)
    pool = torch.as_tensor(c["pool"]).to(DEV, dtype)
    bt = torch.as_tensor(table_array(c["tables"])).to(DEV)
    ctx = torch.tensor(c["lens"], dtype=torch.int32, device=DEV)
    q = torch.as_tensor(c["q"], device=DEV)
    return pool, bt, ctx, q, c["scale"]


def _oracle(q, k, v, bt, ctx, scale):
    return paged_attention_torch(q.cpu(), k.cpu(), v.cpu(), bt.cpu(), ctx.cpu(), scale)


def _maxerr(a, b) -> float:
    return (a.detach().float().cpu() - b.detach().float().cpu()).abs().max().item()


# ---------------------------------------------------------------------------
# the reference's kernel gates
# ---------------------------------------------------------------------------


def test_v1_matches_torch_reference():
    """tests/test_torch_engine.py:199-218, tolerance 1e-3."""
    m1, _, _ = _mods()
    pool, bt, ctx, q, scale = _ref_case()
    got = m1.paged_attention(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
    want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
    np.testing.assert_allclose(got.cpu().numpy(), want.numpy(), rtol=1e-3, atol=1e-3)


def test_v2_matches_reference_and_v1():
    """tests/test_torch_engine.py:284-319 (seeds 5 and 9), tolerance 1e-3."""
    m1, m2, _ = _mods()
    assert m2.is_available(), m2.build_error()
    for seed in (5, 9):
        pool, bt, ctx, q, scale = _ref_case(seed=seed)
        a = m1.paged_attention(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
        b = m2.paged_attention_v2(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
        want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale)
        np.testing.assert_allclose(b.cpu().numpy(), want.numpy(), rtol=1e-3, atol=1e-3)
        np.testing.assert_allclose(a.cpu().numpy(), b.cpu().numpy(), rtol=1e-3, atol=1e-3)


def test_v3_every_split_count_matches_reference():
    """tests/test_torch_engine.py:405-429: splits {0,1,2,4,8,16,64}, 1e-3."""
    _, _, m3 = _mods()
    pool, bt, ctx, q, scale = _ref_case()
    want = _oracle(q, pool[0, 0], pool[0, 1], bt, ctx, scale).numpy()
    for splits in (0, 1, 2, 4, 8, 16, 64):
        got = m3.paged_attention_v3(q, pool[0, 0], pool[0, 1], bt, ctx, scale, splits)
        np.testing.assert_allclose(got.cpu().numpy(), want, rtol=1e-3, atol=1e-3,
                                   err_msg=f"num_splits={splits}")


def test_choose_num_splits_uses_the_device_cu_count():
    """paged_attn_v3.py:212-232 with the device's CU count."""
    _, _, m3 = _mods()
    from oracle.splits import choose_num_splits

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for args in [(16, 12, 512), (32, 12, 2048), (1, 1, 16), (64, 32, 8192), (2, 2, 40)]:
        assert m3.choose_num_splits(*args) == choose_num_splits(*args, cus), args


def test_all_three_entry_points_agree_under_fuzz():
    """tests/test_torch_engine.py:432-470: 15 trials, fp16 KV, BS in {8,16,32}, err < 5e-3."""
    m1, m2, m3 = _mods()
    rng = np.random.default_rng(7)
    gen = torch.Generator(device=DEV).manual_seed(7)
    for trial in range(15):
        n_seqs = int(rng.integers(1, 9))
        bs = int(rng.choice([8, 16, 32]))
        lens = [int(rng.integers(1, 700)) for _ in range(n_seqs)]
        need = sum(-(-n // bs) for n in lens) + 8
        seqs = []
        for n in lens:
            rng.integers(1, 4000, size=n)
            k = rng.standard_normal((4, 4, n, 64)).astype(np.float16)
            seqs.append((k, k))
        pool_np, tables = lay_out(seqs, bs, max(32, need), 4, np.float16)
        pool = torch.as_tensor(pool_np, device=DEV)
        q = torch.randn(n_seqs, 4, 64, device=DEV, generator=gen)
        bt = torch.as_tensor(table_array(tables), device=DEV)
        ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
        kp, vp = pool[0, 0], pool[0, 1]
        ref = _oracle(q, kp, vp, bt, ctx, 0.125)
        for name, got in (("v1", m1.paged_attention(q, kp, vp, bt, ctx, 0.125)),
                          ("v2", m2.paged_attention_v2(q, kp, vp, bt, ctx, 0.125)),
                          ("v3", m3.paged_attention_v3(q, kp, vp, bt, ctx, 0.125, 0))):
            err = _maxerr(got, ref)
            assert err < 5e-3, f"{name} trial {trial} lens={lens} bs={bs} err={err:.2e}"


# ---------------------------------------------------------------------------
# dtypes, head dims, block sizes, GQA, edge cases
# ---------------------------------------------------------------------------


def _random_case(lens, H, Hkv, D, bs, dtype, seed, nb_extra=8, shuffle=True):
    rng = np.random.default_rng(seed)
    need = sum(-(-n // bs) for n in lens)
    nb = need + nb_extra
    perm = rng.permutation(nb) if shuffle else np.arange(nb)
    tables, i = [], 0
    for n in lens:
        k = -(-n // bs)
        tables.append([int(x) for x in perm[i:i + k]])
        i += k
    gen = torch.Generator(device=DEV).manual_seed(seed)
    pool = torch.randn((1, 2, nb, bs, Hkv, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((len(lens), H, D), generator=gen, device=DEV)
    bt = torch.as_tensor(table_array(tables), device=DEV)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    return pool, q, bt, ctx


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [32, 64, 128, 256])
def test_decode_dtypes_and_head_dims(dtype, D):
    """Every (dtype, head_dim) instantiation vs the oracle, 2e-3 max-abs."""
    m1, m2, m3 = _mods()
    lens = [1, 15, 16, 17, 100, 300]
    pool, q, bt, ctx = _random_case(lens, 4, 4, D, 16, dtype, seed=D)
    scale = D ** -0.5
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, scale)
    for got in (m1.paged_attention(q, kp, vp, bt, ctx, scale),
                m2.paged_attention_v2(q, kp, vp, bt, ctx, scale),
                m3.paged_attention_v3(q, kp, vp, bt, ctx, scale, 5)):
        assert _maxerr(got, want) <= 2e-3


@pytest.mark.parametrize("bs", [1, 2, 4, 8, 32])
def test_decode_block_sizes(bs):
    """Pages smaller than one wave-wide load take the per-lane addressing path."""
    m1, _, m3 = _mods()
    lens = [3, 64, 257, 600]
    pool, q, bt, ctx = _random_case(lens, 4, 4, 64, bs, torch.float16, seed=100 + bs)
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, 0.125)
    assert _maxerr(m1.paged_attention(q, kp, vp, bt, ctx, 0.125), want) <= 2e-3
    assert _maxerr(m3.paged_attention_v3(q, kp, vp, bt, ctx, 0.125, 3), want) <= 2e-3


@pytest.mark.parametrize("H,Hkv", [(8, 2), (8, 1), (12, 4), (6, 6), (5, 5), (32, 16), (32, 4),
                                   (24, 2), (16, 1), (64, 8)])
def test_decode_gqa_and_odd_head_counts(H, Hkv):
    """GQA/MQA head mapping (one wave serves 1, 2, 4 or 8 query heads of a
    group), and head counts that do not fill a workgroup, on every entry point."""
    m1, m2, m3 = _mods()
    pool, q, bt, ctx = _random_case([40, 333, 1029], H, Hkv, 128, 16, torch.bfloat16,
                                    seed=H * 10 + Hkv)
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, 128 ** -0.5)
    assert _maxerr(m1.paged_attention(q, kp, vp, bt, ctx, 128 ** -0.5), want) <= 2e-3
    assert _maxerr(m2.paged_attention_v2(q, kp, vp, bt, ctx, 128 ** -0.5), want) <= 2e-3
    for n in (0, 3, 16):
        assert _maxerr(m3.paged_attention_v3(q, kp, vp, bt, ctx, 128 ** -0.5, n), want) <= 2e-3


def test_zero_context_gives_zero_rows():
    """ctx <= 0 is undefined in the reference (its kernels return without
    writing, its torch path gives NaN); libhsattn defines it as a zero row."""
    m1, m2, m3 = _mods()
    pool, q, bt, ctx = _random_case([20, 5, 30], 4, 4, 64, 16, torch.float16, seed=3)
    ctx[1] = 0
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, 0.125)
    for got in (m1.paged_attention(q, kp, vp, bt, ctx, 0.125),
                m2.paged_attention_v2(q, kp, vp, bt, ctx, 0.125),
                m3.paged_attention_v3(q, kp, vp, bt, ctx, 0.125, 4)):
        g = got.cpu()
        assert torch.all(g[1] == 0)
        assert _maxerr(g[[0, 2]], want[[0, 2]]) <= 2e-3


def test_context_beyond_table_and_negative_entries():
    """ctx larger than the table holds is clamped to MB * BS, and -1 entries
    inside the context read block 0 -- both as the torch reference does."""
    m1, _, m3 = _mods()
    pool, q, bt, ctx = _random_case([40, 64], 4, 4, 64, 16, torch.float16, seed=11)
    ctx[0] = 10_000            # table has 3 blocks = 48 positions
    bt[1, 2] = -1              # hole inside sequence 1's context
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, 0.125)
    for got in (m1.paged_attention(q, kp, vp, bt, ctx, 0.125),
                m3.paged_attention_v3(q, kp, vp, bt, ctx, 0.125, 2)):
        assert _maxerr(got, want) <= 2e-3


def test_split_invariance_and_partition_sizes():
    """The result may not depend on the decomposition: one pass, num_splits
    slices and fixed partitions of several sizes all agree."""
    from heteroserve import _hip

    _mods()
    pool, q, bt, ctx = _random_case([1, 255, 256, 257, 1000, 2500], 8, 8, 128, 16,
                                    torch.bfloat16, seed=21)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = 128 ** -0.5
    want = _oracle(q, kp, vp, bt, ctx, scale)
    outs = [_hip.decode(q, kp, vp, bt, ctx, scale, num_splits=s) for s in (1, 2, 3, 17, 64)]
    outs += [_hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=p)
             for p in (16, 64, 256, 512, 4096)]
    for o in outs:
        assert _maxerr(o, want) <= 2e-3
        assert _maxerr(o, outs[0]) <= 1e-4


def test_small_grid_default_partition():
    """With the library's default decomposition a small batch gets more waves
    on the CUs: the workspace query for C1's 8 x 12 rows with a 512-token
    table reports 32-token partitions (16 per row); the call itself, whose
    rows fit one workgroup, splits each row over a workgroup's waves instead
    (no merge).  The result agrees with explicit 512-token partitions and the
    oracle."""
    from heteroserve import _hip

    _mods()
    lib = _hip.lib()
    B, H, D, MB = 8, 12, 64, 32
    ws = lib.hs_decode_workspace_bytes(B, H, H, D, 16, MB, 0, 0)
    acc = B * H * 16 * D * 4
    assert ws == (acc + 255) // 256 * 256 + B * H * 16 * 2 * 4
    big = lib.hs_decode_workspace_bytes(64, 32, 32, 128, 16, 512, 0, 0)
    assert big == 64 * 32 * 16 * 128 * 4 + 64 * 32 * 16 * 2 * 4   # C2 keeps 512 tokens
    pool, q, bt, ctx = _random_case([16, 100, 257, 300, 401, 480, 511, 512], H, H, D, 16,
                                    torch.float16, seed=33)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    got = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
    fixed = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=512)
    assert _maxerr(got, _oracle(q, kp, vp, bt, ctx, scale)) <= 2e-3
    assert _maxerr(got, fixed) <= 1e-4


@pytest.mark.parametrize("H,Hkv,D,dtype", [
    (12, 12, 64, torch.float16),    # C1's geometry: 16 waves per workgroup
    (8, 8, 128, torch.bfloat16),
    (8, 4, 64, torch.float32),      # G = 2
    (16, 4, 128, torch.float32),    # G = 4
    (16, 2, 64, torch.float32),     # G = 8: 8 waves per workgroup
    (4, 4, 256, torch.float16),     # head dim 256: 8 waves per workgroup
    (6, 2, 32, torch.float32),      # 3 query heads per KV head (one per wave), head dim 32
])
def test_workgroup_split_decode(H, Hkv, D, dtype):
    """Small grids of short rows (the default decomposition, up to 1024 keys
    by the table's width, where the VALU kernel runs): one workgroup per
    (row, head group) splits the row's keys over its waves and merges their
    states in LDS.  Rows of 0, 1, 7 and 9 tokens (empty and ragged slices,
    a zero row), full rows and every length between, against the oracle and
    explicit 64-token partitions, twice (bit-identical)."""
    from heteroserve import _hip

    _mods()
    lens = [0, 1, 7, 9, 16, 100, 255, 333, 512, 700, 1000, 1024]
    pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=52)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    got = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
    want = _oracle(q, kp, vp, bt, ctx, scale)
    assert _maxerr(got[1:], want[1:]) <= 1e-4
    assert torch.count_nonzero(got[0]) == 0                       # context 0: a zero row
    part = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=64)
    assert _maxerr(got, part) <= 1e-5
    assert torch.equal(got, _hip.decode(q, kp, vp, bt, ctx, scale, 0))


def test_one_partition_rows_stay_on_the_matrix_cores():
    """A large batch whose table is no wider than one fixed partition (64
    sequences, contexts up to 700 tokens, 4 query heads per KV head, bf16,
    768-token partitions) has one partition per row.  Fixed partitions stay
    on the split-operand matrix-core kernel then (it writes the rows itself,
    no merge) instead of the one-pass VALU kernel.  Checked against the
    oracle; the path is checked by its result: bit-identical to a 1024-token
    plan (also one partition a row, the same walk), and not bit-identical to
    the one-pass fp32 kernel (v2).  The library default on this grid (the
    even split) agrees with both to the split operands' tolerance.  bench.py's
    GQA one-partition leg times them."""
    from heteroserve import _hip

    _, m2, _ = _mods()
    rng = np.random.default_rng(5)
    lens = [int(x) for x in rng.integers(100, 700, size=64, endpoint=True)]
    pool, q, bt, ctx = _random_case(lens, 32, 8, 128, 16, torch.bfloat16, seed=5)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = 128 ** -0.5
    assert bt.shape[1] * 16 <= 768
    one = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=768)
    want = _oracle(q, kp, vp, bt, ctx, scale)
    assert _maxerr(one, want) <= 5e-5
    assert torch.equal(one, _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=1024))
    v2 = m2.paged_attention_v2(q, kp, vp, bt, ctx, scale)
    assert not torch.equal(one, v2)
    default = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
    assert _maxerr(default, want) <= 5e-5
    assert _maxerr(default, one) <= 5e-5


@pytest.mark.parametrize("H,Hkv,D,dtype,lens", [
    (32, 8, 128, torch.bfloat16, [1000, 3000]),          # G = 4: 768-token default
    (32, 4, 128, torch.bfloat16, [700, 2100, 40]),       # G = 8: 384-token default
    (12, 3, 64, torch.float16, [1500]),                  # G = 4 at head dim 64
])
def test_small_grid_gqa_default_partition(H, Hkv, D, dtype, lens):
    """Grouped-query batches too small for the CUs: the split-operand
    decode's default partition (768 tokens up to 4 query heads per KV head,
    384 up to 8) is halved, never below one page per wave, until the grid
    has 8 waves per CU (up to 4 query heads per KV head) or 4 (above); the
    lengths this visits (384, 192, 96, 64 and 48, 32
    tokens) are no powers of two.  Results match the oracle and the one-pass
    fp32 kernel to the split operands' precision, and a rerun is
    bit-identical."""
    from heteroserve import _hip

    _, m2, _ = _mods()
    pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=41)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    got = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
    assert _maxerr(got, _oracle(q, kp, vp, bt, ctx, scale)) <= 5e-5
    assert _maxerr(got, m2.paged_attention_v2(q, kp, vp, bt, ctx, scale)) <= 5e-5
    assert torch.equal(got, _hip.decode(q, kp, vp, bt, ctx, scale, 0))


@pytest.mark.parametrize("H,Hkv,D,dtype", [
    (32, 8, 128, torch.bfloat16),   # llama3-8b shape (config.py:85-93), G = 4
    (32, 1, 128, torch.bfloat16),   # MQA: two head chunks of 16
    (40, 1, 128, torch.float16),    # G = 40: head chunks of 16, 16 and 8
    (64, 2, 64, torch.bfloat16),    # G = 32 at head_dim 64
    (16, 2, 32, torch.float16),     # G = 8 at head_dim 32
    (12, 3, 128, torch.bfloat16),   # G = 4, 3 KV heads
])
def test_gqa_matrix_core_decode(H, Hkv, D, dtype):
    """Grouped-query decode on the matrix cores (16-token pages, fixed
    partitions up to 1024 tokens): every partition length from 16 to 1024
    tokens vs the oracle (2e-3) and vs the one-pass VALU kernel (v2), on
    contexts that end inside, at and past page and partition boundaries."""
    from heteroserve import _hip

    m1, m2, _ = _mods()
    lens = [1, 15, 16, 17, 33, 100, 511, 512, 513, 1500, 3000]
    pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=H * 7 + Hkv + D)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    want = _oracle(q, kp, vp, bt, ctx, scale)
    one_pass = m2.paged_attention_v2(q, kp, vp, bt, ctx, scale)
    assert _maxerr(one_pass, want) <= 2e-3
    outs = [m1.paged_attention(q, kp, vp, bt, ctx, scale)]
    outs += [_hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=p)
             for p in (16, 48, 128, 512, 1024)]
    for o in outs:
        assert _maxerr(o, want) <= 2e-3
        assert _maxerr(o, one_pass) <= 2e-3


def test_gqa_matrix_core_table_edges():
    """The matrix-core GQA path reads -1 table entries inside the context as
    block 0 and clamps ctx to the table, as the VALU path and the torch
    reference do, and gives zero rows for ctx <= 0."""
    m1, _, _ = _mods()
    pool, q, bt, ctx = _random_case([40, 64, 300], 16, 2, 128, 16, torch.bfloat16, seed=13)
    ctx[0] = 10_000            # table holds 3 blocks = 48 positions
    bt[1, 2] = -1              # hole inside sequence 1's context
    ctx[2] = 0
    kp, vp = pool[0, 0], pool[0, 1]
    want = _oracle(q, kp, vp, bt, ctx, 0.125)
    got = m1.paged_attention(q, kp, vp, bt, ctx, 0.125).cpu()
    assert torch.all(got[2] == 0)
    assert _maxerr(got[[0, 1]], want[[0, 1]]) <= 2e-3


@pytest.mark.parametrize("H,Hkv,D,dtype,lens,edges", [
    # C2-like ragged batch with empty, one-token and page-edge rows, a context
    # past the table, a negative one and a -1 hole
    (32, 8, 128, torch.bfloat16,
     [0, 1, 15, 16, 17, 8000, 0, 2047, 33, 5000] + [int(x) for x in
                                                    np.random.default_rng(3).integers(64, 4000, 54)],
     True),
    # four long rows: ranges of more than 64 pages (several block-id windows)
    (32, 8, 32, torch.float16, [70000, 69999, 70001, 65536], False),
    # 300 rows: the row scans run over several 64-row chunks; G = 2
    (16, 8, 64, torch.bfloat16,
     [int(x) for x in np.random.default_rng(4).integers(0, 2000, 300)], False),
    # plain multi-head attention (the VALU walk): the same edge rows
    (32, 32, 128, torch.bfloat16,
     [0, 1, 15, 16, 17, 8000, 0, 2047, 33, 5000] + [int(x) for x in
                                                    np.random.default_rng(5).integers(64, 4000, 54)],
     True),
    (16, 16, 64, torch.float16,
     [int(x) for x in np.random.default_rng(6).integers(0, 2000, 300)], False),
    (8, 8, 256, torch.bfloat16, [70000, 69999, 70001, 65536], False),
    # an odd head count: the last two-head workgroup has one live wave
    (5, 5, 128, torch.bfloat16,
     [int(x) for x in np.random.default_rng(7).integers(1, 3000, 120)], False),
])
def test_even_split_decode(H, Hkv, D, dtype, lens, edges):
    """The default decomposition of decode on 16-bit caches with up to 4
    query heads per KV head, on grids that fill the device: all pages of the
    batch cut into one equal range per workgroup, rows cut across ranges
    merged afterwards (the split-operand matrix cores for grouped heads, the
    VALU walk for plain multi-head attention).  Against the oracle to the
    split operands' tolerance, against fixed 512-token partitions, and
    bit-identical on a rerun; rows without keys are zero."""
    from heteroserve import _hip

    pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=len(lens) + D)
    if edges:
        ctx[5] = bt.shape[1] * 16 + 999     # clamped to the table
        ctx[6] = -3                         # no keys
        bt[7, 5] = -1                       # hole: read as block 0, like the oracle
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    got = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
    want = _oracle(q, kp, vp, bt, ctx, scale)
    live = (ctx > 0).cpu()              # the oracle's softmax over no keys is undefined
    assert _maxerr(got.cpu()[live], want[live]) <= SPLIT_TOL[dtype]
    assert torch.all(got.cpu()[~live] == 0)
    fixed = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=512)
    assert _maxerr(got, fixed) <= SPLIT_TOL[dtype]
    assert torch.equal(got, _hip.decode(q, kp, vp, bt, ctx, scale, 0))


# Split-operand matrix-core decode: hi + lo terms of the cache's type for q
# and the probabilities; fp32-grade results.  Tolerances (max-abs, O(1)
# outputs): bf16 5e-5 (hi + lo carry 16 significant bits), fp16 1e-5 (22
# bits), against the reference tests' 2e-3.
SPLIT_TOL = {torch.bfloat16: 5e-5, torch.float16: 1e-5}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,Hkv,D", [
    (4, 2, 128),     # G = 2, MFMA columns: hi/lo pairs of 2 heads
    (12, 4, 64),     # G = 3: odd group, columns 3..7 and 11..15 idle
    (24, 4, 128),    # G = 6
    (32, 4, 128),    # G = 8: all 16 columns in use
    (24, 2, 64),     # G = 12: hi and lo as two products
    (48, 2, 128),    # G = 24: a chunk of 16 heads and one of 8
    (8, 4, 32),      # head dim 32: one page per load, one QK k-step
    (40, 1, 32),     # head dim 32, G = 40
])
def test_split_operand_decode(H, Hkv, D, dtype):
    """Grouped-query decode of a bf16 or fp16 cache runs on the matrix cores
    with q and the probabilities split into hi + lo terms of the cache's
    type: fp32-grade results for every group size and both column layouts,
    on partitions from one page to 1024 tokens."""
    from heteroserve import _hip

    lens = [1, 15, 16, 17, 100, 511, 513, 2000]
    pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=H + 3 * Hkv + D)
    kp, vp = pool[0, 0], pool[0, 1]
    scale = D ** -0.5
    want = _oracle(q, kp, vp, bt, ctx, scale)
    for p in (16, 128, 1024):
        got = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=p)
        assert _maxerr(got, want) <= SPLIT_TOL[dtype], (H, Hkv, D, p)


def test_split_operand_decode_fuzz():
    """Seeded random cache types, group sizes (2..32 query heads per KV head,
    odd ones included), head dims (32, 64, 128), batch shapes and partition
    lengths for the split-operand matrix-core decode, each against the oracle."""
    from heteroserve import _hip

    rng = np.random.default_rng(2024)
    groups = [(4, 2), (6, 3), (8, 2), (12, 4), (15, 3), (20, 4), (24, 3), (32, 8), (40, 5),
              (48, 3), (64, 4), (64, 2)]
    for case in range(24):
        H, Hkv = groups[case % len(groups)]
        dtype = (torch.bfloat16, torch.float16)[case % 2]
        D = int(rng.choice([32, 64, 128]))
        lens = [int(x) for x in rng.integers(1, 1500, size=int(rng.integers(1, 7)))]
        pt = int(rng.choice([0, 16, 48, 256, 1024]))
        pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=100 + case)
        kp, vp = pool[0, 0], pool[0, 1]
        scale = D ** -0.5
        got = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=pt)
        want = _oracle(q, kp, vp, bt, ctx, scale)
        assert _maxerr(got, want) <= SPLIT_TOL[dtype], (case, dtype, H, Hkv, D, lens, pt)


def test_even_split_decode_fuzz():
    """Seeded random batches through the default decomposition on grids large
    enough for the even split: plain multi-head attention (the VALU walk) and
    2 to 4 query heads per KV head (the split-operand matrix cores), bf16 and
    fp16 caches, head dims 32 to 256, empty and clamped rows; each against
    the oracle and against fixed partitions."""
    from heteroserve import _hip

    rng = np.random.default_rng(4242)
    heads = [(32, 32), (16, 16), (12, 12), (32, 8), (16, 4), (24, 12), (8, 8), (20, 5)]
    for case in range(10):
        H, Hkv = heads[case % len(heads)]
        dtype = (torch.bfloat16, torch.float16)[case % 2]
        D = int(rng.choice([32, 64, 128, 256] if H == Hkv else [32, 64, 128]))
        B = int(rng.integers(64, 260))
        lens = [int(x) for x in rng.integers(0, 3000, size=B)]
        pool, q, bt, ctx = _random_case(lens, H, Hkv, D, 16, dtype, seed=500 + case)
        if case % 3 == 0:
            ctx[1] = bt.shape[1] * 16 + 77      # clamped to the table
            ctx[2] = -5                         # no keys
        kp, vp = pool[0, 0], pool[0, 1]
        scale = D ** -0.5
        got = _hip.decode(q, kp, vp, bt, ctx, scale, 0)
        want = _oracle(q, kp, vp, bt, ctx, scale)
        live = (ctx > 0).cpu()
        info = (case, dtype, H, Hkv, D, B)
        assert _maxerr(got.cpu()[live], want[live]) <= SPLIT_TOL[dtype], info
        assert torch.all(got.cpu()[~live] == 0), info
        fixed = _hip.decode(q, kp, vp, bt, ctx, scale, 0, partition_tokens=512)
        assert _maxerr(got, fixed) <= SPLIT_TOL[dtype], info


def test_errors_are_raised_with_reference_messages():
    m1, m2, _ = _mods()
    pool, q, bt, ctx = _random_case([10], 4, 4, 64, 16, torch.float16, seed=1)
    kp, vp = pool[0, 0], pool[0, 1]
    with pytest.raises(RuntimeError, match="q must be on CUDA"):
        m1.paged_attention(q.cpu(), kp, vp, bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="divisible"):
        m2.paged_attention_v2(q[:, :3].contiguous(), kp[:, :, :2].contiguous(),
                              vp[:, :, :2].contiguous(), bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="head_dim"):
        m1.paged_attention(q[..., :48].contiguous(), kp[..., :48].contiguous(),
                           vp[..., :48].contiguous(), bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="float32"):
        m1.paged_attention(q.half(), kp, vp, bt, ctx, 0.1)


# ---------------------------------------------------------------------------
# benchmark configurations at full size
# ---------------------------------------------------------------------------


def _config(name):
    from hsbench import cases

    return cases.CONFIGS[name](DEV)


def _check_sequences(case, got, seqs, tol):
    kc, vc = case.k_cache, case.v_cache
    for b in seqs:
        n = int(case.ctx[b])
        nblk = -(-n // 16)
        blocks = case.block_tables[b, :nblk]
        kb = kc.index_select(0, blocks.long()).cpu()
        vb = vc.index_select(0, blocks.long()).cpu()
        want = decode_one(case.q[b].cpu(), kb, vb, torch.arange(nblk, dtype=torch.int32),
                          n, case.scale)
        err = _maxerr(got[b], want)
        assert err <= tol, f"{case.name} sequence {b} ctx {n}: max err {err:.2e}"


def test_c1_full_batch_against_the_oracle():
    m1, _, m3 = _mods()
    case = _config("C1")
    want = _oracle(case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
                   case.scale)
    for got in (m1.paged_attention(case.q, case.k_cache, case.v_cache, case.block_tables,
                                   case.context_lens, case.scale),
                m3.paged_attention_v3(case.q, case.k_cache, case.v_cache, case.block_tables,
                                      case.context_lens, case.scale, 8)):
        assert _maxerr(got, want) <= 2e-3


@pytest.mark.parametrize("name", ["C2", "C2-gqa", "C3", "C5-decode"])
def test_large_configs(name):
    """Full-size batches: every sequence against the per-sequence oracle at
    2e-3, and the whole batch through the decomposition-invariance property
    (one pass and 13 splits against the default partitions)."""
    m1, m2, m3 = _mods()
    case = _config(name)
    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
            case.scale)
    fast = m1.paged_attention(*args)
    _check_sequences(case, fast, range(len(case.ctx)), 2e-3)
    one_pass = m2.paged_attention_v2(*args)
    split = m3.paged_attention_v3(*args, 13)
    assert _maxerr(fast, one_pass) <= 2e-3
    assert _maxerr(fast, split) <= 2e-3
    assert torch.isfinite(fast).all()
    del case
    torch.cuda.empty_cache()


# ---------------------------------------------------------------------------
# shared pages (prefix caching): hs_decode_shared
# ---------------------------------------------------------------------------


def _shared_pages_case(ctx, groups, H, Hkv, D, dtype, seed):
    """Block tables where each group (members, n_blocks) starts with the same
    n_blocks block ids; every other page is private.  Pool filled from N(0, 1)."""
    rng = np.random.default_rng(seed)
    need = [-(-int(n) // 16) for n in ctx]
    nb = sum(need) + 16
    perm = iter(rng.permutation(nb).tolist())
    prefix_of = {}
    for members, n_blocks in groups:
        ids = [next(perm) for _ in range(n_blocks)]
        for b in members:
            prefix_of[b] = ids
    tables = []
    for b, n in enumerate(need):
        t = list(prefix_of.get(b, [])[:n])
        while len(t) < n:
            t.append(next(perm))
        tables.append(t)
    gen = torch.Generator(device=DEV).manual_seed(seed)
    pool = torch.randn((nb, 16, Hkv, D), generator=gen, device=DEV).to(dtype)
    vpool = torch.randn((nb, 16, Hkv, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((len(ctx), H, D), generator=gen, device=DEV)
    width = max(need)
    bt = torch.full((len(ctx), width), -1, dtype=torch.int32)
    for b, t in enumerate(tables):
        bt[b, :len(t)] = torch.tensor(t, dtype=torch.int32)
    return (q, pool, vpool, bt.to(DEV), torch.tensor(ctx, dtype=torch.int32, device=DEV),
            D ** -0.5)


def _oracle_rows(q, kc, vc, bt, ctx, scale, rows):
    out = {}
    for b in rows:
        n = int(ctx[b])
        nblk = -(-n // 16)
        blocks = bt[b, :nblk].long()
        out[b] = decode_one(q[b].cpu(), kc.index_select(0, blocks).cpu(),
                            vc.index_select(0, blocks).cpu(),
                            torch.arange(nblk, dtype=torch.int32), n, scale)
    return out


@pytest.mark.parametrize("H,Hkv,D,dtype,pt,ctx,groups", [
    # a group of 8 over 1024 tokens (members at 512 tokens have only that
    # partition, members below 1024 share partition 0 only), a pair (too few
    # to group), a group of exactly 4 over one partition, private sequences
    (8, 8, 128, torch.bfloat16, 0,
     [1024, 1100, 1536, 2000, 530, 512, 1031, 4000, 1500, 1700, 600, 777, 513, 640, 90, 3000],
     [(range(0, 8), 64), ([8, 9], 96), ([10, 11, 12, 13], 40)]),
    # GQA, 4 query heads per KV head: 8 sequences per unit, 40 sharers
    (16, 4, 64, torch.float16, 0, [2048 + 37 * i for i in range(40)] + [700, 3000],
     [(range(0, 40), 128)]),
    # 70 sharers of 256-token partitions: units of 32, 32 and 6
    (4, 4, 32, torch.bfloat16, 256, [1300 + 11 * i for i in range(70)], [(range(0, 70), 80)]),
    # 8 and 16 query heads per KV head: the unshared partitions run on the
    # matrix-core GQA kernel, which skips the shared ones too
    (32, 4, 128, torch.bfloat16, 0, [1100 + 57 * i for i in range(12)] + [300, 5000],
     [(range(0, 12), 64)]),
    (32, 2, 64, torch.float16, 0, [700 + 90 * i for i in range(9)], [(range(0, 9), 40)]),
])
def test_shared_pages_decode(H, Hkv, D, dtype, pt, ctx, groups):
    """Sequences holding the same pages: their shared partitions are read once
    for the whole group on the matrix cores, with split operands.  Every
    sequence against the per-sequence oracle at the split-operand tolerance;
    outputs of sequences in no group are the plain path's, bit for bit."""
    from heteroserve import _hip

    _mods()
    q, kc, vc, bt, cl, scale = _shared_pages_case(ctx, groups, H, Hkv, D, dtype, seed=len(ctx))
    plain = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, partition_tokens=pt)
    shared = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, partition_tokens=pt,
                         shared_pages=True)
    assert torch.isfinite(shared).all()
    want = _oracle_rows(q, kc, vc, bt, cl, scale, range(len(ctx)))
    for b, w in want.items():
        err = _maxerr(shared[b], w)
        assert err <= SPLIT_TOL[dtype], f"sequence {b} ctx {ctx[b]}: {err:.2e}"
    grouped = {b for members, _ in groups if len(members) >= 4 for b in members}
    # hs_decode's default for 2..4 query heads per KV head on a grid that
    # fills the device is the even split, another cut of the rows than the
    # fixed partitions this entry point keeps: there the ungrouped rows agree
    # to the split operands' tolerance, elsewhere bit for bit
    exact = not (pt == 0 and 2 <= H // Hkv <= 4)
    for b in range(len(ctx)):
        if b not in grouped:
            if exact:
                assert torch.equal(shared[b], plain[b]), b
            else:
                assert _maxerr(shared[b], plain[b]) <= SPLIT_TOL[dtype], b
    # a sequence's result depends on nothing but its own query and pages: the
    # same call again, and the batch in reverse order, give the same bits
    again = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, partition_tokens=pt,
                        shared_pages=True)
    assert torch.equal(again, shared)
    flip = torch.arange(len(ctx) - 1, -1, -1, device=DEV)
    rev = _hip.decode(q[flip].contiguous(), kc, vc, bt[flip].contiguous(), cl[flip].contiguous(),
                      scale, num_splits=0, partition_tokens=pt, shared_pages=True)
    assert torch.equal(rev[flip], shared)


def test_shared_pages_partial_members():
    """Sequences whose context ends inside a shared partition (a prefix they
    have not grown past) join the group of that partition's full holders:
    their own keys are masked at their context, one ending in partition 0 is
    the row's only partition (written directly), and a sequence whose pages
    leave the shared prefix inside the partition stays on its own there.
    Every sequence against the oracle; the call is deterministic on a rerun
    and on the reversed batch."""
    from heteroserve import _hip

    _mods()
    ctx = [1100, 1500, 2000, 1024, 700, 300, 900, 520, 512, 3000]
    groups = [(range(0, 6), 64)]
    q, kc, vc, bt, cl, scale = _shared_pages_case(ctx, groups, 8, 8, 128, torch.bfloat16, seed=77)
    bt[6, :40] = bt[0, :40]     # 900 tokens: the prefix's first 40 pages, then its own
    bt[7, :33] = bt[0, :33]     # 520 tokens: 33 pages, all the prefix's
    bt[8, :32] = bt[0, :32]     # 512 tokens: partition 0 exactly
    out = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, partition_tokens=512,
                      shared_pages=True)
    want = _oracle_rows(q, kc, vc, bt, cl, scale, range(len(ctx)))
    for b, w in want.items():
        assert _maxerr(out[b], w) <= SPLIT_TOL[torch.bfloat16], (b, ctx[b])
    again = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, partition_tokens=512,
                        shared_pages=True)
    assert torch.equal(again, out)
    flip = torch.arange(len(ctx) - 1, -1, -1, device=DEV)
    rev = _hip.decode(q[flip].contiguous(), kc, vc, bt[flip].contiguous(), cl[flip].contiguous(),
                      scale, num_splits=0, partition_tokens=512, shared_pages=True)
    assert torch.equal(rev[flip], out)


def test_shared_pages_c5():
    """C5's decode batch (half the sequences share a 1024-token prefix, some
    of them ending inside it): the shared-page path against the plain (fp32
    VALU) one, and every sequence against the oracle, at the bf16
    split-operand tolerance."""
    from heteroserve import _hip

    _mods()
    case = _config("C5-decode")
    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens,
            case.scale)
    plain = _hip.decode(*args, num_splits=0)
    shared = _hip.decode(*args, num_splits=0, shared_pages=True)
    tol = SPLIT_TOL[case.k_cache.dtype]
    assert _maxerr(shared, plain) <= tol
    _check_sequences(case, shared, range(len(case.ctx)), tol)
    del case
    torch.cuda.empty_cache()


def test_shared_pages_fallbacks():
    """Geometries the shared-page kernel does not serve run hs_decode's path:
    fp32 pools give the plain result bit for bit; num_splits != 0 is refused."""
    from heteroserve import _hip

    _mods()
    q, kc, vc, bt, cl, scale = _shared_pages_case([1024] * 6, [(range(6), 64)], 4, 4, 64,
                                                  torch.float32, seed=3)
    plain = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0)
    shared = _hip.decode(q, kc, vc, bt, cl, scale, num_splits=0, shared_pages=True)
    assert torch.equal(plain, shared)
    with pytest.raises(RuntimeError, match="num_splits"):
        _hip.decode(q, kc, vc, bt, cl, scale, num_splits=2, shared_pages=True)
