"""hs_decode_noalloc: hs_decode with its partition states in the library's
fixed device scratch instead of a caller workspace.

Called through the C ABI and compared with hs_decode on the same inputs: the
same kernels and decomposition run, so the outputs must be bit-identical.
Two calls in a row on one device share the scratch, the second with a
smaller batch (the scratch keeps the first call's contents, which must not
leak into the second result); a call needing more than the fixed size is
refused before any launch.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(lens, H, Hkv, D, dtype, seed):
    rng = np.random.default_rng(seed)
    need = [-(-int(n) // 16) for n in lens]
    nb = sum(need) + 8
    perm = rng.permutation(nb)
    bt = torch.full((len(lens), max(need)), -1, dtype=torch.int32)
    i = 0
    for b, k in enumerate(need):
        bt[b, :k] = torch.as_tensor(perm[i:i + k].astype(np.int32))
        i += k
    gen = torch.Generator(device=DEV).manual_seed(seed)
    kc = torch.randn((nb, 16, Hkv, D), generator=gen, device=DEV).to(dtype)
    vc = torch.randn((nb, 16, Hkv, D), generator=gen, device=DEV).to(dtype)
    q = torch.randn((len(lens), H, D), generator=gen, device=DEV)
    ctx = torch.tensor(lens, dtype=torch.int32, device=DEV)
    return q, kc, vc, bt.to(DEV), ctx


def _args(q, kc, vc, bt, ctx, num_splits):
    from heteroserve import _hip

    B, H, D = q.shape
    NB, BS, Hkv, _ = kc.shape
    out = torch.full((B, H, D), float("nan"), device=DEV)
    head = (q.data_ptr(), kc.data_ptr(), vc.data_ptr(), _hip.dtype_code(kc.dtype), NB,
            bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), B, H, Hkv, D, BS, bt.shape[1],
            D ** -0.5, num_splits, 0)
    return out, head


def _both(case, num_splits=0):
    """(hs_decode output with a torch workspace, hs_decode_noalloc output)."""
    from heteroserve import _hip

    lib = _hip.lib()
    stream = torch.cuda.current_stream().cuda_stream
    q, kc, vc, bt, ctx = case
    want, head = _args(q, kc, vc, bt, ctx, num_splits)
    B, H, D = q.shape
    ws_bytes = lib.hs_decode_workspace_bytes(B, H, kc.shape[2], D, 16, bt.shape[1], num_splits, 0)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    _hip.check(lib.hs_decode(*head, ws.data_ptr(), ws_bytes, stream))
    got, head = _args(q, kc, vc, bt, ctx, num_splits)
    _hip.check(lib.hs_decode_noalloc(*head, stream))
    torch.cuda.synchronize()
    return want, got, ws_bytes


@pytest.mark.parametrize("H,Hkv,D,dtype", [
    (32, 32, 128, torch.bfloat16),     # the VALU partition kernel (C2's geometry)
    (32, 4, 128, torch.bfloat16),      # grouped-query heads on the matrix cores
    (12, 12, 64, torch.float16),       # C1's geometry, small-grid partitions
])
def test_noalloc_matches_hs_decode_twice(H, Hkv, D, dtype):
    from heteroserve import _hip

    assert _hip.ready(), _hip.error()
    big = _case([4100, 300, 8192, 17, 2000, 5000, 1, 6000] * 4, H, Hkv, D, dtype, seed=H + D)
    want, got, ws_bytes = _both(big)
    assert ws_bytes > 0
    assert torch.equal(got, want)
    small = _case([700, 33, 1500], H, Hkv, D, dtype, seed=H + D + 1)
    want, got, ws_bytes = _both(small)
    assert ws_bytes > 0
    assert torch.equal(got, want)
    # one pass (no partition states at all) and explicit splits
    want, got, ws_bytes = _both(small, num_splits=1)
    assert ws_bytes == 0 and torch.equal(got, want)
    want, got, _ = _both(small, num_splits=7)
    assert torch.equal(got, want)


def test_noalloc_sizes_for_the_calls_own_cache_dtype():
    """A bf16 cache with 4 query heads per KV head decodes on the split-operand
    matrix cores (64 sequences over a 16384-token table: the even split, a
    few MB of states).  The dtype-free workspace query sizes for the worst
    dtype, an fp32 cache on the VALU kernel's 256-token partitions (64
    partitions, ~68 MB, above the fixed 64 MiB), so the call must be planned
    for its own dtype to be accepted; it must then equal hs_decode."""
    from heteroserve import _hip

    lib = _hip.lib()
    assert lib.hs_decode_workspace_bytes(64, 32, 8, 128, 16, 1024, 0, 0) > (64 << 20)
    lens = [16384, 5, 3000, 700, 16, 9000] + [int(x) for x in
                                              np.random.default_rng(3).integers(1, 400, 58)]
    case = _case(lens, 32, 8, 128, torch.bfloat16, seed=9)
    want, got, _ = _both(case)
    assert torch.equal(got, want)


def test_noalloc_under_graph_capture():
    """Captured into a HIP graph (after one eager call, which looks up the
    scratch address) and replayed three times with eager work in between:
    every replay equals the eager hs_decode result bit for bit."""
    from heteroserve import _hip

    lib = _hip.lib()
    q, kc, vc, bt, ctx = _case([3000, 17, 900, 5000], 32, 8, 128, torch.bfloat16, seed=21)
    want, _, _ = _both((q, kc, vc, bt, ctx))
    out, head = _args(q, kc, vc, bt, ctx, 0)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _hip.check(lib.hs_decode_noalloc(*head, side.cuda_stream))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _hip.check(lib.hs_decode_noalloc(*head, torch.cuda.current_stream().cuda_stream))
    for i in range(3):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i}"


def test_noalloc_refuses_calls_beyond_its_scratch():
    """512 sequences of up to 8192 tokens at 32 heads on an fp32 cache (fixed
    512-token partitions; 16-bit caches take the even split, whose states are
    far smaller) need 136 MB of partition states, more than the fixed 64 MiB:
    HS_EWORKSPACE, nothing launched.  The inputs have the declared sizes, so
    that a regression of the check fails on the assertions rather than
    reading past the tensors."""
    from heteroserve import _hip

    lib = _hip.lib()
    B, H, D, MB = 512, 32, 128, 512
    assert lib.hs_decode_workspace_bytes(B, H, H, D, 16, MB, 0, 0) > (64 << 20)
    gen = torch.Generator(device=DEV).manual_seed(1)
    kc = torch.randn((1, 16, H, D), generator=gen, device=DEV)
    vc = torch.randn((1, 16, H, D), generator=gen, device=DEV)
    q = torch.randn((B, H, D), generator=gen, device=DEV)
    bt = torch.zeros((B, MB), dtype=torch.int32, device=DEV)      # every page is block 0
    ctx = torch.full((B,), MB * 16, dtype=torch.int32, device=DEV)
    out = torch.zeros((B, H, D), device=DEV)
    rc = lib.hs_decode_noalloc(q.data_ptr(), kc.data_ptr(), vc.data_ptr(), 0, kc.shape[0],
                               bt.data_ptr(), ctx.data_ptr(), out.data_ptr(), B, H, H, D,
                               16, MB, 0.1, 0, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == -4
    assert b"fixed" in lib.hs_last_error()
    torch.cuda.synchronize()
    assert not out.any()
