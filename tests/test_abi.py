"""CPU checks of the C-ABI boundary and the Python module state (no GPU needed).

The library must load without a GPU, export every function include/hsattn.h
declares, and reject bad arguments before touching the device.  The Python
modules keep the reference's module-state API and never compute on the CPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hsattn.h"


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from heteroserve import _hip

    if not _hip.lib_path().exists():
        pytest.fail(f"{_hip.lib_path()} missing: run python hetero-serve_amd/build.py")
    return _hip.open_library()


def test_header_declarations_are_bound_by_the_loader():
    from heteroserve import _hip

    assert _declared_functions() == sorted(_hip.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.hs_abi_version() == 5
    assert lib.hs_last_error() == b""


def test_argument_errors_need_no_device(lib):
    """Validation happens before any HIP call: these return codes and
    messages come back on a machine without a GPU."""
    fake = ctypes.c_void_p(0x1000)
    rc = lib.hs_decode(None, None, None, 0, 8, None, None, None, 1, 4, 4, 64, 16, 2,
                       0.1, 0, 0, None, 0, None)
    assert rc == -1 and b"null" in lib.hs_last_error()
    rc = lib.hs_decode(fake, fake, fake, 0, 8, fake, fake, fake, 1, 6, 4, 64, 16, 2,
                       0.1, 0, 0, None, 0, None)
    assert rc == -1 and b"divisible" in lib.hs_last_error()
    rc = lib.hs_decode(fake, fake, fake, 0, 8, fake, fake, fake, 1, 4, 4, 96, 16, 2,
                       0.1, 0, 0, None, 0, None)
    assert rc == -2 and b"head_dim" in lib.hs_last_error()
    rc = lib.hs_decode(fake, fake, fake, 5, 8, fake, fake, fake, 1, 4, 4, 64, 16, 2,
                       0.1, 0, 0, None, 0, None)
    assert rc == -1 and b"dtype" in lib.hs_last_error()
    # partitioned decode needs a workspace
    need = lib.hs_decode_workspace_bytes(2, 4, 4, 64, 16, 64, 0, 0)
    assert need > 0
    rc = lib.hs_decode(fake, fake, fake, 1, 8, fake, fake, fake, 2, 4, 4, 64, 16, 64,
                       0.1, 0, 0, None, 0, None)
    assert rc == -4 and b"workspace" in lib.hs_last_error()
    assert lib.hs_decode_workspace_bytes(2, 4, 4, 64, 16, 64, 1, 0) == 0      # one pass
    assert lib.hs_decode_workspace_bytes(2, 4, 4, 64, 16, 64, 0, 24) == 0     # bad partition
    # shared-page decode: hs_decode's partition states plus the grouping arrays
    base = lib.hs_decode_workspace_bytes(255, 32, 32, 128, 16, 256, 0, 0)
    assert lib.hs_decode_shared_workspace_bytes(255, 32, 32, 128, 16, 256, 0) > base > 0
    assert lib.hs_decode_shared_workspace_bytes(4, 32, 32, 128, 16, 32, 0) == 0   # one partition
    rc = lib.hs_decode_shared(fake, fake, fake, 0, 8, fake, fake, fake, 1, 6, 4, 64, 16, 2,
                              0.1, 0, None, 0, None)
    assert rc == -1 and b"divisible" in lib.hs_last_error()
    assert lib.hs_prefill_workspace_bytes(1, 1024, 32, 128, 0) == 0          # row kernel
    assert lib.hs_prefill_workspace_bytes(0, 1024, 32, 128, 1) == 0          # nothing to do
    rc = lib.hs_prefill(fake, fake, fake, 0, 8, fake, fake, fake, 1, 4, 4, 4, 64, 16, 2,
                        0.1, 1, None, 0, None)
    assert rc == -2 and b"fp16 or bf16" in lib.hs_last_error()
    rc = lib.hs_prefill(fake, fake, fake, 1, 8, fake, fake, fake, 1, 4, 4, 4, 64, 32, 2,
                        0.1, 1, None, 0, None)
    assert rc == -2 and b"block_size == 16" in lib.hs_last_error()
    rc = lib.hs_kv_pack(None, 1, 8, 1024, None, 3, None, None)
    assert rc == -1
    assert lib.hs_kv_pack(None, 1, 8, 1024, None, 0, None, None) == 0      # nothing to do
    rc = lib.hs_kv_gather(fake, 8, 16, 512, fake, 2, 1, 33, fake, None)
    assert rc == -1 and b"capacity" in lib.hs_last_error()
    rc = lib.hs_profile_next_launch(fake, None)
    assert rc == -1
    assert lib.hs_profile_next_launch(None, None) == 0
    # writes of new K/V rows
    rc = lib.hs_kv_scatter(fake, fake, 2, 128, 4, 64, fake, 3, fake, fake, 0, 100, None)
    assert rc == -1 and b"stride" in lib.hs_last_error()
    rc = lib.hs_kv_scatter(fake, fake, 7, 128, 4, 64, fake, 3, fake, fake, 0, 256, None)
    assert rc == -1 and b"dtype" in lib.hs_last_error()
    rc = lib.hs_kv_scatter(fake, fake, 2, 128, 4, 64, None, 3, fake, fake, 0, 256, None)
    assert rc == -1 and b"null" in lib.hs_last_error()
    assert lib.hs_kv_scatter(None, None, 2, 128, 4, 64, None, 0, None, None, 0, 256, None) == 0
    rc = lib.hs_kv_append(fake, fake, 2, 8, 0, 4, 64, fake, 1, 2, fake, None, 3, fake, fake, 0,
                          256, None)
    assert rc == -1 and b"positive" in lib.hs_last_error()
    rc = lib.hs_kv_append(fake, fake, 2, 8, 16, 4, 64, fake, 0, 2, fake, None, 3, fake, fake, 0,
                          256, None)                              # no table rows
    assert rc == -1 and b"positive" in lib.hs_last_error()
    rc = lib.hs_kv_append(fake, fake, 2, 8, 16, 4, 64, None, 1, 2, fake, None, 3, fake, fake, 0,
                          256, None)
    assert rc == -1 and b"null" in lib.hs_last_error()


def test_extreme_sizes_are_refused_not_wrapped(lib):
    """Sizes near the int limits: the size queries return 0 (cannot serve)
    rather than a wrapped value, and the entry points fail with a reason before
    touching the device.  tests/test_sanitized_abi.py runs this under UBSan,
    which aborts on any signed overflow in the size and grid arithmetic."""
    M = 2 ** 31 - 1
    fake = ctypes.c_void_p(0x1000)
    assert lib.hs_decode_workspace_bytes(M, M, 1, 256, 16, M, 0, 16) == 0
    assert lib.hs_decode_workspace_bytes(M, 32, 32, 128, 16, M, 0, 0) == 0
    assert lib.hs_decode_workspace_bytes(M, M, M, 256, M, M, 0, 0) == 0
    # large but representable: reported exactly (P = 64 splits, (D + 2) floats)
    assert lib.hs_decode_workspace_bytes(M, 64, 1, 128, 16, M, 64, 0) == M * 64 * 64 * 520
    assert lib.hs_decode_shared_workspace_bytes(M, 32, 32, 128, 16, M, 0) == 0
    assert lib.hs_prefill_workspace_bytes(M, M, M, 128, 1) == 0
    rc = lib.hs_decode(fake, fake, fake, 2, 8, fake, fake, fake, M, 32, 32, 128, 16, M, 0.1,
                       0, 0, fake, 2 ** 62, None)
    assert rc == -2 and b"too large" in lib.hs_last_error()
    rc = lib.hs_decode_noalloc(fake, fake, fake, 2, 8, fake, fake, fake, M, 32, 32, 128, 16, M,
                               0.1, 0, 0, None)
    assert rc == -2 and b"too large" in lib.hs_last_error()
    rc = lib.hs_prefill(fake, fake, fake, 2, 8, fake, fake, fake, M, M, 4, 4, 64, 16, 2, 0.1,
                        1, None, 0, None)
    assert rc == -1 and b"too large" in lib.hs_last_error()
    rc = lib.hs_kv_pack(fake, M, M, 2 ** 62, fake, M, fake, None)
    assert rc == -2 and b"too large" in lib.hs_last_error()
    rc = lib.hs_kv_gather(fake, 8, 16, 2 ** 62, fake, M, M, M, fake, None)
    assert rc == -2 and b"too large" in lib.hs_last_error()
    rc = lib.hs_kv_scatter(fake, fake, 2, 2 ** 62, 4, 64, fake, 3, fake, fake, 0, 2 ** 62, None)
    assert rc == -2 and b"too large" in lib.hs_last_error()


def test_workspace_size_formula(lib):
    """hs_decode's workspace: (rows * H * P * D) floats, padded to 256 bytes,
    then rows * H * P (max, sum) pairs; P = ceil(MB * BS / partition).  The
    default partition is 512 tokens, min(512, 1024 / G) when one wave serves
    G query heads of a GQA group (G = 1, 2, 4, 8, the largest dividing H / Hkv),
    and 512 again when H / Hkv >= 8 and Hkv * ceil(H / Hkv / 32) <= 2.  bf16
    caches with 2 or more query heads per KV head (16-token pages, head_dim
    64/128) default to 768 tokens up to 4 heads per KV head, 384 up to 8 and
    256 above; the query takes no dtype, so it sizes for the shortest."""
    B, H, D, BS, MB = 3, 5, 128, 16, 100

    def ws(P):
        acc = (B * H * P * D * 4 + 255) // 256 * 256
        return acc + B * H * P * 8

    for part, P in ((256, 7), (512, 4), (16, 100)):
        assert lib.hs_decode_workspace_bytes(B, H, H, D, BS, MB, 0, part) == ws(P)
    assert lib.hs_decode_workspace_bytes(B, H, H, D, BS, MB, 9, 0) == ws(9)
    H = 32
    for Hkv, part in ((32, 512), (16, 512), (8, 256), (4, 128), (1, 256), (2, 256)):
        P = -(-(MB * BS) // part)
        acc = (B * H * P * D * 4 + 255) // 256 * 256
        assert lib.hs_decode_workspace_bytes(B, H, Hkv, D, BS, MB, 0, 0) == acc + B * H * P * 8
    H = 96                                     # G = 96: three 32-head waves per KV head
    for Hkv, part in ((1, 128), (3, 128)):
        P = -(-(MB * BS) // part)
        acc = (B * H * P * D * 4 + 255) // 256 * 256
        assert lib.hs_decode_workspace_bytes(B, H, Hkv, D, BS, MB, 0, 0) == acc + B * H * P * 8
    assert lib.hs_decode_workspace_bytes(B, H, 5, D, BS, MB, 0, 0) == 0   # H % Hkv != 0


def test_module_state_without_a_device(monkeypatch):
    """On a host without a HIP device the modules report why, keep the
    reference's availability API, and raise instead of computing."""
    import torch

    from heteroserve.model import (paged_attn, paged_attn_prefill, paged_attn_v2,
                                   paged_attn_v3, paged_attn_wmma)

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    assert paged_attn.which_backend() == "torch"
    assert "no HIP device" in paged_attn.build_error()
    for m in (paged_attn_v2, paged_attn_v3, paged_attn_prefill, paged_attn_wmma):
        assert m.is_available() is False
        assert m.build_error()
    q = torch.zeros(1, 4, 64)
    k = torch.zeros(4, 16, 4, 64)
    bt = torch.zeros(1, 1, dtype=torch.int32)
    ctx = torch.ones(1, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="unavailable"):
        paged_attn.paged_attention(q, k, k, bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="unavailable"):
        paged_attn_v2.paged_attention_v2(q, k, k, bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="unavailable"):
        paged_attn_v3.paged_attention_v3(q, k, k, bt, ctx, 0.1, 4)
    with pytest.raises(RuntimeError, match="unavailable"):
        paged_attn_prefill.paged_attention_prefill(q[:, None], k, k, bt, ctx, 0.1)
    with pytest.raises(RuntimeError, match="unavailable"):
        paged_attn_wmma.paged_attention_prefill_wmma(q[:, None], k, k, bt, ctx, 0.1)
    # the reference's geometry gate (tests/test_torch_engine.py:642-653)
    assert paged_attn_wmma.supports(32, 64, torch.float16) is False
    assert paged_attn_wmma.supports(16, 64, torch.float32) is False
    assert paged_attn_wmma.supports(16, 48, torch.float16) is False
    assert paged_attn_v2.bytes_moved(16, 512, 12, 64, 2) == 25_165_824
    assert paged_attn_v2.peak_bandwidth_gbs() is None


def test_disable_flag_is_honoured(monkeypatch):
    """HETEROSERVE_DISABLE_CUDA_KERNEL (reference paged_attn.py:208-210)."""
    import importlib

    from heteroserve import _hip

    monkeypatch.setenv("HETEROSERVE_DISABLE_CUDA_KERNEL", "1")
    fresh = importlib.reload(_hip)
    try:
        assert not fresh.ready()
        assert "HETEROSERVE_DISABLE_CUDA_KERNEL" in fresh.error()
    finally:
        monkeypatch.delenv("HETEROSERVE_DISABLE_CUDA_KERNEL")
        importlib.reload(_hip)


def test_errors_are_per_thread(lib):
    """hs_last_error is thread-local: hetero-serve's worker calls the library
    from its executor thread (the step) and its event-loop thread (pack and
    unpack) at the same time (worker.py:448, :527, :562-563), so one thread's
    failure must never show up as the other's message.  Two threads fail in
    different ways, many times over, and each reads back only its own."""
    import threading

    fake = ctypes.c_void_p(0x1000)
    seen = {"a": set(), "b": set()}
    start = threading.Barrier(2)

    def fail_divisible():
        start.wait()
        for _ in range(2000):
            rc = lib.hs_decode(fake, fake, fake, 0, 8, fake, fake, fake, 1, 6, 4, 64, 16, 2,
                               0.1, 0, 0, None, 0, None)
            assert rc == -1
            seen["a"].add(lib.hs_last_error())

    def fail_block_size():
        start.wait()
        for _ in range(2000):
            rc = lib.hs_prefill(fake, fake, fake, 1, 8, fake, fake, fake, 1, 4, 4, 4, 64, 32, 2,
                                0.1, 1, None, 0, None)
            assert rc == -2
            seen["b"].add(lib.hs_last_error())

    threads = [threading.Thread(target=fail_divisible), threading.Thread(target=fail_block_size)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert len(seen["a"]) == 1 and b"divisible" in next(iter(seen["a"]))
    assert len(seen["b"]) == 1 and b"block_size == 16" in next(iter(seen["b"]))
