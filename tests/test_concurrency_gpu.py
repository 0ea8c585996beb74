"""Concurrent use of libhsattn, the way hetero-serve's worker uses it.

The worker runs a step (paged decode) in its executor thread
(worker.py:562-563) while its event-loop thread exports and imports KV
blocks for migration (worker.py:448 pack, :527 unpack).  Here two Python
threads do the same on their own HIP streams (default priority), many times
over: the decode thread's outputs must stay bit-identical to a single-threaded
run, and every pack and unpack must stay bit-exact.  ctypes releases the GIL
around each library call, so the host layers of both threads really overlap.
"""

from __future__ import annotations

import threading

import numpy as np
import pytest

torch = pytest.importorskip("torch")

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _bits(t):
    width = {2: torch.int16, 4: torch.int32}[t.element_size()]
    return t.view(width)


def test_decode_and_migration_on_two_threads():
    from heteroserve import _hip
    from heteroserve.kv import pack
    from heteroserve.model import paged_attn
    from hsbench import cases

    assert _hip.ready(), _hip.error()
    rng = np.random.default_rng(11)
    ctx = rng.integers(200, 3000, size=24, endpoint=True)
    case = cases.build_decode("conc", ctx, 16, 16, 128, 8192, torch.bfloat16, DEV, 11, rng=rng)
    args = (case.q, case.k_cache, case.v_cache, case.block_tables, case.context_lens, case.scale)
    want = paged_attn.paged_attention(*args)          # single-threaded reference

    ids = rng.choice(case.pool.shape[2], size=512, replace=False).tolist()
    want_payload = pack.export_blocks_device(case.pool, ids)
    dst = torch.zeros_like(case.pool)                  # migration target: not read by decode
    new_ids = rng.choice(dst.shape[2], size=512, replace=False).tolist()
    torch.cuda.synchronize()

    iters = 60
    errors: list[str] = []
    start = threading.Barrier(2)

    def step_thread():
        s = torch.cuda.Stream(device=DEV)
        try:
            with torch.cuda.stream(s):
                start.wait()
                for i in range(iters):
                    got = paged_attn.paged_attention(*args)
                    if not torch.equal(_bits(got), _bits(want)):
                        errors.append(f"decode differs at iteration {i}")
                        return
        except Exception as e:   # reported by the main thread
            errors.append(f"decode thread: {e!r}")

    def migration_thread():
        s = torch.cuda.Stream(device=DEV)
        try:
            with torch.cuda.stream(s):
                start.wait()
                for i in range(iters):
                    payload = pack.export_blocks_device(case.pool, ids)
                    pack.write_blocks_device(dst, new_ids, payload)
                    if not torch.equal(_bits(payload), _bits(want_payload)):
                        errors.append(f"pack differs at iteration {i}")
                        return
                    if not torch.equal(_bits(dst[:, :, new_ids]), _bits(case.pool[:, :, ids])):
                        errors.append(f"unpack differs at iteration {i}")
                        return
        except Exception as e:
            errors.append(f"migration thread: {e!r}")

    threads = [threading.Thread(target=step_thread), threading.Thread(target=migration_thread)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads), "a worker thread did not finish"
    torch.cuda.synchronize()
    assert not errors, errors
