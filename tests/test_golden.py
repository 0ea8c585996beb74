"""Known-answer vectors (tests/golden/paged_attention_golden.npz).

The fixture holds, per case, a digest of the reference test suite's inputs and
the fp64 brute-force output for them (tests/golden/make_golden.py).  The CPU
tests rebuild every input, check its digest and hold the oracle to the stored
answer; the GPU tests hold libhsattn's entry points to the same answers, so
the kernels are checked against numbers fixed once, not only against code
that runs beside them.
"""

from __future__ import annotations

import hashlib
import sys
from pathlib import Path

import numpy as np
import pytest

torch = pytest.importorskip("torch")

sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))

import make_golden as mg  # noqa: E402
import oracle.attention as att  # noqa: E402
import oracle.kvpack as kvp  # noqa: E402
import oracle.recurrences as rec  # noqa: E402
from _refcases import (ONLINE_CASES, PREFILL_CASES, SPLIT_CASES, WMMA_TILING_CASES,  # noqa: E402
                       build_paged_case, cpu_fuzz_trials, pack_case, prefill_case,
                       recurrence_case, single_head_case, table_array)

DEV = "cuda:0"
KV_TORCH = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16}


@pytest.fixture(scope="module")
def golden():
    with np.load(mg.FIXTURE) as f:
        return {k: f[k] for k in f.files}


def paged_cases():
    """(name, kind, kv dtype, inputs) for every paged case in the fixture.

    inputs = (q, k_cache, v_cache, block_tables, context_lens, scale) as
    numpy arrays in the dtypes the digest was taken over (fp32 caches; the
    kv dtype says what the test casts them to).
    """
    for seed in (5, 9):
        c = build_paged_case(seed=seed)
        for layer in (0, 3):
            yield (f"decode_seed{seed}_L{layer}", "decode", "f32",
                   (*mg.decode_inputs(c, layer), c["scale"]))
    c = build_paged_case(seed=5)
    for kv in ("f16", "bf16"):
        yield f"decode_seed5_L0_{kv}", "decode", kv, (*mg.decode_inputs(c, 0), c["scale"])
    for c in cpu_fuzz_trials(mg.FUZZ_TRIALS):
        yield f"decode_fuzz{c['trial']}", "decode", "f32", (*mg.decode_inputs(c, 0), c["scale"])
    for i, (lens, S, kvh) in enumerate(PREFILL_CASES):
        c = prefill_case(lens, S, kvh, seed=len(lens) * 7 + S)
        ins = (c["q"], c["pool"][0, 0], c["pool"][0, 1], table_array(c["tables"]),
               np.asarray(lens, dtype=np.int32), c["scale"])
        yield f"prefill{i}", "prefill", "f32", ins
        if i >= 2:
            yield f"prefill{i}_f16", "prefill", "f16", ins
    for ctx, S, D in WMMA_TILING_CASES:
        yield (f"tiled_{ctx}_{S}_{D}_paged_f16", "prefill", "f16",
               (*mg.tiled_paged(ctx, S, D), D ** -0.5))


PAGED = list(paged_cases())


def _digest_inputs(ins):
    return mg.digest(*ins[:5])


# ---------------------------------------------------------------------------
# CPU: inputs rebuild bit for bit, and the oracle gives the stored answers
# ---------------------------------------------------------------------------


def test_fixture_is_complete(golden):
    names = {k.rsplit("__", 1)[0] for k in golden}
    want = {n for n, *_ in PAGED}
    want |= {f"tiled_{c}_{s}_{d}" for c, s, d in WMMA_TILING_CASES}
    want |= {f"online_{n}_{a:g}" for n, a in ONLINE_CASES}
    want |= {f"split_{n}_{s}_{a:g}" for n, s, a in SPLIT_CASES}
    want |= {"pack_model"}
    assert names == want


@pytest.mark.parametrize("name,kind,kv,ins", PAGED, ids=[p[0] for p in PAGED])
def test_paged_inputs_and_oracle(golden, name, kind, kv, ins):
    assert _digest_inputs(ins) == str(golden[f"{name}__digest"]), "inputs no longer rebuild"
    q, kc, vc, bt, ctx, scale = ins
    args = (torch.as_tensor(q), torch.as_tensor(kc).to(KV_TORCH[kv]),
            torch.as_tensor(vc).to(KV_TORCH[kv]), torch.as_tensor(bt), torch.as_tensor(ctx),
            scale)
    fn = att.paged_attention_torch if kind == "decode" else att.paged_attention_prefill_torch
    got = fn(*args).numpy()
    np.testing.assert_allclose(got, golden[f"{name}__expected"], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("ctx,S,D", WMMA_TILING_CASES)
def test_tiled_recurrence_against_golden(golden, ctx, S, D):
    q, k, v = single_head_case(ctx, S, D)
    name = f"tiled_{ctx}_{S}_{D}"
    assert mg.digest(q, k, v) == str(golden[f"{name}__digest"])
    np.testing.assert_allclose(rec.tiled_prefill_reference(q, k, v, D ** -0.5, ctx),
                               golden[f"{name}__expected"], rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("n,amp", ONLINE_CASES)
def test_online_softmax_against_golden(golden, n, amp):
    q, k, v = recurrence_case(n, n, amp)
    name = f"online_{n}_{amp:g}"
    assert mg.digest(q, k, v) == str(golden[f"{name}__digest"])
    np.testing.assert_allclose(rec.online_softmax_reference(q, k, v, 1 / 8),
                               golden[f"{name}__expected"], rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("n,splits,amp", SPLIT_CASES)
def test_split_merge_against_golden(golden, n, splits, amp):
    q, k, v = recurrence_case(n * 31 + splits, n, amp)
    name = f"split_{n}_{splits}_{amp:g}"
    assert mg.digest(q, k, v) == str(golden[f"{name}__digest"])
    np.testing.assert_allclose(rec.split_merge_reference(q, k, v, 1 / 8, splits),
                               golden[f"{name}__expected"], rtol=1e-4, atol=1e-4)


def test_pack_oracle_against_golden(golden):
    p = pack_case()
    ids = np.asarray(p["ids"], dtype=np.int64)
    assert mg.digest(p["pool"], ids) == str(golden["pack_model__digest"])
    packed = kvp.export_blocks(p["pool"], p["ids"])
    assert hashlib.sha256(np.ascontiguousarray(packed).tobytes()).hexdigest() == \
        str(golden["pack_model__packed_sha256"])


def test_generator_reproduces_the_fixture(golden):
    fresh = mg.build()
    assert set(fresh) == set(golden)
    for k, v in fresh.items():
        if v.dtype.kind == "U":
            assert str(v) == str(golden[k]), k
        else:
            np.testing.assert_allclose(v, golden[k], rtol=0, atol=1e-6, err_msg=k)


# ---------------------------------------------------------------------------
# GPU: libhsattn against the stored answers
# ---------------------------------------------------------------------------


def _dev(ins, kv):
    q, kc, vc, bt, ctx, scale = ins
    return (torch.as_tensor(q, device=DEV),
            torch.as_tensor(kc).to(DEV, KV_TORCH[kv]), torch.as_tensor(vc).to(DEV, KV_TORCH[kv]),
            torch.as_tensor(bt, device=DEV), torch.as_tensor(ctx, device=DEV), scale)


def _err(got, want):
    return float(np.abs(got.detach().float().cpu().numpy() - want).max())


@pytest.mark.gpu
@pytest.mark.parametrize("name,kind,kv,ins", PAGED, ids=[p[0] for p in PAGED])
def test_library_against_golden(golden, name, kind, kv, ins):
    """fp32 caches: the reference's 1e-3 gate; fp16/bf16: the 2e-3 gate."""
    from heteroserve.model import (paged_attn, paged_attn_prefill, paged_attn_v2, paged_attn_v3,
                                   paged_attn_wmma)

    want = golden[f"{name}__expected"]
    args = _dev(ins, kv)
    tol = 1e-3 if kv == "f32" else 2e-3
    if kind == "decode":
        outs = {"v1": paged_attn.paged_attention(*args),
                "v2": paged_attn_v2.paged_attention_v2(*args)}
        for n in (0, 1, 3, 16):
            outs[f"v3/{n}"] = paged_attn_v3.paged_attention_v3(*args, num_splits=n)
    else:
        outs = {}
        if kv == "f32":
            outs["scalar"] = paged_attn_prefill.paged_attention_prefill(*args)
        block_size, head_dim = args[1].shape[1], args[1].shape[3]
        if paged_attn_wmma.supports(block_size, head_dim, args[1].dtype):
            outs["mfma"] = paged_attn_wmma.paged_attention_prefill_wmma(*args)
        assert outs, f"{name}: no prefill kernel serves this case"
    for label, got in outs.items():
        err = _err(got, want)
        assert err <= tol, f"{name} [{label}]: max |err| {err:.2e} > {tol:g}"


@pytest.mark.gpu
def test_pack_against_golden(golden):
    from heteroserve.kv import pack

    p = pack_case()
    payload = pack.export_blocks_device(torch.as_tensor(p["pool"], device=DEV), p["ids"])
    raw = payload.cpu().contiguous().view(torch.uint8).numpy().tobytes()
    assert hashlib.sha256(raw).hexdigest() == str(golden["pack_model__packed_sha256"])
