"""Write tests/golden/paged_attention_golden.npz: known-answer vectors.

Every case replays an input of the reference test suite (its seeds, its
geometry, its RNG call order -- tests/_refcases.py) and stores

* ``<case>__digest``: sha256 of the input bytes in a fixed order, so a change
  in how the inputs are rebuilt (RNG order, block layout, a cast) is caught
  before any output is compared;
* ``<case>__expected``: the output computed by fp64 brute force over the
  gathered true context (tests/_dense.py), which shares no code with the
  oracle or the kernels.  Stored as float32 (the kernels' output type).

The inputs themselves are rebuilt by the tests from the same seeds (they are
megabytes; the digests pin them).  Run from the repository root:

    python tests/golden/make_golden.py          # rewrite the fixture
    python tests/golden/make_golden.py --check  # compare with the committed one
"""

from __future__ import annotations

import argparse
import hashlib
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))

from _dense import dense_causal, dense_decode  # noqa: E402
from _refcases import (ONLINE_CASES, PREFILL_CASES, SPLIT_CASES, WMMA_TILING_CASES,  # noqa: E402
                       build_paged_case, cpu_fuzz_trials, lay_out, pack_case, prefill_case,
                       recurrence_case, single_head_case, table_array)

FIXTURE = HERE / "paged_attention_golden.npz"
FUZZ_TRIALS = 10          # first trials of tests/test_torch_engine.py:359-402


def digest(*arrays) -> str:
    h = hashlib.sha256()
    for a in arrays:
        a = np.ascontiguousarray(a)
        h.update(str(a.dtype).encode())
        h.update(str(a.shape).encode())
        h.update(a.tobytes())
    return h.hexdigest()


def round_to(x: np.ndarray, kv_dtype: str) -> np.ndarray:
    """Values of x after a cast to the KV cache dtype (RNE), as float64."""
    if kv_dtype == "f32":
        return x.astype(np.float32).astype(np.float64)
    if kv_dtype == "f16":
        return x.astype(np.float16).astype(np.float64)
    if kv_dtype == "bf16":
        b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
        b = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16     # round to nearest even
        return b.astype(np.uint32).view(np.float32).astype(np.float64)
    raise ValueError(kv_dtype)


# ---------------------------------------------------------------------------
# case builders: each returns (inputs for the digest, expected output)
# ---------------------------------------------------------------------------


def decode_inputs(c, layer):
    pool = c["pool"][layer]
    return (c["q"], pool[0], pool[1], table_array(c["tables"]),
            np.asarray(c["lens"], dtype=np.int32))


def decode_expected(c, layer, kv_dtype="f32"):
    out = []
    for b, (k, v) in enumerate(c["seqs"]):
        out.append(dense_decode(c["q"][b], round_to(k[layer].transpose(1, 0, 2), kv_dtype),
                                round_to(v[layer].transpose(1, 0, 2), kv_dtype), c["scale"]))
    return np.stack(out)


def prefill_expected(c, layer, kv_dtype="f32"):
    S = c["S"]
    out = []
    for b, (k, v) in enumerate(c["seqs"]):
        out.append(dense_causal(c["q"][b], round_to(k[layer].transpose(1, 0, 2), kv_dtype),
                                round_to(v[layer].transpose(1, 0, 2), kv_dtype), c["scale"],
                                c["lens"][b] - S))
    return np.stack(out)


def tiled_paged(ctx, S, D):
    """A single-head WMMA tiling case laid out as a BS-16 fp16 paged cache.

    Returns q [1, S, 1, D] float32, k/v caches [NB, 16, 1, D] float16, the
    block table and context lengths: the inputs the MFMA prefill kernel is
    given for tests/test_torch_engine.py:610-639's cases.
    """
    q, k, v = single_head_case(ctx, S, D)
    kk = k.astype(np.float16)[None, None]          # [L=1, Hkv=1, ctx, D]
    vv = v.astype(np.float16)[None, None]
    nb = -(-ctx // 16) + 2
    pool, tables = lay_out([(kk, vv)], 16, nb, 1, np.float16)
    return (q.astype(np.float32)[None, :, None, :], pool[0, 0], pool[0, 1],
            table_array(tables), np.asarray([ctx], dtype=np.int32))


def build() -> dict[str, np.ndarray]:
    fx: dict[str, np.ndarray] = {}

    def put(name, inputs, expected):
        fx[f"{name}__digest"] = np.asarray(digest(*inputs))
        fx[f"{name}__expected"] = np.asarray(expected, dtype=np.float32)

    # decode: tests/test_torch_engine.py:179-196 (seed 5) and :303-319 (seed 9)
    for seed in (5, 9):
        c = build_paged_case(seed=seed)
        for layer in (0, 3):
            put(f"decode_seed{seed}_L{layer}", decode_inputs(c, layer), decode_expected(c, layer))
    c = build_paged_case(seed=5)
    for kv in ("f16", "bf16"):
        put(f"decode_seed5_L0_{kv}", decode_inputs(c, 0), decode_expected(c, 0, kv))

    # decode fuzz: :359-402
    for c in cpu_fuzz_trials(FUZZ_TRIALS):
        put(f"decode_fuzz{c['trial']}", decode_inputs(c, 0), decode_expected(c, 0))

    # prefill: :518-546 (seed as the oracle pins use it)
    for i, (lens, S, kvh) in enumerate(PREFILL_CASES):
        c = prefill_case(lens, S, kvh, seed=len(lens) * 7 + S)
        ins = (c["q"], c["pool"][0, 0], c["pool"][0, 1], table_array(c["tables"]),
               np.asarray(lens, dtype=np.int32))
        put(f"prefill{i}", ins, prefill_expected(c, 0))
        if i >= 2:        # ragged batch, GQA, MQA and S = 1 for the fp16 caches
            put(f"prefill{i}_f16", ins, prefill_expected(c, 0, "f16"))

    # WMMA tiling: :610-639, exact (fp64 inputs) and as fp16 paged caches
    for ctx, S, D in WMMA_TILING_CASES:
        q, k, v = single_head_case(ctx, S, D)
        want = dense_causal(q[:, None], k[:, None], v[:, None], D ** -0.5, ctx - S)[:, 0]
        put(f"tiled_{ctx}_{S}_{D}", (q, k, v), want)
        qp, kc, vc, bt, lens = tiled_paged(ctx, S, D)
        kd = k.astype(np.float16).astype(np.float64)[:, None]
        vd = v.astype(np.float16).astype(np.float64)[:, None]
        want16 = dense_causal(qp[0].astype(np.float64), kd, vd, D ** -0.5, ctx - S)
        put(f"tiled_{ctx}_{S}_{D}_paged_f16", (qp, kc, vc, bt, lens), want16[None])

    # recurrences: :257-281 and :327-356
    for n, amp in ONLINE_CASES:
        q, k, v = recurrence_case(n, n, amp)
        put(f"online_{n}_{amp:g}", (q, k, v), dense_decode(q, k, v, 1 / 8))
    for n, splits, amp in SPLIT_CASES:
        q, k, v = recurrence_case(n * 31 + splits, n, amp)
        put(f"split_{n}_{splits}_{amp:g}", (q, k, v), dense_decode(q, k, v, 1 / 8))

    # pack: tests/test_model.py:106-124.  out[i, l, c] = pool[l, c, ids[i]]
    p = pack_case()
    pool, ids = p["pool"], np.asarray(p["ids"], dtype=np.int64)
    packed = np.stack([pool[:, :, i] for i in ids])
    fx["pack_model__digest"] = np.asarray(digest(pool, ids))
    fx["pack_model__packed_sha256"] = np.asarray(hashlib.sha256(packed.tobytes()).hexdigest())
    # the same bytes, read sequence-major from the k/v the test wrote
    kv = np.stack([p["k"], p["v"]], axis=1)                  # [L, 2, H, 16, D]
    per_block = kv.reshape(kv.shape[0], 2, kv.shape[2], len(ids), 4, kv.shape[4])
    assert np.array_equal(packed, per_block.transpose(3, 0, 1, 4, 2, 5))
    return fx


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--check", action="store_true", help="compare with the committed fixture")
    args = ap.parse_args()
    fx = build()
    if args.check:
        with np.load(FIXTURE) as old:
            bad = [k for k in fx if k not in old.files or not (
                np.array_equal(old[k], fx[k]) if fx[k].dtype.kind == "U"
                else np.allclose(old[k], fx[k], rtol=0, atol=1e-6))]
            bad += [k for k in old.files if k not in fx]
        print("fixture matches" if not bad else f"differs: {bad}")
        return 1 if bad else 0
    np.savez_compressed(FIXTURE, **fx)
    print(f"wrote {FIXTURE} ({FIXTURE.stat().st_size} bytes, {len(fx) // 2} cases)")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
