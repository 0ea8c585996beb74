"""CPU oracle for hetero-serve's paged-attention hot path -- TEST INFRASTRUCTURE.

A restatement, in torch (CPU) and numpy, of the reference algorithms the HIP
kernels must reproduce.  Every function cites the reference file:line it
follows (paths relative to the hetero-serve checkout).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed CPU
baseline.  The product (``hetero-serve_amd/``) never imports it and has no CPU
fallback: its entry points raise when libhsattn.so is unavailable.

Every function here is pinned by checks that do not restate it
(tests/test_oracle.py, tests/test_golden.py): fp64 dense brute force on the
reference tests' own parameter sets, closed forms, invariances, explicit
index loops for the pack permutation, and planted mistakes that those checks
must catch.  There is no ``oracle/_ref`` build: the reference's kernels are
CUDA source embedded in Python strings and need nvcc plus torch's extension
builder, which this image does not have.

    attention     paged_attention_torch, paged_attention_prefill_torch,
                  per-sequence forms for configurations too large to pad
    recurrences   online_softmax_reference, split_merge_reference,
                  tiled_prefill_reference, NEG_BIG
    kvpack        export_blocks, write_blocks (numpy and torch forms),
                  gather_kv_batch, KV-row writes, block tables
    splits        choose_num_splits
"""
