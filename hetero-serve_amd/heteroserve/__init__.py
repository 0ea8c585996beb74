"""hetero-serve's paged-attention hot path, rebuilt for MI355X (gfx950).

Only the modules on that path exist here: ``model.paged_attn*`` (decode and
prefill attention entry points with the reference's signatures) and
``kv.pack`` (KV-block pack / unpack / gather).  Their kernels live in
libhsattn.so, loaded through ``heteroserve._hip``.
"""
