"""KV-block movement (migration pack/unpack, contiguous gather) on the GPU."""
