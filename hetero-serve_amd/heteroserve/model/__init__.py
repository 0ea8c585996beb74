"""Paged-attention entry points with hetero-serve's Python signatures."""
