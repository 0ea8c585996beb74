"""Measurement harness of the paged-attention path: synthetic configurations
(``cases``) and timing helpers (``timing``)."""
