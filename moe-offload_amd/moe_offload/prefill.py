"""Chunked prefill through a cached layer (loader.py:566-699) -- see cached_prefill."""
from __future__ import annotations


def cached_prefill(module, x, indices):
    raise NotImplementedError("prefill through a cached layer needs the grouped-GEMM kernel")
