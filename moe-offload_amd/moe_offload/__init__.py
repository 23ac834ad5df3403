"""moe_offload -- MI355X-native routed-expert decode path (fused router, Q2 gather-GEMV,
HBM slot-pool LRU, miss staging from a pinned host expert store).

The compute and the expert cache live in libmoe_offload.so (HIP, gfx950); this package holds
the host side that mirrors the reference loader's API (`mlx-qwen38/loader.py`).
"""
from . import _lib, q2format, synth  # noqa: F401

__all__ = ["_lib", "q2format", "synth"]
