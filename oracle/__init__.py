"""CPU oracle for the routed-expert decode path -- TEST INFRASTRUCTURE ONLY.

Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
anything from this package, and only as the reference the results are compared with (or the timed
CPU baseline), never as the thing measured or shipped.  The product path (`moe-offload_amd/`) never imports it and fails
loudly when its HIP library is missing.

Contents
  q2.py   numpy restatement of the MLX affine group-quantised format, the router rule
          (softmax -> ascending top-k -> renormalise), the next-layer predictor, SwitchGLU,
          the decode stack layer and the prefill chunk/slot bookkeeping.
  lru.c   plain-C restatement of the per-layer slot LRU of `mlx-qwen38/expert_io.c`
          (decode step, router prefetch, state get/set, counters), loaded through `lru.py`.
  lru.py  ctypes binding of lru.c plus an independent pure-Python restatement (OrderedDict
          form, as `mlx-qwen38/loader.py:482-490` keeps it) used to cross-check the C one.
  Makefile builds lru.c into `_build/` and, where the reference tree is present, the
          reference's own `expert_io.c` into `_ref/` (used only to write golden traces).

Pinning (which independent check covers each function) is listed in each module header.
"""
