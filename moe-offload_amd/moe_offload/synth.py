"""Seeded synthetic workloads for the routed-expert decode path.

The reference runs a real checkpoint; without one, every workload here is synthetic, drawn
from `numpy.random.default_rng` with a fixed seed per stream so the GPU path and the CPU
oracle see identical inputs.

  expert_id_stream  single-layer decode id stream: each step draws `k` distinct ids, each
                    with probability `p_reuse` re-used from the previous `window` steps' ids,
                    otherwise drawn from Zipf(s) over the experts (popularity rank mapped to
                    expert ids through a seeded permutation).
  q2_experts        MLX-layout 2-bit g64 expert tensors: codes ~ U{0..3}, scale ~ N(0, std)
                    in fp16, bias = -1.5 * scale.
  router_weight     fp16 [E, H] ~ N(0, 0.02).
"""
from __future__ import annotations

import numpy as np


def expert_id_stream(steps: int = 128, k: int = 10, num_experts: int = 512, zipf_s: float = 1.1,
                     p_reuse: float = 0.7, window: int = 4, seed: int = 2) -> np.ndarray:
    rng = np.random.default_rng(seed)
    w = 1.0 / np.arange(1, num_experts + 1, dtype=np.float64) ** zipf_s
    w /= w.sum()
    cdf = np.cumsum(w)
    perm = rng.permutation(num_experts)
    hist: list[list[int]] = []
    out = np.zeros((steps, k), np.uint32)
    for t in range(steps):
        pool: list[int] = []
        for ids in hist[-window:]:
            for e in ids:
                if e not in pool:
                    pool.append(e)
        ids: list[int] = []
        while len(ids) < k:
            if pool and rng.random() < p_reuse:
                e = pool[int(rng.integers(len(pool)))]
            else:
                r = int(np.searchsorted(cdf, rng.random(), side="right"))
                e = int(perm[min(r, num_experts - 1)])
            if e not in ids:
                ids.append(e)
        hist.append(ids)
        out[t] = ids
    return out


def q2_experts(num_experts: int, hidden: int, inter: int, group: int = 64, scale_std: float = 0.02,
               seed: int = 1):
    """Per-projection MLX-layout tensors (w uint32, scales fp16, biases fp16) for gate/up/down."""
    rng = np.random.default_rng(seed)

    def proj(out_f: int, in_f: int):
        w = rng.integers(0, 2**32, size=(num_experts, out_f, in_f // 16), dtype=np.uint32)
        s = (rng.standard_normal((num_experts, out_f, in_f // group)) * scale_std).astype(np.float16)
        b = (-1.5 * s.astype(np.float32)).astype(np.float16)
        return w, s, b

    gate = proj(inter, hidden)
    up = proj(inter, hidden)
    down = proj(hidden, inter)
    return gate, up, down


def router_weight(num_experts: int, hidden: int, std: float = 0.02, seed: int = 3) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((num_experts, hidden)) * std).astype(np.float16)


def hidden_states(n: int, hidden: int, seed: int = 4) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((n, hidden)).astype(np.float16)


def prefill_routing(n_tok: int = 512, k: int = 10, num_experts: int = 512, sigma: float = 0.34,
                    seed: int = 6):
    """Top-k routing of one prefill chunk: softmax over N(0,1) logits plus a per-expert
    popularity offset ~ N(0, sigma), which stretches tokens-per-expert from ~Binomial (max ~22)
    to a long tail (max 62 at the defaults, mean 10, 496 of 512 experts touched).

    Returns (ids int32 [n_tok, k] in ascending-gate order, scores fp16 [n_tok, k] renormalised).
    """
    rng = np.random.default_rng(seed)
    off = rng.standard_normal(num_experts) * sigma
    logits = rng.standard_normal((n_tok, num_experts)) + off[None]
    g = np.exp(logits - logits.max(axis=1, keepdims=True))
    g /= g.sum(axis=1, keepdims=True)
    ids = np.argsort(g, axis=1, kind="stable")[:, -k:]
    sel = np.take_along_axis(g, ids, axis=1)
    scores = (sel / sel.sum(axis=1, keepdims=True)).astype(np.float16)
    return ids.astype(np.int32), scores
