"""Host bookkeeping of the cached-layer prefill (moe_offload.prefill) against the oracle plan.

The product walks the chunks itself (sort, per-chunk slot plan, final LRU, counters); this
checks every piece against oracle.prefill_plan on random LRU states, capacities and id
multisets, including the empty prefill.  No GPU needed.
"""
import numpy as np
import pytest

from moe_offload import prefill
from oracle import q2


def _product_plan(ids, prior_e, prior_s, cap, k=1):
    order, idx_s, uniq, first_pos, counts = prefill.sort_rows(ids, k)
    hits, misses = prefill.prefill_counts(uniq, counts, set(prior_e))
    s2e = dict(zip(prior_s, prior_e))
    e2s = dict(zip(prior_e, prior_s))
    chunks = []
    for u0 in range(0, len(uniq), cap):
        u1 = min(len(uniq), u0 + cap)
        le, ls = prefill.plan_chunk([int(e) for e in uniq[u0:u1]], s2e, e2s)
        chunks.append((u0, u1, le, ls))
    last = (chunks[-1][1] - chunks[-1][0]) if chunks else 0
    return order, uniq, chunks, prefill.final_lru(s2e, last, cap), hits, misses


def test_prefill_host_plan_matches_oracle():
    rng = np.random.default_rng(7)
    for trial in range(300):
        cap = int(rng.choice([16, 40, 102, 512]))
        n_prior = int(rng.integers(0, cap + 1))
        prior_e = [int(e) for e in rng.choice(512, size=n_prior, replace=False)]
        prior_s = [int(s) for s in rng.choice(cap, size=n_prior, replace=False)]
        m = int(rng.choice([0, 1, 7, 64, 640, 5120]))
        hot = rng.choice(512, size=int(rng.integers(1, 513)), replace=False)
        ids = rng.choice(hot, size=m)
        want = q2.prefill_plan(ids, prior_e, prior_s, cap)
        order, uniq, chunks, new_lru, hits, misses = _product_plan(ids, prior_e, prior_s, cap)
        assert np.array_equal(order, want["order"]), trial
        assert np.array_equal(uniq, want["uniq"]), trial
        assert chunks == [(a, b, list(c), list(d)) for a, b, c, d in want["chunks"]], trial
        assert new_lru == (list(want["new_lru"][0]), list(want["new_lru"][1])), trial
        assert (hits, misses) == (want["add_hits"], want["add_misses"]), trial


def test_resident_plan_rows():
    ids = np.array([[5, 3], [3, 9], [5, 5]], np.int32)
    row_tok, row_out, seg, slot = prefill.resident_plan(ids, 2)
    assert slot.tolist() == [3, 5, 9]
    assert seg.tolist() == [0, 2, 5, 6]
    assert row_out.tolist() == [1, 2, 0, 4, 5, 3]          # stable within an expert
    assert row_tok.tolist() == [0, 1, 0, 2, 2, 1]


def test_tile_segments_known_answer():
    # [0,5) slot 3; an empty segment (dropped); [5,40) slot 9 -> 16 + 16 + 3 rows; [40,48) slot 2
    seg, slot = prefill.tile_segments(np.array([0, 5, 5, 40, 48]), np.array([3, 7, 9, 2]))
    assert seg.tolist() == [0, 5, 21, 37, 40, 48]
    assert slot.tolist() == [3, 9, 9, 9, 2]
    assert seg.dtype == np.int32 and slot.dtype == np.int32


def test_tile_segments_cover_the_same_rows():
    rng = np.random.default_rng(4)
    counts = rng.integers(0, 70, size=200)
    seg = np.append(0, np.cumsum(counts))
    slot = rng.permutation(512)[:200]
    s2, t2 = prefill.tile_segments(seg, slot, rows=16)
    c2 = np.diff(s2)
    assert c2.min() >= 1 and c2.max() <= 16 and s2[0] == 0 and s2[-1] == seg[-1]
    # every row keeps its expert's slot
    want = np.repeat(slot, counts)
    got = np.repeat(t2, c2)
    assert np.array_equal(want, got)
    # a segment splits into ceil(rows / 16) pieces
    assert t2.size == int(np.sum((counts + 15) // 16))
    with pytest.raises(ValueError):
        prefill.tile_segments(np.array([0, 4]), np.array([1, 2]))
    # no segments, and segments that are all empty
    s0, t0 = prefill.tile_segments(np.array([0]), np.array([], np.int32))
    assert s0.tolist() == [0] and t0.size == 0
    s1, t1 = prefill.tile_segments(np.array([3, 3, 3]), np.array([1, 2]))
    assert s1.tolist() == [3] and t1.size == 0
