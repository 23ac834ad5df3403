"""The oracle's restatement of the scheduler variant (oracle/lru.c: o_layer_decode_step_sched,
split lists, per-token accounting) against golden traces written by the reference's own
`mlx-qwen38/cpp/third_party/expert_io.c` (tests/golden/make_sched_traces.py), plus controls
showing the traces tell the scheduler's rules apart from the published ones."""
import pytest

from oracle import lru
from sched_replay import TokenMixin, load, replay

EXPERT_BYTES = 1_536_000


class OracleImpl(TokenMixin):
    def __init__(self, published=False):
        super().__init__()
        self.published = published       # control: the published step/prefetch instead
        self.layers = {}

    def init(self, l, cap):
        self.layers[l] = lru.CLru(l, cap, EXPERT_BYTES)
        lru.set_staged_bytes(l, 0)

    def reset_stats(self, l):
        self.layers[l].reset_stats()

    def reset_cache(self, l):
        self.layers[l].reset_cache()

    def accounting(self, on):
        lru.set_io_accounting(on)

    def begin(self):
        lru.begin_decode_token()

    def end(self):
        return lru.end_decode_token()

    def sched(self, l, ids, preds, nxt, cap, flags):
        if self.published:
            slots, n = [], 0
            if l > 0 and ids:
                slots, pairs = self.layers[l].step(ids)
                n = len(pairs)
            if not (flags & 2) and nxt > 0 and preds:      # published: cap 0 means 32
                self.layers[nxt].prefetch(preds, cap)
            return n, slots
        n, slots, _, _ = lru.decode_step_sched(l, ids, preds, nxt, cap, flags)
        return n, slots

    def step(self, l, ids):
        slots, pairs = self.layers[l].step(ids)
        return len(pairs), slots

    def prefetch(self, l, preds, cap):
        self.layers[l].prefetch(preds, cap)

    def stats(self, l):
        return [int(v) for v in self.layers[l].stats()]

    def state(self, l):
        e, s = self.layers[l].get_state()
        return [list(e), list(s)]

    def set_state(self, l, e, s, add):
        self.layers[l].set_state(e, s, *add)

    def split(self, l):
        h, m, inv = lru.split_inds(l)
        return [h, m, inv]

    def totals(self, n_layers):
        return [int(v) for v in lru.decode_totals(n_layers)]


GOLD = load()


@pytest.mark.parametrize("sc", GOLD["scenarios"], ids=[s["name"] for s in GOLD["scenarios"]])
def test_oracle_sched_matches_reference_traces(sc):
    assert replay(sc, OracleImpl()) > 50


def test_traces_distinguish_scheduler_from_published_rules():
    """The published step (ids-only protection) and prefetch (repeats taken twice, cap 0 -> 32)
    replayed against the same traces must fail: the traces pin what makes the variant differ."""
    failed = []
    for sc in GOLD["scenarios"]:
        try:
            replay(sc, OracleImpl(published=True), check_split=False)
        except AssertionError:
            failed.append(sc["name"])
    # every scenario exercises at least one of the differences (repeated predictions in all,
    # prefetch cap 0 in one)
    assert failed == [s["name"] for s in GOLD["scenarios"]], failed


def test_split_lists_invariants():
    """Split lists of every recorded split: hits ++ misses is a permutation of the step's slots,
    inv maps id i to the position of its slot, and hits are exactly the ids the step did not
    miss (the ids resident before the step)."""
    checked = 0
    for sc in GOLD["scenarios"]:
        for o in sc["ops"]:
            if o["op"] != "sched" or "split" not in o or not (o["flags"] & 4):
                continue
            k, n = len(o["ids"]), o["n_miss"]
            if not 0 < n < k:
                continue
            hit, miss, inv = o["split"]
            assert len(hit) == k - n and len(miss) == n and len(inv) == k
            both = hit + miss
            assert sorted(inv) == list(range(k))
            assert [both[inv[i]] for i in range(k)] == o["slots"]
            checked += 1
    assert checked > 50


def test_scheduler_protection_equals_published_choice_with_distinct_predictions():
    """With distinct predictions and a prefetch cap > 0 the scheduler variant makes exactly the
    published decisions, also in pools so small that the step's ids plus the prefetched experts
    cover every slot (where the reference's own last resort is undefined and the restatement
    spares the step's ids): the prefetched experts are the newest entries, so protecting them
    never changes which unprotected entry is oldest.  Every slot id stays valid and names the
    slot that holds its expert."""
    import numpy as np
    rng = np.random.default_rng(5)
    fallback_steps = 0
    for trial in range(60):
        cap = int(rng.choice([10, 11, 12, 14, 16, 24]))
        a, b = lru.CLru(40, cap), lru.CLru(41, cap)
        lru.set_io_accounting(False)
        for t in range(40):
            preds = [int(v) for v in rng.choice(48, size=12, replace=False)]
            pcap = int(rng.choice([1, 3, 8, 31]))
            lru.decode_step_sched(0, None, preds, 40, pcap, 0)
            b.prefetch(preds, pcap)
            ids = [int(v) for v in rng.choice(48, size=10, replace=False)]
            resident = set(a.get_state()[0])
            fetched = len(set(preds) - resident)
            n, slots, _, _ = lru.decode_step_sched(40, ids, None, -1, 0, 2)
            slots_b, pairs = b.step(ids)
            assert (n, slots) == (len(pairs), slots_b), (trial, t)
            assert a.get_state() == b.get_state() and a.stats() == b.stats(), (trial, t)
            held = dict(zip(*[list(v) for v in a.get_state()]))
            assert all(0 <= s < cap for s in slots) and [held[e] for e in ids] == slots
            fallback_steps += (10 + min(fetched, pcap) > cap)
    assert fallback_steps > 20
