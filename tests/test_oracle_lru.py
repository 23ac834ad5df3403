"""The LRU oracle (C and Python restatements) against golden traces from the reference C."""
import numpy as np
import pytest

from oracle import lru as olru


def _replay_layer(impl_cls, scen, layer_offset=0):
    L = impl_cls(scen["layer"] + layer_offset, scen["capacity"])
    L.reset_stats()
    for op in scen["ops"]:
        if op["op"] == "prefetch":
            L.prefetch(op["preds"], op["cap"])
        elif op["op"] == "step":
            slots, misses = L.step(op["ids"])
            assert slots == op["slots"], f"{scen['name']}: slot ids differ"
            assert len(misses) == op["n_miss"]
        elif op["op"] == "set_state":
            L.set_state(op["eids"], op["slots"], *op["add"])
        elif op["op"] == "load_sync":
            L.load_sync(op["eids"], op["slots"])
        assert L.stats() == op["stats"], f"{scen['name']}: counters differ after {op['op']}"
        if "state" in op:
            assert [list(v) for v in L.get_state()] == op["state"]
    assert [list(v) for v in L.get_state()] == scen["final_state"]


@pytest.mark.parametrize("impl", [olru.CLru, olru.PyLru], ids=["c", "py"])
def test_layer_traces(lru_traces, impl):
    for scen in lru_traces["scenarios"]:
        _replay_layer(impl, scen)


@pytest.mark.parametrize("impl", [olru.CLru, olru.PyLru], ids=["c", "py"])
def test_stack_traces(lru_traces, impl):
    for stk in lru_traces["stacks"]:
        layers = {int(l): impl(int(l), c) for l, c in stk["capacities"].items()}
        for L in layers.values():
            L.reset_stats()
        for op in stk["ops"]:
            L = layers[op["layer"]]
            if op["op"] == "prefetch":
                L.prefetch(op["preds"], op["cap"])
            else:
                slots, misses = L.step(op["ids"])
                assert slots == op["slots"] and len(misses) == op["n_miss"]
        for l, st in stk["layer_stats"].items():
            assert layers[int(l)].stats() == st
        tot = [0] * 6
        for L in layers.values():
            s = L.stats()
            for i, j in enumerate([1, 2, 3, 0, 4, 5]):
                tot[i] += s[j]
        assert tot == stk["totals"]
        if impl is olru.CLru:
            assert olru.decode_totals(stk["n_layers"]) == stk["totals"]
            for l in layers:               # clear so later tests see clean layers
                olru.lib().o_layer_reset_stats(l)


def test_negative_control_mru_order_matters(lru_traces):
    """A planted mistake (refresh ids to MRU in reverse order) must break the golden trace."""
    class Reversed(olru.PyLru):
        def step(self, eids):
            out, pairs = super().step(eids)
            for e in reversed(eids):
                self.lru.move_to_end(e)
            return out, pairs
    scen = lru_traces["scenarios"][0]
    with pytest.raises(AssertionError):
        _replay_layer(Reversed, scen)


def test_invariants_random_streams():
    """Bijection eid<->slot, resident <= capacity, last id of a step is MRU, free slots are
    handed out ascending from empty, prefetched ids become resident."""
    rng = np.random.default_rng(3)
    for cap in (16, 17, 40, 102):
        L = olru.PyLru(9, cap)
        C = olru.CLru(9, cap)
        handed = []                      # slots allocated while the pool is filling
        for t in range(200):
            if rng.random() < 0.5:
                preds = rng.choice(512, size=12, replace=False).tolist()
                a, b = L.prefetch(preds, 3), C.prefetch(preds, 3)
                assert a == b
                for e, _ in a:
                    assert e in L.lru
                handed += [s for _, s in a]
            ids = rng.choice(64 if t % 2 else 512, size=10, replace=False).tolist()
            (s1, m1), (s2, m2) = L.step(ids), C.step(ids)
            assert s1 == s2 and m1 == m2
            handed += [s for _, s in m1]
            e, s = L.get_state()
            assert len(e) <= cap and len(set(e)) == len(e) and len(set(s)) == len(s)
            assert e[-1] == ids[-1]
            assert all(L.lru[x] == y for x, y in zip(e, s))
        assert L.stats() == C.stats()
        assert handed[:cap] == list(range(cap))


def test_bruteforce_tiny_capacity():
    """Exhaustive small case: capacity 2, ids from 4 experts, every 3-step sequence of single-id
    steps; the C restatement agrees with a from-first-principles list model."""
    import itertools
    for seq in itertools.product(range(4), repeat=3):
        C = olru.CLru(10, 2)
        order = []                       # LRU..MRU list of eids (the textbook LRU)
        for e in seq:
            slots, misses = C.step([e])
            if e in order:
                order.remove(e)
                assert misses == []
            else:
                assert len(misses) == 1
                if len(order) == 2:
                    order.pop(0)
            order.append(e)
            assert C.get_state()[0] == order


def test_demand_victims_avoid_in_flight_prefetch_slots():
    """The ordering rule of the device-driven decode (stack.DecodeStack.demand_overlaps_prefetch):
    with capacity >= 2 k + prefetch cap, no demand miss of a step lands in a slot the preceding
    prefetch of that layer fetched into, so demand copies may be queued while prefetch copies
    are still landing.  Checked on the C restatement over random traces at the boundary
    capacity, and shown necessary by finding a collision below it."""
    import numpy as np
    rng = np.random.default_rng(17)
    k, pcap = 10, 3

    def collisions(cap, steps=400, universe=60):
        L = olru.CLru(45, cap)
        hits = 0
        for _ in range(steps):
            preds = [int(v) for v in rng.choice(universe, size=12, replace=False)]
            fetched = {s for _, s in L.prefetch(preds, pcap)}
            ids = [int(v) for v in rng.choice(universe, size=k, replace=False)]
            _, misses = L.step(ids)
            hits += sum(1 for _, s in misses if s in fetched)
        return hits

    for cap in (2 * k + pcap, 2 * k + pcap + 7, 102):
        assert collisions(cap) == 0, cap
    assert collisions(k + 1) > 0
