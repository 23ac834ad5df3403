"""Replay of the scheduler golden traces (tests/golden/lru_sched_traces.json) through an
implementation of the expert-cache ABI: the oracle's C restatement or the product library.

An implementation provides: init(layer, cap), reset_stats(l), reset_cache(l), accounting(on),
begin(), end() -> out10, sched(l, ids, preds, next, cap, flags) -> (n_miss, slots), step(l, ids)
-> (n_miss, slots), prefetch(l, preds, cap), stats(l), state(l), set_state(l, e, s, add),
split(l) -> (hit, miss, inv), totals(n_layers).
"""
from __future__ import annotations

import json
from pathlib import Path

GOLDEN = Path(__file__).resolve().parent / "golden" / "lru_sched_traces.json"
SPLIT = 4


def load():
    return json.loads(GOLDEN.read_text())


def replay(sc, impl, check_split=True, check_tokens=True):
    """Replays one scenario; returns the number of records compared.  check_split /
    check_tokens off: the split lists / per-token counters are not compared (implementations
    without them)."""
    for l, cap in sc["capacities"].items():
        impl.init(int(l), cap)
        impl.reset_stats(int(l))
    acct = any(o["op"] == "token" and any(o["out10"]) for o in sc["ops"])
    impl.accounting(acct)
    seen_split = set()
    n = 0
    name = sc["name"]
    for i, o in enumerate(sc["ops"]):
        where = f"{name} op {i} ({o['op']})"
        op = o["op"]
        if op == "reset_cache":
            impl.reset_cache(o["layer"])
            assert impl.state(o["layer"]) == o["state"], where
        elif op == "sched":
            if o["layer"] == 0:                      # prefetch-only call after the resident layer
                impl.begin_if_needed()
            n_miss, slots = impl.sched(o["layer"], o["ids"], o["preds"], o["next"], o["cap"], o["flags"])
            assert n_miss == o["n_miss"], where
            if "slots" in o:
                assert slots == o["slots"], where
                assert impl.stats(o["layer"]) == o["stats"], where
                k = len(o["ids"])
                if (o["flags"] & SPLIT) and 0 < n_miss < k:
                    seen_split.add(o["layer"])
                if check_split and o["layer"] in seen_split:
                    assert impl.split(o["layer"]) == o["split"], where
            if "next_stats" in o:
                assert impl.stats(o["next"]) == o["next_stats"], where
        elif op == "step":
            n_miss, slots = impl.step(o["layer"], o["ids"])
            assert (n_miss, slots) == (o["n_miss"], o["slots"]), where
            assert impl.stats(o["layer"]) == o["stats"], where
        elif op == "prefetch":
            impl.prefetch(o["layer"], o["preds"], o["cap"])
            assert impl.stats(o["layer"]) == o["next_stats"], where
        elif op == "token":
            if check_tokens:
                assert impl.end() == o["out10"], where
            impl.token_done()
        elif op == "set_state":
            impl.set_state(o["layer"], o["eids"], o["slots"], o["add"])
            assert impl.state(o["layer"]) == o["state"], where
        else:
            raise AssertionError(f"unknown op {op}")
        n += 1
    impl.accounting(False)
    assert impl.totals(sc["n_layers"]) == sc["totals"], name
    for l, st in sc["final_states"].items():
        assert impl.state(int(l)) == st, f"{name} final state of layer {l}"
    for l, st in sc["layer_stats"].items():
        assert impl.stats(int(l)) == st, f"{name} final counters of layer {l}"
    return n


class TokenMixin:
    """Token bracketing as the trace generator did: c_begin_decode_token before the
    prefetch-only call that opens each token, c_end_decode_token at the token record."""

    def __init__(self):
        self._open = False

    def begin_if_needed(self):
        if not self._open:
            self.begin()
            self._open = True

    def token_done(self):
        self._open = False
