#!/usr/bin/env python3
"""Write golden LRU traces with the reference's own `mlx-qwen38/expert_io.c`.

The reference C file is compiled from its source tree by `oracle/Makefile` into
`oracle/_ref/libexpert_io_ref.so` (build container only).  This script drives it through
ctypes with seeded id streams and records every observable decision:

  per decode step : slot ids written to the slot-index buffer, the miss count, the 18 counters
  per prefetch    : the 18 counters and the LRU->MRU state afterwards
  periodically    : `c_layer_get_lru_state`
  at the end      : `c_get_decode_totals`

No I/O is performed: layers are initialised with fd = -1 and zero row bytes (the pattern the
reference's own `cpp/tests/test_kernels.cpp:508-515` uses), so every queued read has length 0.
The output is data only (tests/golden/lru_traces.json); the tests replay the recorded inputs
through the oracle and the HIP library and compare against the recorded outputs.

    make -C oracle && python tests/golden/make_lru_traces.py
"""
from __future__ import annotations

import ctypes
import json
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "moe-offload_amd"))
from moe_offload.synth import expert_id_stream  # noqa: E402

REF = ROOT / "oracle" / "_ref" / "libexpert_io_ref.so"
OUT = Path(__file__).resolve().parent / "lru_traces.json"


def load_ref():
    lib = ctypes.CDLL(str(REF))
    u64p, i32p, u32p = (ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_int32),
                        ctypes.POINTER(ctypes.c_uint32))
    lib.c_layer_init.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, u64p, u64p, u64p, ctypes.c_uint64]
    lib.c_layer_step_decode_ex.argtypes = [ctypes.c_int, u32p, ctypes.c_int, ctypes.c_int]
    lib.c_layer_step_decode_ex.restype = ctypes.c_int
    lib.c_layer_start_prefetch.argtypes = [ctypes.c_int, i32p, ctypes.c_int, ctypes.c_int]
    lib.c_layer_wait_prefetch.argtypes = [ctypes.c_int]
    lib.c_layer_load_sync.argtypes = [ctypes.c_int, i32p, i32p, ctypes.c_int, ctypes.c_int]
    lib.c_layer_get_lru_state.argtypes = [ctypes.c_int, i32p, i32p, ctypes.POINTER(ctypes.c_int)]
    lib.c_layer_set_lru_state.argtypes = [ctypes.c_int, i32p, i32p, ctypes.c_int,
                                          ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
    lib.c_layer_get_stats.argtypes = [ctypes.c_int, u64p]
    lib.c_get_decode_totals.argtypes = [ctypes.c_int, u64p]
    lib.c_layer_reset_cache.argtypes = [ctypes.c_int]
    lib.c_layer_reset_stats.argtypes = [ctypes.c_int]
    return lib


class RefLayer:
    def __init__(self, lib, layer, cap):
        self.lib, self.layer, self.cap = lib, layer, cap
        self.slot_buf = (ctypes.c_uint32 * 16)()
        z = (ctypes.c_uint64 * 9)()
        lib.c_layer_init(layer, -1, cap, z, z, z, ctypes.addressof(self.slot_buf))

    def step(self, eids):
        a = (ctypes.c_uint32 * len(eids))(*[int(e) for e in eids])
        n = self.lib.c_layer_step_decode_ex(self.layer, a, len(eids), 1)
        self.lib.c_layer_wait_prefetch(self.layer)
        return n, [int(v) for v in self.slot_buf[:len(eids)]]

    def prefetch(self, preds, cap):
        a = (ctypes.c_int32 * max(1, len(preds)))(*[int(p) for p in preds])
        self.lib.c_layer_start_prefetch(self.layer, a, len(preds), cap)
        self.lib.c_layer_wait_prefetch(self.layer)

    def load_sync(self, eids, slots):
        n = len(eids)
        self.lib.c_layer_load_sync(self.layer, (ctypes.c_int32 * max(n, 1))(*eids),
                                   (ctypes.c_int32 * max(n, 1))(*slots), n, 1)

    def state(self):
        e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int()
        self.lib.c_layer_get_lru_state(self.layer, e, s, ctypes.byref(c))
        return [list(e[:c.value]), list(s[:c.value])]

    def set_state(self, eids, slots, r, h, m):
        n = len(eids)
        self.lib.c_layer_set_lru_state(self.layer, (ctypes.c_int32 * max(n, 1))(*eids),
                                       (ctypes.c_int32 * max(n, 1))(*slots), n, r, h, m)

    def stats(self):
        o = (ctypes.c_uint64 * 18)()
        self.lib.c_layer_get_stats(self.layer, o)
        return [int(v) for v in o]


def predictions(rng, ids_next, m=12, recall=0.6, num_experts=512):
    """A noisy top-m guess of the next step's ids: some true ids in rank order plus random ones."""
    out = []
    for e in ids_next:
        if rng.random() < recall and int(e) not in out:
            out.append(int(e))
    while len(out) < m:
        e = int(rng.integers(num_experts))
        if e not in out:
            out.append(e)
    rng.shuffle(out)
    return out[:m]


def scenario_decode(lib, name, layer, cap, ids, prefetch=None, seed=0, state_every=16,
                    set_state_every=0):
    """One layer driven by an id stream; optional prefetch before each step; optional periodic
    state export/import (state re-imported in a rotated order to exercise set_lru_state)."""
    rng = np.random.default_rng(seed)
    L = RefLayer(lib, layer, cap)
    ops = []
    for t, step_ids in enumerate(ids):
        if prefetch is not None:
            nxt = ids[t]
            preds = predictions(rng, nxt, m=prefetch[0])
            L.prefetch(preds, prefetch[1])
            ops.append({"op": "prefetch", "preds": preds, "cap": prefetch[1], "stats": L.stats(),
                        "state": L.state()})
        n, slots = L.step([int(e) for e in step_ids])
        rec = {"op": "step", "ids": [int(e) for e in step_ids], "n_miss": n, "slots": slots,
               "stats": L.stats()}
        if state_every and (t + 1) % state_every == 0:
            rec["state"] = L.state()
        ops.append(rec)
        if set_state_every and (t + 1) % set_state_every == 0:
            e, s = L.state()
            rot = int(rng.integers(1, max(2, len(e))))
            e2, s2 = e[rot:] + e[:rot], s[rot:] + s[:rot]
            keep = int(rng.integers(len(e2) // 2, len(e2) + 1))
            e2, s2 = e2[:keep], s2[:keep]
            r, h, m = int(rng.integers(0, 100)), int(rng.integers(0, 50)), int(rng.integers(0, 20))
            L.set_state(e2, s2, r, h, m)
            ops.append({"op": "set_state", "eids": e2, "slots": s2, "add": [r, h, m],
                        "stats": L.stats(), "state": L.state()})
        if set_state_every and (t + 1) % (2 * set_state_every) == 0:
            le = sorted(rng.choice(512, size=int(rng.integers(1, 20)), replace=False).tolist())
            ls = [int(v) for v in rng.integers(0, cap, size=len(le))]
            L.load_sync(le, ls)
            ops.append({"op": "load_sync", "eids": le, "slots": ls, "stats": L.stats()})
    return {"name": name, "layer": layer, "capacity": cap, "ops": ops, "final_state": L.state()}


def scenario_stack(lib, name, n_layers, caps, steps, k, prefetch, seed):
    """Multi-layer decode in the loader's call order: for each token, prefetch(1) after layer 0,
    then step(l) followed by prefetch(l+1) for l = 1..n-2, and step(n-1)."""
    rng = np.random.default_rng(seed)
    layers = {l: RefLayer(lib, l, caps[l]) for l in range(1, n_layers)}
    for l in layers.values():
        lib.c_layer_reset_stats(l.layer)
    streams = {l: expert_id_stream(steps=steps, k=k, seed=seed + l) for l in layers}
    ops = []
    for t in range(steps):
        if prefetch:
            preds = predictions(rng, streams[1][t], m=prefetch[0])
            layers[1].prefetch(preds, prefetch[1])
            ops.append({"op": "prefetch", "layer": 1, "preds": preds, "cap": prefetch[1]})
        for l in range(1, n_layers):
            ids = [int(e) for e in streams[l][t]]
            n, slots = layers[l].step(ids)
            ops.append({"op": "step", "layer": l, "ids": ids, "n_miss": n, "slots": slots})
            if prefetch and l + 1 < n_layers:
                preds = predictions(rng, streams[l + 1][t], m=prefetch[0])
                layers[l + 1].prefetch(preds, prefetch[1])
                ops.append({"op": "prefetch", "layer": l + 1, "preds": preds, "cap": prefetch[1]})
    tot = (ctypes.c_uint64 * 6)()
    lib.c_get_decode_totals(n_layers, tot)
    return {"name": name, "n_layers": n_layers, "capacities": {str(l): caps[l] for l in layers},
            "ops": ops, "totals": [int(v) for v in tot],
            "layer_stats": {str(l): layers[l].stats() for l in layers}}


def main() -> int:
    if not REF.exists():
        print(f"build the reference first: make -C oracle ({REF} missing)", file=sys.stderr)
        return 1
    lib = load_ref()
    ids_c2 = expert_id_stream(steps=128, k=10, seed=2)
    rng = np.random.default_rng(7)
    uniform = [rng.choice(512, size=10, replace=False).tolist() for _ in range(96)]
    small = [rng.choice(40, size=16, replace=False).tolist() for _ in range(64)]
    out = {
        "ref_expert_bytes": 1_536_000,
        "scenarios": [
            scenario_decode(lib, "config2_cap102_noprefetch", 1, 102, ids_c2.tolist()),
            scenario_decode(lib, "config2_cap102_prefetch12x3", 2, 102, ids_c2.tolist(),
                            prefetch=(12, 3), seed=11),
            scenario_decode(lib, "uniform_cap16_prefetch12x3_state", 3, 16, uniform,
                            prefetch=(12, 3), seed=12, state_every=8, set_state_every=10),
            scenario_decode(lib, "uniform_cap24_prefetch32x0", 4, 24, uniform[:48],
                            prefetch=(32, 0), seed=13, state_every=4),
            scenario_decode(lib, "small_pool_k16_cap16_fallback", 5, 16, small,
                            prefetch=(20, 40), seed=14, state_every=4),
            scenario_decode(lib, "cap512_all_fit", 6, 512, uniform[:64], state_every=32),
        ],
        "stacks": [
            scenario_stack(lib, "stack8_cap20pct_prefetch", 8, {l: 102 for l in range(1, 8)},
                           steps=24, k=10, prefetch=(12, 3), seed=21),
            scenario_stack(lib, "stack6_cap16_noprefetch", 6, {l: 16 + l for l in range(1, 6)},
                           steps=24, k=10, prefetch=None, seed=31),
        ],
    }
    OUT.write_text(json.dumps(out, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
