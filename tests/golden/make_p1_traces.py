"""Write tests/golden/p1_traces.json.gz: random call sequences of the P1 I/O scheduler and what the
reference's own io_sched.cpp (mlx-qwen38/cpp/src, compiled from source with oracle/p1_ref_shim.cpp
into oracle/_ref/libp1_ref.so by `make -C oracle ref`) returns for them, without reader threads.

Each trace runs in a child process with a time limit: without reader threads the reference sleeps
forever where a wait has nothing left to run (e.g. waiting for a prefetch that was started, then
dropped), and such traces are kept only as `deadlock` records (the oracle must raise at the same
call).  Every kept trace is also replayed through the oracle (oracle/p1.py), which must agree.

Usage: python tests/golden/make_p1_traces.py [n_traces]
"""
from __future__ import annotations

import gzip
import json
import multiprocessing as mp
import os
import random
import sys
import tempfile
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

from p1_replay import OracleAdapter, RefAdapter, apply_op, make_file, replay  # noqa: E402

N_EXP = 32
ROW_BYTES = [100_352, 128, 128, 100_352, 128, 128, 100_352, 128, 128]   # weights > 100000 B go first
LAYERS = (1, 2)


def gen_trace(seed: int) -> dict:
    r = random.Random(seed)
    cap = r.choice([4, 5, 6, 8, 12])
    k = r.randint(2, min(4, cap - 1))
    ops = []
    for l in LAYERS:
        ops.append({"op": "init", "l": l, "cap": cap})
        if r.random() < 0.7:                       # the reference tests start from a loaded pool
            n = r.randint(1, cap)
            e = r.sample(range(N_EXP), n)
            s = list(range(n))
            ops.append({"op": "load_sync", "l": l, "eids": e, "slots": s, "prefill": r.random() < 0.5})
            ops.append({"op": "set_lru", "l": l, "eids": e, "slots": s, "add": [n, 0, n]})
    n_steps = r.randint(15, 40)
    held = []                                       # explicit pins, released a few calls later
    for _ in range(n_steps):
        for l in LAYERS:
            if held and r.random() < 0.5:
                ops.append(held.pop(0))
            if r.random() < 0.8:
                ops.append({"op": "unpin_layer", "l": l})
            if r.random() < 0.15:
                ops.append({"op": "invalidate", "l": l, "rate": r.choice([0.3, 0.5, 1.0])})
            eids = r.sample(range(N_EXP), k)
            ops.append({"op": "step", "l": l, "eids": eids, "check": r.random() < 0.3})
            if r.random() < 0.85:
                ops.append({"op": "wait_urgent", "l": l})
            nl = LAYERS[(LAYERS.index(l) + 1) % len(LAYERS)]
            if r.random() < 0.8:
                m = r.randint(1, 8)
                ops.append({"op": "prefetch", "l": nl, "preds": r.sample(range(N_EXP), m),
                            "maxf": r.choice([1, 2, 3, 3, 5])})
            x = r.random()
            if x < 0.05:
                ops.append({"op": "wait_all", "l": nl})
            elif x < 0.08:
                sl = r.sample(range(cap), 1)
                ops.append({"op": "pin", "l": l, "slots": sl})
                held.append({"op": "unpin", "l": l, "slots": sl, "check": True})
            elif x < 0.09:
                ops.append({"op": "unpin", "l": l, "slots": r.sample(range(cap), 2)})
            elif x < 0.13:
                ops.append({"op": "get_lru", "l": l, "check": True})
            elif x < 0.15:
                ops.append({"op": "reset_stats", "l": l})
            elif x < 0.16:
                ops.append({"op": "reset_cache", "l": l})
            elif x < 0.19:
                ops.append({"op": "resize", "l": l, "cap": r.choice([3, 4, 6, 8, 12, 14])})
    ops[-1]["check"] = True
    return {"seed": seed, "cap": cap, "k": k, "rng_seed": seed * 7919 + 1, "ops": ops}


def bind_resizes(trace: dict) -> dict:
    """Give every `resize` its arguments as the reference runner computes them
    (cpp/src/loader.cpp:1053-1180, test_io_sched.cpp:318-352): unpin the layer, join its reads, read
    its LRU order, keep the most recent min(count, new capacity) experts in slots 0.. and copy their
    rows.  The state comes from the oracle run up to that call (it raises Deadlock where the
    reference would hang; the caller drops the trace then)."""
    orc = OracleAdapter(N_EXP, ROW_BYTES)
    orc.seed_rng(trace["rng_seed"])
    caps, out = {}, []
    for op in trace["ops"]:
        if op["op"] == "resize":
            l = op["l"]
            for q in ({"op": "unpin_layer", "l": l}, {"op": "wait_all", "l": l}, {"op": "get_lru", "l": l}):
                apply_op(orc, q, caps)
                out.append(q)
            eids, slots = orc.get_lru(l)
            new_cap = max(op["cap"], trace["k"] + 1)
            keep = min(len(eids), new_cap)
            op = {"op": "resize", "l": l, "cap": new_cap, "eids": eids[len(eids) - keep:],
                  "slots": list(range(keep)), "old_slots": slots[len(slots) - keep:], "check": True}
        apply_op(orc, op, caps)
        out.append(op)
    return dict(trace, ops=out)


def _run_full(trace, path, offs, q):
    fd = os.open(path, os.O_RDONLY)
    ad = RefAdapter(fd, offs, N_EXP, ROW_BYTES, threads=0)
    q.put(replay(ad, trace))


def run_ref(trace, path, offs, timeout=10.0):
    """The reference's records, or None when a call never returns (a child process, killed)."""
    ctx = mp.get_context("fork")
    q = ctx.Queue()
    p = ctx.Process(target=_run_full, args=(trace, path, offs, q))
    p.start()
    try:
        recs = q.get(timeout=timeout)
    except Exception:
        recs = None
    p.join(1.0)
    if p.is_alive():
        p.kill()
        p.join()
    return recs


def main():
    n = int(sys.argv[1]) if len(sys.argv) > 1 else 40
    from oracle import p1 as op1
    tmp = tempfile.mkdtemp(prefix="p1_traces_")
    path = os.path.join(tmp, "experts.bin")
    offs = make_file(path, LAYERS, N_EXP, ROW_BYTES)
    kept, hung = [], 0
    seed = 0
    while len(kept) < n:
        seed += 1
        try:
            tr = bind_resizes(gen_trace(seed))
        except op1.Deadlock:
            hung += 1
            continue
        recs = run_ref(tr, path, offs)
        orc = OracleAdapter(N_EXP, ROW_BYTES)
        if recs is None:
            hung += 1
            try:
                replay(orc, tr)
                raise SystemExit(f"seed {seed}: the reference hangs, the oracle does not")
            except op1.Deadlock:
                pass
            continue
        got = replay(orc, tr)
        for i, (a, b) in enumerate(zip(recs, got)):
            if a != b:
                raise SystemExit(f"seed {seed} call {i} {tr['ops'][i]}: reference {a} oracle {b}")
        tr["expect"] = recs
        kept.append(tr)
    out = {"n_exp": N_EXP, "row_bytes": ROW_BYTES, "layers": list(LAYERS), "traces": kept,
           "hung_traces_skipped": hung}
    with gzip.open(HERE / "p1_traces.json.gz", "wt") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"{len(kept)} traces, {sum(len(t['ops']) for t in kept)} calls, {hung} hanging traces skipped")


if __name__ == "__main__":
    main()
