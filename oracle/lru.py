"""Bindings and a second restatement of the slot LRU -- test infrastructure only.

`CLru`  : ctypes wrapper of `_build/liblru_oracle.so` (lru.c, the linked-list restatement).
`PyLru` : independent pure-Python restatement in the OrderedDict form that the reference's
          Python loader keeps alongside the C table (`mlx-qwen38/loader.py:408-410,482-490`),
          extended with the decode step / prefetch / counters of `mlx-qwen38/expert_io.c:527-708`.
Both expose the same methods so tests can run them side by side against the golden traces
written by the reference's own expert_io.c (tests/golden/make_lru_traces.py).
"""
from __future__ import annotations

import ctypes
from collections import OrderedDict
from pathlib import Path

NUM_EXPERTS = 512
NUM_TENSORS = 9
REF_EXPERT_BYTES = 1_536_000  # the reference's compile-time EXPERT_BYTES (expert_io.c:21)

_HERE = Path(__file__).resolve().parent
LIB_PATH = _HERE / "_build" / "liblru_oracle.so"
REF_LIB_PATH = _HERE / "_ref" / "libexpert_io_ref.so"


def build() -> None:
    """Compile lru.c (and the reference expert_io.c when its source tree is present)."""
    import subprocess
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    u32p, i32p, u64p = (ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int32),
                        ctypes.POINTER(ctypes.c_uint64))
    lib.o_layer_init.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint64]
    lib.o_layer_reset_cache.argtypes = [ctypes.c_int]
    lib.o_layer_reset_stats.argtypes = [ctypes.c_int]
    lib.o_layer_step_decode.argtypes = [ctypes.c_int, u32p, ctypes.c_int, u32p, i32p, i32p]
    lib.o_layer_step_decode.restype = ctypes.c_int
    lib.o_layer_start_prefetch.argtypes = [ctypes.c_int, i32p, ctypes.c_int, ctypes.c_int, i32p, i32p]
    lib.o_layer_start_prefetch.restype = ctypes.c_int
    lib.o_layer_load_sync.argtypes = [ctypes.c_int, i32p, i32p, ctypes.c_int, ctypes.c_int]
    lib.o_layer_get_lru_state.argtypes = [ctypes.c_int, i32p, i32p, ctypes.POINTER(ctypes.c_int)]
    lib.o_layer_set_lru_state.argtypes = [ctypes.c_int, i32p, i32p, ctypes.c_int,
                                          ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
    lib.o_layer_get_stats.argtypes = [ctypes.c_int, u64p]
    lib.o_get_decode_totals.argtypes = [ctypes.c_int, u64p]
    lib.o_layer_decode_step_sched.argtypes = [ctypes.c_int, i32p, ctypes.c_int, i32p, ctypes.c_int, ctypes.c_int,
                                              ctypes.c_int, ctypes.c_int, u32p, i32p, i32p, i32p, i32p,
                                              ctypes.POINTER(ctypes.c_int)]
    lib.o_layer_decode_step_sched.restype = ctypes.c_int
    lib.o_layer_get_split_inds.argtypes = [ctypes.c_int, u32p, u32p, i32p, i32p]
    lib.o_set_io_accounting.argtypes = [ctypes.c_int]
    lib.o_begin_decode_token.argtypes = []
    lib.o_end_decode_token.argtypes = [u64p]
    lib.o_layer_set_staged_bytes.argtypes = [ctypes.c_int, ctypes.c_uint64]
    return lib


_LIB = None


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is None:
        _LIB = _load()
    return _LIB


class CLru:
    """One layer of the C restatement."""

    def __init__(self, layer: int, capacity: int, expert_bytes: int = REF_EXPERT_BYTES):
        self.layer, self.capacity = layer, capacity
        lib().o_layer_init(layer, capacity, expert_bytes)

    def reset_cache(self):
        lib().o_layer_reset_cache(self.layer)

    def reset_stats(self):
        lib().o_layer_reset_stats(self.layer)

    def step(self, eids):
        k = len(eids)
        a = (ctypes.c_uint32 * k)(*eids)
        out = (ctypes.c_uint32 * k)()
        me, ms = (ctypes.c_int32 * 16)(), (ctypes.c_int32 * 16)()
        n = lib().o_layer_step_decode(self.layer, a, k, out, me, ms)
        return list(out), list(zip(me[:n], ms[:n]))

    def prefetch(self, preds, max_fetch):
        n = len(preds)
        a = (ctypes.c_int32 * max(n, 1))(*preds)
        fe, fs = (ctypes.c_int32 * 32)(), (ctypes.c_int32 * 32)()
        m = lib().o_layer_start_prefetch(self.layer, a, n, max_fetch, fe, fs)
        return list(zip(fe[:m], fs[:m]))

    def load_sync(self, eids, slots, is_prefill=1):
        n = len(eids)
        lib().o_layer_load_sync(self.layer, (ctypes.c_int32 * max(n, 1))(*eids),
                                (ctypes.c_int32 * max(n, 1))(*slots), n, is_prefill)

    def get_state(self):
        e, s, c = (ctypes.c_int32 * NUM_EXPERTS)(), (ctypes.c_int32 * NUM_EXPERTS)(), ctypes.c_int(0)
        lib().o_layer_get_lru_state(self.layer, e, s, ctypes.byref(c))
        return list(e[:c.value]), list(s[:c.value])

    def set_state(self, eids, slots, add_req=0, add_hits=0, add_miss=0):
        n = len(eids)
        lib().o_layer_set_lru_state(self.layer, (ctypes.c_int32 * max(n, 1))(*eids),
                                    (ctypes.c_int32 * max(n, 1))(*slots), n, add_req, add_hits, add_miss)

    def stats(self):
        out = (ctypes.c_uint64 * 18)()
        lib().o_layer_get_stats(self.layer, out)
        return list(out)


def decode_totals(num_layers: int):
    out = (ctypes.c_uint64 * 6)()
    lib().o_get_decode_totals(num_layers, out)
    return list(out)


SCHED_SYNC_DEMAND, SCHED_NO_PREFETCH, SCHED_SPLIT = 1, 2, 4


def decode_step_sched(layer, eids, pred, next_layer, prefetch_cap, flags):
    """Scheduler entry point of the C restatement.

    Returns (n_miss, slots of the step's ids, demand (eid, slot) pairs, prefetch (eid, slot) pairs).
    `eids` / `pred` may be None (skipped step / no prefetch)."""
    k = len(eids) if eids is not None else 0
    n_pred = len(pred) if pred is not None else 0
    ea = (ctypes.c_int32 * max(k, 1))(*(eids or []))
    pa = (ctypes.c_int32 * max(n_pred, 1))(*(pred or []))
    out = (ctypes.c_uint32 * 16)()
    me, ms, fe, fs = ((ctypes.c_int32 * 32)() for _ in range(4))
    nf = ctypes.c_int(0)
    n = lib().o_layer_decode_step_sched(layer, ea if eids is not None else None, k,
                                        pa if pred is not None else None, n_pred, next_layer, prefetch_cap,
                                        flags, out, me, ms, fe, fs, ctypes.byref(nf))
    kk = min(k, 16)
    return n, list(out[:kk]), list(zip(me[:n], ms[:n])), list(zip(fe[:nf.value], fs[:nf.value]))


def layer_stats(layer):
    """The 18 counters of a layer of the C restatement."""
    out = (ctypes.c_uint64 * 18)()
    lib().o_layer_get_stats(layer, out)
    return [int(v) for v in out]


def split_inds(layer):
    """(hit slots, miss slots, inverse order) stored by the last split of `layer`."""
    h, m = (ctypes.c_uint32 * 16)(), (ctypes.c_uint32 * 16)()
    inv, c = (ctypes.c_int32 * 16)(), (ctypes.c_int32 * 3)()
    lib().o_layer_get_split_inds(layer, h, m, inv, c)
    return list(h[:c[0]]), list(m[:c[1]]), list(inv[:c[2]])


def set_io_accounting(on: bool):
    lib().o_set_io_accounting(1 if on else 0)


def begin_decode_token():
    lib().o_begin_decode_token()


def end_decode_token():
    out = (ctypes.c_uint64 * 10)()
    lib().o_end_decode_token(out)
    return list(out)


def set_staged_bytes(layer, nbytes):
    lib().o_layer_set_staged_bytes(layer, nbytes)


class PyLru:
    """Pure-Python restatement (OrderedDict: first = LRU, last = MRU)."""

    def __init__(self, layer: int, capacity: int, expert_bytes: int = REF_EXPERT_BYTES):
        self.layer, self.capacity, self.expert_bytes = layer, capacity, expert_bytes
        self.st = [0] * 18
        self.reset_cache()

    def reset_cache(self):
        self.lru: OrderedDict[int, int] = OrderedDict()
        self.free = list(range(self.capacity - 1, -1, -1))
        self.snap = None  # (resident set, pred set, fetched set)

    def reset_stats(self):
        self.st = [0] * 18

    def _alloc(self, protected: set[int]) -> int:
        if self.free:
            return self.free.pop()
        for e in self.lru:
            if e not in protected:
                return self.lru.pop(e)
        return self.lru.popitem(last=False)[1]

    def _insert(self, e: int, s: int):
        if e in self.lru:
            self.lru.move_to_end(e)
        else:
            self.lru[e] = s

    def _runs(self, eids):
        if not eids:
            return
        v = sorted(eids)
        runs = 1 + sum(1 for a, b in zip(v, v[1:]) if b != a + 1)
        self.st[16] += len(v) * NUM_TENSORS
        self.st[17] += runs * NUM_TENSORS

    def step(self, eids):
        want = set(eids)
        self.st[0] += len(eids)
        if self.snap is not None:
            res, pred, fet = self.snap
            miss_before = want - res
            self.st[10] += len(want & pred)
            self.st[11] += len(want)
            self.st[12] += len(pred)
            self.st[13] += len(miss_before & fet)
            self.st[14] += len(miss_before)
            self.st[15] += len(fet)
        misses = []
        for e in eids:
            if e in self.lru:
                if self.snap is None or e in self.snap[0]:
                    self.st[1] += 1
                else:
                    self.st[2] += 1
            else:
                self.st[3] += 1
                misses.append(e)
        self.snap = None
        pairs = []
        for e in misses:
            s = self._alloc(want)
            self._insert(e, s)
            pairs.append((e, s))
        self.st[4] += len(misses) * self.expert_bytes
        out = []
        for e in eids:
            self.lru.move_to_end(e)
            out.append(self.lru[e])
        self._runs(misses)
        return out, pairs

    def prefetch(self, preds, max_fetch):
        cap = max_fetch if 0 < max_fetch < 32 else 32
        res = set(self.lru)
        pred, fet, pick = set(), set(), []
        for e in preds:
            if e < 0 or e >= NUM_EXPERTS:
                continue
            pred.add(e)
            if e not in self.lru and len(pick) < cap:
                pick.append(e)
                fet.add(e)
        self.snap = (res, pred, fet)
        pairs = []
        for e in reversed(pick):
            s = self._alloc(pred)
            self._insert(e, s)
            pairs.append((e, s))
        self.st[5] += len(pick) * self.expert_bytes
        self._runs([e for e, _ in pairs])
        return pairs

    def load_sync(self, eids, slots, is_prefill=1):
        if not eids:
            return
        if is_prefill:
            self.st[9] += len(eids) * self.expert_bytes
        self._runs(list(eids))

    def get_state(self):
        return list(self.lru.keys()), list(self.lru.values())

    def set_state(self, eids, slots, add_req=0, add_hits=0, add_miss=0):
        self.st[6] += add_req
        self.st[7] += add_hits
        self.st[8] += add_miss
        self.lru = OrderedDict()
        self.snap = None
        used = set()
        for e, s in zip(eids, slots):
            used.add(s)
            self._insert(e, s)
        self.free = [s for s in range(self.capacity - 1, -1, -1) if s not in used]

    def stats(self):
        return list(self.st)
