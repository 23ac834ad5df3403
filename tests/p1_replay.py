"""Replay of P1 I/O scheduler traces (test infrastructure).

A trace is a list of scheduler calls (`layer_init`, `step`, `start_prefetch`, waits, pins,
`force_invalidate`, `load_sync`, LRU state get/set, `resize`, resets).  `replay(adapter, trace)`
runs it on one implementation and records, after every call, its result, after every step and
forced invalidation the layer's 15 deterministic counters (io_wait_ns left out), and where the
call asks for it, the counters, the pin counts and which expert's bytes each slot of each tensor
holds.

Adapters: `RefAdapter` (the reference's io_sched.cpp built from source with oracle/p1_ref_shim.cpp,
oracle/_ref/libp1_ref.so), `OracleAdapter` (oracle/p1.py) and `ProductAdapter` (the library's
moe_p1_* C-ABI).  The ctypes adapters read from a real file whose rows carry a pattern that names
(layer, expert, tensor), into host-memory slot buffers.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

STAT_IDX = [i for i in range(16) if i != 10]          # io_wait_ns (index 10) is timing
SCRUB_BYTE = 0xA5


def row_pattern(layer: int, eid: int, tensor: int, nbytes: int) -> np.ndarray:
    """The bytes of (layer, expert, tensor)'s row: a 64-bit mix of the four coordinates."""
    w = np.arange(nbytes // 8, dtype=np.uint64)
    x = (np.uint64(layer) << np.uint64(48)) ^ (np.uint64(eid) << np.uint64(32)) ^ \
        (np.uint64(tensor) << np.uint64(24)) ^ w
    x ^= x >> np.uint64(30)
    x *= np.uint64(0xBF58476D1CE4E5B9)
    x ^= x >> np.uint64(27)
    x *= np.uint64(0x94D049BB133111EB)
    x ^= x >> np.uint64(31)
    return x.view(np.uint8)


def make_file(path, layers, n_exp, row_bytes):
    """Write the expert file; returns {layer: [offset of tensor t]}."""
    offs, pos = {}, 0
    with open(path, "wb") as f:
        for l in layers:
            offs[l] = []
            for t, rb in enumerate(row_bytes):
                offs[l].append(pos)
                for e in range(n_exp):
                    f.write(row_pattern(l, e, t, rb).tobytes())
                pos += n_exp * rb
    return offs


def decode_content(bufs, layer, n_exp, row_bytes):
    """[t][slot] -> expert id whose row the slot holds, 'scrub', or None."""
    keys = [{row_pattern(layer, e, t, 8).tobytes(): e for e in range(n_exp)} for t in range(len(row_bytes))]
    out = []
    for t, b in enumerate(bufs):
        col = []
        for s in range(b.shape[0]):
            row = b[s]
            if t == 0 and np.all(row[:min(64, row.size)] == SCRUB_BYTE):
                col.append("scrub")
                continue
            e = keys[t].get(row[:8].tobytes())
            if e is not None and not np.array_equal(row, row_pattern(layer, e, t, row.size)):
                e = "torn"
            col.append(e)
        out.append(col)
    return out


class _CtypesBase:
    """Shared buffer handling for the ctypes adapters (host-memory slot buffers)."""

    def __init__(self, fd, offs, n_exp, row_bytes):
        self.fd, self.offs, self.n_exp, self.rb = fd, offs, n_exp, list(row_bytes)
        self.bufs, self.slot_inds = {}, {}
        self.retired = []          # replaced buffers stay alive: a dropped read may still name them

    def _alloc(self, layer, cap):
        if layer in self.bufs:
            self.retired.append(self.bufs[layer])
        self.bufs[layer] = [np.full((cap, rb), 0xCD, np.uint8) for rb in self.rb]
        self.slot_inds[layer] = np.zeros(16, np.uint32)

    def _ptrs(self, layer):
        return (ctypes.c_uint64 * 9)(*[b.ctypes.data for b in self.bufs[layer]])

    def content(self, layer):
        return decode_content(self.bufs[layer], layer, self.n_exp, self.rb)

    def resize_buffers(self, layer, cap, old_slots):
        new = [np.full((cap, rb), 0xCD, np.uint8) for rb in self.rb]
        for i, s in enumerate(old_slots):
            for t in range(len(self.rb)):
                new[t][i] = self.bufs[layer][t][s]
        self.retired.append(self.bufs[layer])
        self.bufs[layer] = new


def _i32(v):
    return (ctypes.c_int32 * max(len(v), 1))(*v)


def _u32(v):
    return (ctypes.c_uint32 * max(len(v), 1))(*v)


class RefAdapter(_CtypesBase):
    LIB = Path(__file__).resolve().parents[1] / "oracle" / "_ref" / "libp1_ref.so"

    def __init__(self, fd, offs, n_exp, row_bytes, threads=0):
        super().__init__(fd, offs, n_exp, row_bytes)
        L = ctypes.CDLL(str(self.LIB))
        vp = ctypes.c_void_p
        L.r_p1_new.restype = vp
        for n in ("r_p1_free", "r_p1_set_unpin_cb", "r_p1_wait_all"):
            getattr(L, n).argtypes = [vp]
        L.r_p1_layer_init.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                      ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint64]
        L.r_p1_resize.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_uint64,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
        for n in ("r_p1_reset_cache", "r_p1_reset_stats", "r_p1_wait_urgent", "r_p1_wait_layer_all",
                  "r_p1_unpin_layer"):
            getattr(L, n).argtypes = [vp, ctypes.c_int]
        L.r_p1_start_prefetch.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.r_p1_step_decode.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
        L.r_p1_pin.argtypes = L.r_p1_unpin.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_int]
        L.r_p1_pin_count.argtypes = [vp, ctypes.c_int, ctypes.c_int]
        L.r_mt64_new.restype = vp
        L.r_mt64_new.argtypes = [ctypes.c_uint64]
        L.r_mt64_free.argtypes = [vp]
        L.r_mt64_next.restype = ctypes.c_uint64
        L.r_mt64_next.argtypes = [vp]
        L.r_mt64_uniform.restype = ctypes.c_double
        L.r_mt64_uniform.argtypes = [vp]
        L.r_p1_force_invalidate.argtypes = [vp, ctypes.c_int, ctypes.c_double, vp]
        L.r_p1_load_sync.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.r_p1_get_lru.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        L.r_p1_set_lru.argtypes = [vp, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
        L.r_p1_stats.argtypes = L.r_p1_total.argtypes = [vp, ctypes.c_int, ctypes.c_void_p]
        self.L = L
        self.h = L.r_p1_new(threads)
        L.r_p1_set_unpin_cb(self.h)
        self.rng = None

    def close(self):
        self.L.r_p1_free(self.h)
        if self.rng:
            self.L.r_mt64_free(self.rng)

    def seed_rng(self, seed):
        self.rng = self.L.r_mt64_new(seed)

    def layer_init(self, l, cap):
        self._alloc(l, cap)
        u64 = ctypes.c_uint64 * 9
        self.L.r_p1_layer_init(self.h, l, self.fd, cap, len(self.rb), u64(*self.offs[l]), u64(*self.rb),
                               self._ptrs(l), self.slot_inds[l].ctypes.data)

    def resize(self, l, cap, eids, slots, old_slots):
        self.resize_buffers(l, cap, old_slots)
        self.L.r_p1_resize(self.h, l, cap, self._ptrs(l), self.slot_inds[l].ctypes.data, _i32(eids), _i32(slots),
                           len(eids))

    def reset_cache(self, l):
        self.L.r_p1_reset_cache(self.h, l)

    def reset_stats(self, l):
        self.L.r_p1_reset_stats(self.h, l)

    def start_prefetch(self, l, preds, maxf):
        self.L.r_p1_start_prefetch(self.h, l, _i32(preds), len(preds), maxf)

    def step(self, l, eids):
        out = (ctypes.c_uint32 * len(eids))()
        n = self.L.r_p1_step_decode(self.h, l, _u32(eids), len(eids), out)
        return n, list(out)

    def wait_urgent(self, l):
        self.L.r_p1_wait_urgent(self.h, l)

    def wait_layer_all(self, l):
        self.L.r_p1_wait_layer_all(self.h, l)

    def unpin_layer(self, l):
        self.L.r_p1_unpin_layer(self.h, l)

    def pin(self, l, slots):
        self.L.r_p1_pin(self.h, l, _u32(slots), len(slots))

    def unpin(self, l, slots):
        self.L.r_p1_unpin(self.h, l, _u32(slots), len(slots))

    def pin_counts(self, l, cap):
        return [self.L.r_p1_pin_count(self.h, l, s) for s in range(cap)]

    def force_invalidate(self, l, rate):
        return self.L.r_p1_force_invalidate(self.h, l, rate, self.rng)

    def load_sync(self, l, eids, slots, prefill):
        self.L.r_p1_load_sync(self.h, l, _i32(eids), _i32(slots), len(eids), int(prefill))

    def get_lru(self, l):
        e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
        self.L.r_p1_get_lru(self.h, l, e, s, ctypes.byref(n))
        return list(e[:n.value]), list(s[:n.value])

    def set_lru(self, l, eids, slots, a, b, c):
        self.L.r_p1_set_lru(self.h, l, _i32(eids), _i32(slots), len(eids), a, b, c)

    def stats(self, l):
        out = (ctypes.c_uint64 * 16)()
        self.L.r_p1_stats(self.h, l, out)
        return [int(out[i]) for i in STAT_IDX]


class OracleAdapter:
    def __init__(self, n_exp, row_bytes):
        from oracle import p1
        self.p1mod = p1
        self.P = p1.P1()
        self.P.reader_cb = self.P.unpin_layer_slots
        self.n_exp, self.rb = n_exp, list(row_bytes)
        self.rng = None

    def close(self):
        pass

    def seed_rng(self, seed):
        self.rng = self.p1mod.MT64(seed)

    def layer_init(self, l, cap):
        self.P.layer_init(l, cap, self.rb)

    def resize(self, l, cap, eids, slots, old_slots):
        old = self.P.layers[l].content
        new = [[col[s] if s < len(col) else None for s in old_slots] + [None] * (cap - len(old_slots)) for col in old]
        self.P.resize_layer(l, cap, eids, slots, content=new)

    def reset_cache(self, l):
        self.P.reset_cache(l)

    def reset_stats(self, l):
        self.P.reset_stats(l)

    def start_prefetch(self, l, preds, maxf):
        self.P.start_prefetch(l, preds, maxf)

    def step(self, l, eids):
        return self.P.step_decode(l, eids)

    def wait_urgent(self, l):
        self.P.wait_layer_urgent(l)

    def wait_layer_all(self, l):
        self.P.wait_layer_all(l)

    def unpin_layer(self, l):
        self.P.unpin_layer_slots(l)

    def pin(self, l, slots):
        self.P.pin_slots(l, slots)

    def unpin(self, l, slots):
        self.P.unpin_slots(l, slots)

    def pin_counts(self, l, cap):
        return [self.P.get_slot_pin_count(l, s) for s in range(cap)]

    def force_invalidate(self, l, rate):
        return self.P.force_invalidate(l, rate, self.rng.uniform)

    def load_sync(self, l, eids, slots, prefill):
        self.P.load_sync(l, eids, slots, prefill)

    def get_lru(self, l):
        return self.P.get_lru_state(l)

    def set_lru(self, l, eids, slots, a, b, c):
        self.P.set_lru_state(l, eids, slots, a, b, c)

    def stats(self, l):
        st = self.P.get_layer_stats(l)
        return [st[k] for i, k in enumerate(self.p1mod.STAT_KEYS) if i != 10]

    def content(self, l):
        return [list(col) for col in self.P.layers[l].content]


def apply_op(ad, op, caps):
    """Run one call on adapter `ad` (caps: layer -> capacity, kept across calls); its record."""
    kind, l = op["op"], op.get("l", 0)
    rec = {}
    if kind == "init":
        ad.layer_init(l, op["cap"])
        caps[l] = op["cap"]
    elif kind == "resize":
        ad.resize(l, op["cap"], op["eids"], op["slots"], op["old_slots"])
        caps[l] = op["cap"]
    elif kind == "reset_cache":
        ad.reset_cache(l)
    elif kind == "reset_stats":
        ad.reset_stats(l)
    elif kind == "prefetch":
        ad.start_prefetch(l, op["preds"], op["maxf"])
    elif kind == "step":
        n, slots = ad.step(l, op["eids"])
        rec["ret"], rec["slots"] = n, slots
    elif kind == "wait_urgent":
        ad.wait_urgent(l)
    elif kind == "wait_all":
        ad.wait_layer_all(l)
    elif kind == "unpin_layer":
        ad.unpin_layer(l)
    elif kind == "pin":
        ad.pin(l, op["slots"])
    elif kind == "unpin":
        ad.unpin(l, op["slots"])
    elif kind == "invalidate":
        rec["ret"] = ad.force_invalidate(l, op["rate"])
    elif kind == "load_sync":
        ad.load_sync(l, op["eids"], op["slots"], op["prefill"])
    elif kind == "get_lru":
        rec["lru"] = [list(v) for v in ad.get_lru(l)]
    elif kind == "set_lru":
        ad.set_lru(l, op["eids"], op["slots"], *op["add"])
    else:
        raise ValueError(kind)
    if op.get("check") or kind in ("step", "invalidate"):
        rec["stats"] = ad.stats(l)
    if op.get("check"):
        rec["pins"] = ad.pin_counts(l, caps[l])
        rec["content"] = ad.content(l)
    return rec


def replay(ad, trace):
    """Run the trace's calls on adapter `ad`; returns one record per call."""
    caps = {}
    if trace.get("rng_seed") is not None:
        ad.seed_rng(trace["rng_seed"])
    return [apply_op(ad, op, caps) for op in trace["ops"]]


class ProductAdapter(_CtypesBase):
    """The library's moe_p1_* entry points (no reader callback: pinned slots are released by the
    scheduler's own reader wait, which unpins the layer -- what the reference runner's callback
    does)."""

    def __init__(self, fd, offs, n_exp, row_bytes, threads=0, lib=None):
        super().__init__(fd, offs, n_exp, row_bytes)
        from moe_offload import _lib
        self._libmod = _lib
        self.L = lib or _lib.lib()
        self.h = self.L.moe_p1_create()
        self.L.moe_p1_init(self.h, threads)
        self.rng = None
        self.draw = ctypes.cast(self.L.moe_p1_mt64_uniform, ctypes.c_void_p)

    def close(self):
        self.L.moe_p1_destroy(self.h)
        if self.rng:
            self.L.moe_p1_mt64_destroy(self.rng)

    def seed_rng(self, seed):
        self.rng = self.L.moe_p1_mt64_create(seed)

    def layer_init(self, l, cap):
        self._alloc(l, cap)
        u64 = ctypes.c_uint64 * 9
        self.L.moe_p1_layer_init(self.h, l, self.fd, cap, len(self.rb), u64(*self.offs[l]), u64(*self.rb),
                                 self._ptrs(l), self.slot_inds[l].ctypes.data)

    def resize(self, l, cap, eids, slots, old_slots):
        self.resize_buffers(l, cap, old_slots)
        self.L.moe_p1_resize_layer(self.h, l, cap, self._ptrs(l), self.slot_inds[l].ctypes.data, _i32(eids),
                                   _i32(slots), len(eids))

    def reset_cache(self, l):
        self.L.moe_p1_reset_cache(self.h, l)

    def reset_stats(self, l):
        self.L.moe_p1_reset_stats(self.h, l)

    def start_prefetch(self, l, preds, maxf):
        self.L.moe_p1_start_prefetch(self.h, l, _i32(preds), len(preds), maxf)

    def step(self, l, eids):
        out = (ctypes.c_uint32 * len(eids))()
        n = self.L.moe_p1_step_decode(self.h, l, _u32(eids), len(eids), out)
        return n, list(out)

    def wait_urgent(self, l):
        self.L.moe_p1_wait_layer_urgent(self.h, l)

    def wait_layer_all(self, l):
        self.L.moe_p1_wait_layer_all(self.h, l)

    def unpin_layer(self, l):
        self.L.moe_p1_unpin_layer_slots(self.h, l)

    def pin(self, l, slots):
        self.L.moe_p1_pin_slots(self.h, l, _u32(slots), len(slots))

    def unpin(self, l, slots):
        self.L.moe_p1_unpin_slots(self.h, l, _u32(slots), len(slots))

    def pin_counts(self, l, cap):
        return [self.L.moe_p1_get_slot_pin_count(self.h, l, s) for s in range(cap)]

    def force_invalidate(self, l, rate):
        return self.L.moe_p1_force_invalidate(self.h, l, rate, self.draw, self.rng)

    def load_sync(self, l, eids, slots, prefill):
        self.L.moe_p1_load_sync(self.h, l, _i32(eids), _i32(slots), len(eids), int(prefill))

    def get_lru(self, l):
        e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
        self.L.moe_p1_get_lru_state(self.h, l, e, s, ctypes.byref(n))
        return list(e[:n.value]), list(s[:n.value])

    def set_lru(self, l, eids, slots, a, b, c):
        self.L.moe_p1_set_lru_state(self.h, l, _i32(eids), _i32(slots), len(eids), a, b, c)

    def stats(self, l):
        out = (ctypes.c_uint64 * 16)()
        self.L.moe_p1_get_layer_stats(self.h, l, out)
        return [int(out[i]) for i in STAT_IDX]
