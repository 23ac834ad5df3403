"""GPU parity of the slot tables and miss staging.

* device-driven tables (single-wave kernels) replay the reference expert_io.c golden traces;
* host-driven (DMA) and device-driven (kernel) staging leave pool[slot] == store[eid];
* the config-2 single-layer decode (128 steps, 102 slots, Zipf id stream) gives the reference's
  slot/miss sequence and SwitchGLU outputs within 1e-2 x RMS of the oracle, in both modes.
"""
import ctypes

import numpy as np
import pytest

from helpers import E, H, I, K, assert_close_rms, experts_np, oracle_moe

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def L():
    from moe_offload import _lib
    assert torch.cuda.is_available()
    lib = _lib.lib()
    lib.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    return lib


def _check(lib):
    from moe_offload import _lib
    _lib.check_error("native")


def _stats(lib, layer):
    o = (ctypes.c_uint64 * 18)()
    lib.c_layer_get_stats(layer, o)
    return list(o)


def _state(lib, layer):
    e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int()
    lib.c_layer_get_lru_state(layer, e, s, ctypes.byref(c))
    return [list(e[:c.value]), list(s[:c.value])]


def _init_layer(lib, layer, cap, store_ptr=0, blob=1_536_000, pool_ptr=0, slot_ptr=0):
    u64 = ctypes.c_uint64 * 9
    lib.c_layer_init(layer, -1, cap, u64(store_ptr, *[0] * 8), u64(blob, *[0] * 8), u64(pool_ptr, *[0] * 8), slot_ptr)
    _check(lib)


def test_device_table_replays_reference_traces(L, lru_traces):
    stream = torch.cuda.current_stream().cuda_stream
    for n, scen in enumerate(lru_traces["scenarios"]):
        layer = 50 + n
        slots = torch.zeros(16, dtype=torch.int32, device="cuda")
        _init_layer(L, layer, scen["capacity"], slot_ptr=slots.data_ptr())
        assert L.c_layer_set_device_mode(layer, 1) == 0, scen["name"]
        for op in scen["ops"]:
            if op["op"] == "prefetch":
                p = torch.tensor(op["preds"], dtype=torch.int32, device="cuda")
                assert L.c_layer_start_prefetch_dev(layer, p.data_ptr(), p.numel(), op["cap"], 0, stream) == 0
            elif op["op"] == "step":
                ids = torch.tensor(op["ids"], dtype=torch.int32, device="cuda")
                assert L.c_layer_step_decode_dev(layer, ids.data_ptr(), ids.numel(), 0, stream) == 0
                got = slots[:ids.numel()].cpu().tolist()
                assert got == op["slots"], (scen["name"], op)
            elif op["op"] == "set_state":
                e, s = op["eids"], op["slots"]
                L.c_layer_set_lru_state(layer, (ctypes.c_int32 * max(1, len(e)))(*e),
                                        (ctypes.c_int32 * max(1, len(s)))(*s), len(e), *op["add"])
            elif op["op"] == "load_sync":
                e, s = op["eids"], op["slots"]
                L.c_layer_load_sync(layer, (ctypes.c_int32 * len(e))(*e), (ctypes.c_int32 * len(s))(*s), len(e), 1)
            _check(L)
            assert _stats(L, layer) == op["stats"], (scen["name"], op["op"])
            if "state" in op:
                assert _state(L, layer) == op["state"], scen["name"]
        assert _state(L, layer) == scen["final_state"]
        assert L.c_layer_table_status(layer) == 0


class DeviceSched:
    """Device-driven tables in scheduler mode, driven with the golden scheduler traces: the
    step and the next layer's prefetch of a c_layer_decode_step_sched call run as the device
    table kernels (published ops of the mixed scenario with scheduler mode switched off).  A
    step whose call carries the SPLIT flag runs with table mode bit 1, so the kernel records the
    split lists; accounting and token bracketing go through the same c_set_io_accounting /
    c_begin_decode_token / c_end_decode_token calls as host tables, whose counters the device
    tables keep themselves.  Miss counts are read as the change of the layer's demand-miss
    counter.  Layers keep the trace's numbers: layer 1's cache reset restarts the token
    numbering, as the trace expects."""

    def __init__(self, lib):
        from sched_replay import TokenMixin
        self._tokens = TokenMixin()
        self.L = lib
        self.slots, self.misses, self.mode = {}, {}, {}
        self.stream = torch.cuda.current_stream().cuda_stream

    def begin_if_needed(self):
        if not self._tokens._open:
            self.L.c_begin_decode_token(0)
            self._tokens._open = True

    def token_done(self):
        self._tokens._open = False

    def end(self):
        o = (ctypes.c_uint64 * 10)()
        self.L.c_end_decode_token(o)
        _check(self.L)
        return list(o)

    def init(self, l, cap):
        self.slots[l] = torch.zeros(16, dtype=torch.int32, device="cuda")
        _init_layer(self.L, l, cap, slot_ptr=self.slots[l].data_ptr())
        assert self.L.c_layer_set_device_mode(l, 1) == 0
        self._set_mode(l, 1)
        self.misses[l] = 0

    def _set_mode(self, l, mode):
        if self.mode.get(l) != mode:
            assert self.L.c_layer_set_sched(l, mode) == 0
            self.mode[l] = mode

    def reset_stats(self, l):
        self.L.c_layer_reset_stats(l)
        self.misses[l] = 0

    def reset_cache(self, l):
        self.L.c_layer_reset_cache(l)

    def accounting(self, on):
        self.L.c_set_io_accounting(1 if on else 0)

    def _step(self, l, ids):
        t = torch.tensor(ids, dtype=torch.int32, device="cuda")
        assert self.L.c_layer_step_decode_dev(l, t.data_ptr(), len(ids), 0, self.stream) == 0
        _check(self.L)
        m = self.stats(l)[3]
        n, self.misses[l] = m - self.misses[l], m
        return n, self.slots[l][:len(ids)].cpu().tolist()

    def _prefetch(self, l, preds, cap):
        p = torch.tensor(preds, dtype=torch.int32, device="cuda")
        assert self.L.c_layer_start_prefetch_dev(l, p.data_ptr(), len(preds), cap, 0, self.stream) == 0
        _check(self.L)

    def sched(self, l, ids, preds, nxt, cap, flags):
        from sched_replay import SPLIT
        if l > 0 and ids:
            self._set_mode(l, 1 | (2 if flags & SPLIT else 0))
            n, slots = self._step(l, ids)
        else:
            n, slots = 0, []
        if not (flags & 2) and nxt > 0 and preds:
            self._set_mode(nxt, self.mode.get(nxt, 1) | 1)
            self._prefetch(nxt, preds, cap)
        return n, slots

    def _published(self, l, fn):
        self._set_mode(l, 0)
        return fn()

    def step(self, l, ids):
        return self._published(l, lambda: self._step(l, ids))

    def prefetch(self, l, preds, cap):
        self._published(l, lambda: self._prefetch(l, preds, cap))

    def stats(self, l):
        return _stats(self.L, l)

    def state(self, l):
        return _state(self.L, l)

    def set_state(self, l, e, s, add):
        self.L.c_layer_set_lru_state(l, (ctypes.c_int32 * max(1, len(e)))(*e),
                                     (ctypes.c_int32 * max(1, len(s)))(*s), len(e), *add)

    def split(self, l):
        h = (ctypes.c_uint32 * 16)(*([0xFFFFFFFF] * 16))
        m = (ctypes.c_uint32 * 16)(*([0xFFFFFFFF] * 16))
        inv = (ctypes.c_int32 * 16)(*([-7] * 16))
        self.L.c_layer_get_split_inds(l, h, m, inv)
        _check(self.L)
        return [[v for v in h if v != 0xFFFFFFFF], [v for v in m if v != 0xFFFFFFFF], [v for v in inv if v != -7]]

    def totals(self, n_layers):
        t = [0] * 6
        for l in range(1, n_layers):
            st = self.stats(l)
            for i, w in enumerate((1, 2, 3, 0, 4, 5)):     # c_get_decode_totals' order
                t[i] += st[w]
        return t


def test_device_tables_replay_reference_scheduler_traces(L):
    """Scheduler-mode device tables against the reference's cpp/third_party/expert_io.c traces:
    decisions, counters, split lists and per-token accounting."""
    from sched_replay import load, replay
    try:
        for sc in load()["scenarios"]:
            assert replay(sc, DeviceSched(L)) > 50, sc["name"]
    finally:
        L.c_set_io_accounting(0)
        for l in range(1, 8):                 # back to host tables for the tests that follow
            L.c_layer_init(l, -1, 16, None, None, None, 0)
        torch.cuda.synchronize()


def test_device_table_rejects_bad_ids(L):
    stream = torch.cuda.current_stream().cuda_stream
    slots = torch.zeros(16, dtype=torch.int32, device="cuda")
    _init_layer(L, 60, 32, slot_ptr=slots.data_ptr())
    assert L.c_layer_set_device_mode(60, 1) == 0
    ids = torch.tensor([1, 2, 999, 4], dtype=torch.int32, device="cuda")
    assert L.c_layer_step_decode_dev(60, ids.data_ptr(), 4, 0, stream) == 0
    assert L.c_layer_table_status(60) == 1
    assert _stats(L, 60)[0] == 0 and _state(L, 60) == [[], []]


@pytest.mark.parametrize("mode", ["host", "device"])
def test_staging_fills_slots_with_the_right_experts(L, mode):
    """Small blobs (hidden 256, inter 128): after every step and prefetch, the slots of the
    step's experts hold exactly those experts' bytes."""
    from moe_offload import q2format
    stream = torch.cuda.current_stream().cuda_stream
    blob = q2format.expert_bytes(256, 128)
    n_exp, cap = 512, 24
    ptr = L.c_host_alloc(n_exp * blob)
    assert ptr
    try:
        store = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(n_exp, blob))
        store[:] = np.random.default_rng(0).integers(0, 256, size=store.shape, dtype=np.uint8)
        store_dev = torch.from_numpy(store.copy()).to("cuda")
        pool = torch.zeros((cap, blob), dtype=torch.uint8, device="cuda")
        slots = torch.zeros(16, dtype=torch.int32, device="cuda")
        layer = 61 if mode == "host" else 62
        _init_layer(L, layer, cap, store_ptr=ptr, blob=blob, pool_ptr=pool.data_ptr(), slot_ptr=slots.data_ptr())
        if mode == "device":
            assert L.c_layer_set_device_mode(layer, 1) == 0
        rng = np.random.default_rng(1)
        for t in range(40):
            preds = rng.choice(96, size=12, replace=False).astype(np.int32)
            ids = rng.choice(96, size=K, replace=False).astype(np.uint32)
            if mode == "host":
                L.c_layer_start_prefetch12(layer, 3, *[int(v) for v in preds])
                L.c_layer_step_decode10_async(layer, *[int(v) for v in ids])
                L.c_layer_wait_prefetch(layer)
            else:
                p = torch.from_numpy(preds).to("cuda")
                i = torch.from_numpy(ids.astype(np.int32)).to("cuda")
                assert L.c_layer_start_prefetch_dev(layer, p.data_ptr(), 12, 3, 0, stream) == 0
                assert L.c_layer_step_decode_dev(layer, i.data_ptr(), K, 0, stream) == 0
            _check(L)
            sl = slots[:K].long()
            assert torch.equal(pool[sl], store_dev[torch.from_numpy(ids.astype(np.int64)).to("cuda")]), f"step {t}"
        # every resident slot holds its expert
        e, s = _state(L, layer)
        assert torch.equal(pool[torch.tensor(s, device="cuda")], store_dev[torch.tensor(e, device="cuda")])
        torch.cuda.synchronize()
        L.c_sync_copies()
    finally:
        torch.cuda.synchronize()
        L.c_sync_copies()
        L.c_layer_init(61 if mode == "host" else 62, -1, 16, None, None, None, 0)
        L.c_host_free(ptr)


def test_load_sync_copies(L):
    """c_layer_load_sync from a pinned store (CU copy kernel, 128 pairs per launch): 300 pairs in
    one call land in their slots; a slot named twice in one call holds the later pair's expert,
    as when the copies run one after the other (expert_io.c:710-724)."""
    from moe_offload import q2format
    blob = q2format.expert_bytes(256, 128)
    n_exp, cap, layer = 512, 300, 63
    ptr = L.c_host_alloc(n_exp * blob)
    assert ptr
    try:
        store = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(n_exp, blob))
        store[:] = np.random.default_rng(5).integers(0, 256, size=store.shape, dtype=np.uint8)
        store_dev = torch.from_numpy(store.copy()).to("cuda")
        pool = torch.zeros((cap, blob), dtype=torch.uint8, device="cuda")
        slots = torch.zeros(16, dtype=torch.int32, device="cuda")
        _init_layer(L, layer, cap, store_ptr=ptr, blob=blob, pool_ptr=pool.data_ptr(), slot_ptr=slots.data_ptr())
        rng = np.random.default_rng(6)
        eids = rng.choice(n_exp, size=cap, replace=False).astype(np.int32)
        sl = rng.permutation(cap).astype(np.int32)
        c32 = ctypes.c_int32 * cap
        L.c_layer_load_sync(layer, c32(*eids.tolist()), c32(*sl.tolist()), cap, 1)
        _check(L)
        torch.cuda.synchronize()
        assert torch.equal(pool[torch.from_numpy(sl.astype(np.int64)).to("cuda")],
                           store_dev[torch.from_numpy(eids.astype(np.int64)).to("cuda")])
        # slot 5 named twice (expert 7, then 9), slot 6 once
        pairs_e, pairs_s = [7, 11, 9], [5, 6, 5]
        c3 = ctypes.c_int32 * 3
        L.c_layer_load_sync(layer, c3(*pairs_e), c3(*pairs_s), 3, 1)
        _check(L)
        torch.cuda.synchronize()
        assert torch.equal(pool[5], store_dev[9]) and torch.equal(pool[6], store_dev[11])
    finally:
        torch.cuda.synchronize()
        L.c_sync_copies()
        L.c_layer_init(layer, -1, 16, None, None, None, 0)
        L.c_host_free(ptr)


def test_host_staging_small_pool_victims_of_inflight_prefetch(L):
    """Host-driven staging at the 16-slot floor with prefetch cap 8: a demand miss then takes a
    slot that the prefetch just before it is still filling, and the two copies must land in
    order (the later one wins).  After every step the step's slots hold its experts; a
    load_sync right after a prefetch (the prefill chunk's pattern) must win over it too."""
    from moe_offload import q2format
    blob = q2format.expert_bytes(256, 128)
    n_exp, cap, layer = 512, 16, 63
    ptr = L.c_host_alloc(n_exp * blob)
    assert ptr
    try:
        store = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(n_exp, blob))
        store[:] = np.random.default_rng(5).integers(0, 256, size=store.shape, dtype=np.uint8)
        store_dev = torch.from_numpy(store.copy()).to("cuda")
        pool = torch.zeros((cap, blob), dtype=torch.uint8, device="cuda")
        slots = torch.zeros(16, dtype=torch.int32, device="cuda")
        _init_layer(L, layer, cap, store_ptr=ptr, blob=blob, pool_ptr=pool.data_ptr(), slot_ptr=slots.data_ptr())
        rng = np.random.default_rng(6)
        collisions = 0
        for t in range(60):
            preds = rng.choice(200, size=12, replace=False).astype(np.int32)
            ids = rng.choice(200, size=K, replace=False).astype(np.uint32)
            before = set(_state(L, layer)[0])
            L.c_layer_start_prefetch12(layer, 8, *[int(v) for v in preds])
            e0, s0 = _state(L, layer)
            pf_slots = {sl for e, sl in zip(e0, s0) if e not in before}      # being filled now
            L.c_layer_step_decode10_async(layer, *[int(v) for v in ids])
            L.c_layer_wait_prefetch(layer)
            _check(L)
            got = slots[:K].cpu().tolist()
            collisions += len(pf_slots & {sl for sl, e in zip(got, ids) if int(e) not in set(e0)})
            sl = slots[:K].long()
            assert torch.equal(pool[sl], store_dev[torch.from_numpy(ids.astype(np.int64)).to("cuda")]), f"step {t}"
            if t % 10 == 9:
                # a blocking load right behind a prefetch into the same slots
                L.c_layer_start_prefetch12(layer, 8, *[int(v) for v in rng.choice(200, size=12, replace=False)])
                le = rng.choice(np.arange(300, 512), size=cap, replace=False).astype(np.int32)
                ls = np.arange(cap, dtype=np.int32)
                L.c_layer_load_sync(layer, le.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                    ls.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), cap, 1)
                _check(L)
                assert torch.equal(pool, store_dev[torch.from_numpy(le.astype(np.int64)).to("cuda")]), f"load {t}"
                L.c_layer_reset_cache(layer)
        assert collisions > 0, "the id stream never made a demand miss take an in-flight prefetch slot"
        torch.cuda.synchronize()
        L.c_sync_copies()
    finally:
        torch.cuda.synchronize()
        L.c_sync_copies()
        L.c_layer_init(layer, -1, 16, None, None, None, 0)
        L.c_host_free(ptr)


@pytest.fixture(scope="module")
def config2_store(L):
    """512 experts at H=2048, I=512 in a pinned host store (503 MB)."""
    mlx, blobs = experts_np(E, H, I, seed=1)
    blob = blobs.shape[1]
    ptr = L.c_host_alloc(E * blob)
    assert ptr
    store = np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)), shape=(E, blob))
    store[:] = blobs
    del blobs
    yield mlx, ptr, blob
    torch.cuda.synchronize()
    L.c_sync_copies()
    for layer in (57, 58):
        L.c_layer_init(layer, -1, 16, None, None, None, 0)
    L.c_host_free(ptr)


@pytest.mark.parametrize("mode", ["host", "device"])
def test_config2_single_layer_decode(L, lru_traces, config2_store, mode):
    from moe_offload import synth
    mlx, ptr, blob = config2_store
    stream = torch.cuda.current_stream().cuda_stream
    trace = next(s for s in lru_traces["scenarios"] if s["name"] == "config2_cap102_noprefetch")
    steps = [op for op in trace["ops"] if op["op"] == "step"]
    ids_all = synth.expert_id_stream(steps=128, k=K, seed=2)
    assert ids_all.tolist() == [op["ids"] for op in steps]
    cap = 102
    layer = 57 if mode == "host" else 58
    pool = torch.zeros((cap, blob), dtype=torch.uint8, device="cuda")
    slots = torch.zeros(16, dtype=torch.int32, device="cuda")
    _init_layer(L, layer, cap, store_ptr=ptr, blob=blob, pool_ptr=pool.data_ptr(), slot_ptr=slots.data_ptr())
    assert L.c_layer_set_format(layer, H, I, 64) == 0
    if mode == "device":
        assert L.c_layer_set_device_mode(layer, 1) == 0
    xs = synth.hidden_states(128, H, seed=31)
    rng = np.random.default_rng(32)
    h_ws = torch.empty(K * I, dtype=torch.float16, device="cuda")
    y = torch.empty(H, dtype=torch.float32, device="cuda")
    for t in range(128):
        ids = ids_all[t]
        sc = rng.dirichlet(np.ones(K)).astype(np.float16)
        sct = torch.from_numpy(sc).to("cuda")
        xt = torch.from_numpy(xs[t]).to("cuda")
        if mode == "host":
            n = L.c_layer_step_decode10_async(layer, *[int(v) for v in ids])
            if n > 0:
                L.c_layer_wait_prefetch(layer)
        else:
            i = torch.from_numpy(ids.astype(np.int32)).to("cuda")
            assert L.c_layer_step_decode_dev(layer, i.data_ptr(), K, 0, stream) == 0
        assert L.c_layer_switch_glu(layer, xt.data_ptr(), sct.data_ptr(), None, h_ws.data_ptr(), y.data_ptr(), 0,
                                    K, stream) == 0
        _check(L)
        assert slots[:K].cpu().tolist() == steps[t]["slots"], f"step {t}"
        if t % 8 == 0 or t == 127:
            assert_close_rms(y.cpu().numpy(), oracle_moe(xs[t], ids, sc, mlx), 1e-2, f"step {t}")
    st = _stats(L, layer)
    ref = steps[-1]["stats"]
    assert st[:4] == ref[:4]                                   # requests, hits, misses
    assert st[4] == ref[3] * blob                              # real bytes per miss
