"""P1 I/O scheduler (the C++ runner's `--io p1` cache, mlx-qwen38/cpp/src/io_sched.{h,cpp}) on the CPU.

* the oracle (oracle/p1.py) and the library (moe_p1_*, no reader threads, host-memory slot
  buffers) replay the golden traces that the reference's own io_sched.cpp wrote
  (tests/golden/make_p1_traces.py): slots, pending counts, 15 counters, pin counts and which
  expert's bytes every slot row holds, call for call;
* where the reference build is present, the oracle also matches it on fresh random traces;
* the generator behind force_invalidate: std::mt19937_64's known answer and libstdc++'s
  uniform_real_distribution, in the oracle and in the library;
* the reference's own test scenarios (cpp/tests/test_io_sched.cpp): queued prefetches cancelled and
  promoted with exact counts; an allocation that meets pinned slots waits for the reader callback
  while a concurrent "GPU reader" holds them; a 250-step stress with 8 reader threads, 4 layers,
  resizes, forced invalidations and concurrent readers that check every slot's bytes.
"""
from __future__ import annotations

import ctypes
import gzip
import json
import os
import random
import threading
from pathlib import Path

import numpy as np
import pytest

from oracle import p1 as op1
from p1_replay import OracleAdapter, ProductAdapter, RefAdapter, make_file, replay, row_pattern

HERE = Path(__file__).resolve().parent
GOLDEN = HERE / "golden" / "p1_traces.json.gz"


@pytest.fixture(scope="module")
def golden():
    return json.load(gzip.open(GOLDEN, "rt"))


@pytest.fixture(scope="module")
def expert_file(tmp_path_factory, golden):
    path = tmp_path_factory.mktemp("p1") / "experts.bin"
    offs = make_file(path, golden["layers"], golden["n_exp"], golden["row_bytes"])
    fd = os.open(path, os.O_RDONLY)
    yield fd, offs
    os.close(fd)


def _lib():
    from moe_offload import _lib as lm
    return lm.lib()


def test_mt64_known_answer_and_uniform_draws():
    g = op1.MT64(5489)
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042          # [rand.predef]: the 10000th value of mt19937_64
    L = _lib()
    h = L.moe_p1_mt64_create(5489)
    o = op1.MT64(5489)
    try:
        for _ in range(2000):
            assert L.moe_p1_mt64_uniform(h) == o.uniform()
        assert L.moe_p1_mt64_next(h) == o()
    finally:
        L.moe_p1_mt64_destroy(h)
    assert op1.MT64(1).uniform() < 1.0


def _check_replay(ad_factory, golden):
    for tr in golden["traces"]:
        ad = ad_factory()
        try:
            got = replay(ad, tr)
        finally:
            ad.close()
        assert len(got) == len(tr["expect"])
        for i, (want, have) in enumerate(zip(tr["expect"], got)):
            assert have == want, f"seed {tr['seed']} call {i} {tr['ops'][i]}"


def test_oracle_replays_reference_traces(golden):
    _check_replay(lambda: OracleAdapter(golden["n_exp"], golden["row_bytes"]), golden)


def test_library_replays_reference_traces(golden, expert_file):
    fd, offs = expert_file
    _check_replay(lambda: ProductAdapter(fd, offs, golden["n_exp"], golden["row_bytes"], threads=0), golden)


@pytest.mark.skipif(not RefAdapter.LIB.exists(), reason="reference build absent (oracle/_ref)")
def test_oracle_matches_reference_build_on_fresh_traces(golden, expert_file):
    import sys
    sys.path.insert(0, str(HERE / "golden"))
    import make_p1_traces as gen
    fd, offs = expert_file
    checked = 0
    for seed in range(10_001, 10_013):
        try:
            tr = gen.bind_resizes(gen.gen_trace(seed))
        except op1.Deadlock:
            continue
        recs = gen.run_ref(tr, os.readlink(f"/proc/self/fd/{fd}"), offs)
        if recs is None:                         # the reference sleeps forever: the oracle must raise
            with pytest.raises(op1.Deadlock):
                replay(OracleAdapter(golden["n_exp"], golden["row_bytes"]), tr)
            continue
        assert replay(OracleAdapter(golden["n_exp"], golden["row_bytes"]), tr) == recs, seed
        checked += 1
    assert checked >= 6


# -- the reference's own scenarios (cpp/tests/test_io_sched.cpp) on the library ---------------------
N_EXP, NT = 32, 9
ROW = [1024, 256, 256, 1024, 256, 256, 1024, 256, 256]       # test_io_sched.cpp:28-32


class Bufs:
    def __init__(self, layer, cap):
        self.layer, self.cap = layer, cap
        self.t = [np.full((cap, rb), 0xCD, np.uint8) for rb in ROW]
        self.slot_inds = np.zeros(16, np.uint32)

    def ptrs(self):
        return (ctypes.c_uint64 * 9)(*[a.ctypes.data for a in self.t])

    def verify(self, eid, slot):
        for t, rb in enumerate(ROW):
            assert np.array_equal(self.t[t][slot], row_pattern(self.layer, eid, t, rb)), (self.layer, eid, slot, t)


@pytest.fixture(scope="module")
def scen_file(tmp_path_factory):
    path = tmp_path_factory.mktemp("p1s") / "synth.bin"
    offs = make_file(path, [1, 2, 3, 4], N_EXP, ROW)
    fd = os.open(path, os.O_RDONLY)
    yield fd, offs
    os.close(fd)


def _u64(v):
    return (ctypes.c_uint64 * 9)(*v)


def _i32(v):
    return (ctypes.c_int32 * len(v))(*v)


def _u32(v):
    return (ctypes.c_uint32 * len(v))(*v)


def _stats(L, h, l):
    out = (ctypes.c_uint64 * 16)()
    L.moe_p1_get_layer_stats(h, l, out)
    return dict(zip(op1.STAT_KEYS, [int(v) for v in out]))


def _init_layer(L, h, fd, offs, l, buf, eids):
    L.moe_p1_layer_init(h, l, fd, buf.cap, NT, _u64(offs[l]), _u64(ROW), buf.ptrs(), buf.slot_inds.ctypes.data)
    slots = list(range(len(eids)))
    L.moe_p1_load_sync(h, l, _i32(eids), _i32(slots), len(eids), 1)
    L.moe_p1_set_lru_state(h, l, _i32(eids), _i32(slots), len(eids), len(eids), 0, len(eids))
    for e, s in zip(eids, slots):
        buf.verify(e, s)


def test_cancel_and_promote(scen_file):
    """test_io_sched.cpp:150-200: queued prefetches {10, 11, 12}; the step routes {0, 10, 20, 21}:
    two cancelled, one promoted (not read twice), two demand reads."""
    fd, offs = scen_file
    L = _lib()
    h = L.moe_p1_create()
    L.moe_p1_init(h, 0)
    try:
        buf = Bufs(1, 4)
        _init_layer(L, h, fd, offs, 1, buf, [0, 1, 2, 3])
        L.moe_p1_unpin_layer_slots(h, 1)
        L.moe_p1_start_prefetch(h, 1, _i32([10, 11, 12]), 3, 3)
        route = [0, 10, 20, 21]
        out = (ctypes.c_uint32 * 4)()
        assert L.moe_p1_step_decode(h, 1, _u32(route), 4, out) > 0
        L.moe_p1_wait_layer_urgent(h, 1)
        for e, s in zip(route, out):
            buf.verify(e, s)
        assert list(buf.slot_inds[:4]) == list(out)
        st = _stats(L, h, 1)
        assert (st["prefetch_issued"], st["prefetch_cancelled"], st["prefetch_promoted"], st["prefetch_used"],
                st["urgent_reads"]) == (3, 2, 1, 1, 2)
        assert st["bytes"] == 3 * sum(ROW)             # the promoted prefetch and the two misses, once each
    finally:
        L.moe_p1_destroy(h)


def test_pin_waits_and_reader_callback(scen_file):
    """test_io_sched.cpp:202-255: 4 of 6 slots pinned by a slow "GPU reader"; a prefetch of 3 new
    experts must wait for it through the reader callback (pin_waits >= 1) and never touch its slots."""
    fd, offs = scen_file
    L = _lib()
    h = L.moe_p1_create()
    L.moe_p1_init(h, 4)
    gpu_done = threading.Event()
    reader = {}

    @ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_void_p)
    def wait_reader(layer, _user):
        t = reader.get(layer)
        if t is not None:
            t.join()
        assert gpu_done.is_set()
        L.moe_p1_unpin_layer_slots(h, layer)

    try:
        buf = Bufs(1, 6)
        _init_layer(L, h, fd, offs, 1, buf, [0, 1, 2, 3, 4, 5])
        L.moe_p1_set_wait_reader_callback(h, ctypes.cast(wait_reader, ctypes.c_void_p), None)
        step = [0, 1, 2, 3]
        out = (ctypes.c_uint32 * 4)()
        if L.moe_p1_step_decode(h, 1, _u32(step), 4, out) > 0:
            L.moe_p1_wait_layer_urgent(h, 1)
        slots = list(out)

        def gpu():
            threading.Event().wait(0.015)
            for e, s in zip(step, slots):
                buf.verify(e, s)
            gpu_done.set()

        reader[1] = threading.Thread(target=gpu)
        reader[1].start()
        L.moe_p1_start_prefetch(h, 1, _i32([10, 11, 12]), 3, 3)
        L.moe_p1_wait_layer_all(h, 1)
        assert gpu_done.is_set()
        assert _stats(L, h, 1)["pin_waits"] >= 1
        e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
        L.moe_p1_get_lru_state(h, 1, e, s, ctypes.byref(n))
        for i in range(n.value):
            buf.verify(e[i], s[i])
    finally:
        L.moe_p1_set_wait_reader_callback(h, None, None)
        L.moe_p1_destroy(h)


def test_high_concurrency_stress(scen_file):
    """test_io_sched.cpp:257-442: 8 reader threads, 4 layers of 12 slots, top-4 steps and top-6 /
    cap-3 prefetches of the next layer, resize to 8 at step 100 and to 14 at step 160, forced
    invalidation of 30% every third step; a concurrent reader checks every step's slots."""
    fd, offs = scen_file
    L = _lib()
    h = L.moe_p1_create()
    L.moe_p1_init(h, 8)
    assert L.moe_p1_num_threads(h) == 8
    layers = [1, 2, 3, 4]
    bufs = {l: Bufs(l, 12) for l in layers}
    readers: dict[int, threading.Thread] = {}
    errors = []
    lock = threading.Lock()

    def wait_gpu(l):
        with lock:
            t = readers.pop(l, None)
        if t is not None:
            t.join()
        L.moe_p1_unpin_layer_slots(h, l)

    @ctypes.CFUNCTYPE(None, ctypes.c_int, ctypes.c_void_p)
    def cb(l, _u):
        wait_gpu(l)

    rng = random.Random(123456789)
    mt = L.moe_p1_mt64_create(123456789)
    draw = ctypes.cast(L.moe_p1_mt64_uniform, ctypes.c_void_p)
    checks = 0
    try:
        for l in layers:
            _init_layer(L, h, fd, offs, l, bufs[l], list(range(12)))
        L.moe_p1_set_wait_reader_callback(h, ctypes.cast(cb, ctypes.c_void_p), None)
        for step in range(250):
            if step in (100, 160):
                new_cap = 8 if step == 100 else 14
                for l in layers:
                    wait_gpu(l)
                    L.moe_p1_wait_layer_all(h, l)
                    e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
                    L.moe_p1_get_lru_state(h, l, e, s, ctypes.byref(n))
                    keep = min(n.value, new_cap)
                    kept = [e[i] for i in range(n.value - keep, n.value)]
                    old = [s[i] for i in range(n.value - keep, n.value)]
                    nb = Bufs(l, new_cap)
                    for i, os_ in enumerate(old):
                        for t in range(NT):
                            nb.t[t][i] = bufs[l].t[t][os_]
                    bufs[l] = nb
                    L.moe_p1_resize_layer(h, l, new_cap, nb.ptrs(), nb.slot_inds.ctypes.data, _i32(kept),
                                          _i32(list(range(keep))), keep)
            for l in layers:
                eids = rng.sample(range(N_EXP), 4)
                pred = rng.sample(range(N_EXP), 6)
                wait_gpu(l)
                if step % 3 == 1:
                    L.moe_p1_force_invalidate(h, l, 0.30, draw, mt)
                out = (ctypes.c_uint32 * 4)()
                n = L.moe_p1_step_decode(h, l, _u32(eids), 4, out)
                assert n >= 0, _lib_error()
                if n > 0:
                    L.moe_p1_wait_layer_urgent(h, l)
                slots = list(out)
                b = bufs[l]

                def gpu(b=b, eids=eids, slots=slots):
                    try:
                        for e, s in zip(eids, slots):
                            b.verify(e, s)
                    except AssertionError as ex:
                        errors.append(str(ex))

                t = threading.Thread(target=gpu)
                with lock:
                    readers[l] = t
                t.start()
                checks += 4
                if l + 1 in bufs:
                    L.moe_p1_start_prefetch(h, l + 1, _i32(pred), 6, 3)
        for l in layers:
            wait_gpu(l)
        L.moe_p1_wait_all(h)
        assert not errors, errors[:3]
        tot = (ctypes.c_uint64 * 16)()
        L.moe_p1_get_total_stats(h, 5, tot)
        t = dict(zip(op1.STAT_KEYS, [int(v) for v in tot]))
        assert t["decode_requests"] == 250 * 4 * 4
        assert t["urgent_reads"] > 0 and t["prefetch_issued"] > 0 and t["forced_invalidations"] > 0
        assert t["prefetch_cancelled"] + t["prefetch_wasted"] + t["prefetch_used"] == t["prefetch_issued"]
        assert t["bytes"] > 0
        assert checks == 4000
    finally:
        L.moe_p1_set_wait_reader_callback(h, None, None)
        L.moe_p1_destroy(h)
        L.moe_p1_mt64_destroy(mt)


def _lib_error():
    from moe_offload import _lib as lm
    return lm.last_error()


def test_rejects_bad_ids_and_reports_unfreeable_pins(scen_file):
    fd, offs = scen_file
    L = _lib()
    h = L.moe_p1_create()
    L.moe_p1_init(h, 0)
    try:
        buf = Bufs(2, 4)
        _init_layer(L, h, fd, offs, 2, buf, [0, 1, 2, 3])
        L.c_clear_error()
        assert L.moe_p1_step_decode(h, 2, _u32([1, 600]), 2, None) == -1
        assert "out of range" in _lib_error()
        L.c_clear_error()
        L.moe_p1_pin_slots(h, 2, _u32([0, 1, 2, 3]), 4)          # every slot held by an explicit pin
        assert L.moe_p1_step_decode(h, 2, _u32([9]), 1, None) == -1
        assert "pinned" in _lib_error()
        L.c_clear_error()
        L.moe_p1_unpin_slots(h, 2, _u32([0, 1, 2, 3]), 4)
        assert L.moe_p1_step_decode(h, 2, _u32([9]), 1, None) == 1
        L.moe_p1_wait_layer_urgent(h, 2)
        assert _lib_error() == ""
    finally:
        L.moe_p1_destroy(h)


def test_cpp_class_binds_like_the_reference_class(tmp_path):
    """include/moe_io_sched.hpp compiled into a C++ program (as the runner includes io_sched.h):
    the cancel/promote scenario and a forced invalidation driven by a std::mt19937_64 give what
    the oracle gives, and the generator advances by exactly the draws the oracle made."""
    import shutil
    import subprocess
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("no g++")
    root = HERE.parent
    libdir = root / "moe-offload_amd" / "moe_offload"
    exe = tmp_path / "p1_class_test"
    subprocess.run([cxx, "-std=c++17", "-O1", "-I", str(root / "include"), str(HERE / "cpp" / "p1_class_test.cpp"),
                    "-L", str(libdir), "-lmoe_offload", f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    res = subprocess.run([str(exe), str(tmp_path / "experts.bin")], check=True, capture_output=True, text=True)
    got = json.loads(res.stdout.strip().splitlines()[-1])
    P = op1.P1()
    P.reader_cb = P.unpin_layer_slots
    P.layer_init(1, 4, ROW)
    P.load_sync(1, [0, 1, 2, 3], [0, 1, 2, 3], True)
    P.set_lru_state(1, [0, 1, 2, 3], [0, 1, 2, 3], 4, 0, 4)
    P.unpin_layer_slots(1)
    P.start_prefetch(1, [10, 11, 12], 3)
    pending, slots = P.step_decode(1, [0, 10, 20, 21])
    P.wait_layer_urgent(1)
    st = P.get_layer_stats(1)
    P.unpin_layer_slots(1)
    g = op1.MT64(7)
    inv = P.force_invalidate(1, 0.5, g.uniform)
    eids, sl = P.get_lru_state(1)
    assert got["bytes_ok"] and got["threads"] == 0
    assert (got["pending"], got["slots"]) == (pending, slots)
    assert (got["issued"], got["cancelled"], got["promoted"], got["used"], got["urgent"]) == \
        (st["prefetch_issued"], st["prefetch_cancelled"], st["prefetch_promoted"], st["prefetch_used"],
         st["urgent_reads"]) == (3, 2, 1, 1, 2)
    assert got["invalidated"] == inv
    assert got["lru"] == [[e, s] for e, s in zip(eids, sl)]
    assert got["next_draw"] == g()
