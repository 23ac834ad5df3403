"""Restatement of the reference's P1 I/O scheduler -- test infrastructure only.

Follows `mlx-qwen38/cpp/src/io_sched.cpp` (class `P1IoScheduler`, declared in `io_sched.h:46-245`)
in its deterministic form: no reader threads, so a queued read runs only when a caller that has to
wait executes it (as the reference's waits do with `pop_next_task_locked` + `execute_task`,
io_sched.cpp:787-815,827-848,414-423).  A wait that would block with nothing left to run raises
`Deadlock` (the reference would sleep on its condition variable forever there).

Every method cites the lines it restates.  Slot contents are modelled, not read: `content[t][s]` is
the expert whose tensor-t bytes slot s holds (`SCRUB` after force_invalidate's 64-byte scrub of
tensor 0, None if never written), so tests can check the bytes a product wrote.

Pinned by the golden traces that the reference's own io_sched.cpp, compiled from source, writes
(tests/golden/make_p1_traces.py -> tests/golden/p1_traces.json) and by the reference's own test
scenarios (cpp/tests/test_io_sched.cpp:150-200: cancel / promote counts).
"""
from __future__ import annotations

from collections import deque

NUM_EXPERTS = 512
MAX_LAYERS = 64
MAX_TENSORS = 9
DEFAULT_EXPERT_BYTES = 1_536_000          # io_sched.h:21
LARGE_ROW = 100_000                       # io_sched.cpp:443-447: weights before scales/biases
MAX_RUN = 16                              # io_sched.cpp:481: at most 16 experts per coalesced read
SCRUB = "scrub"

STAT_KEYS = ["decode_requests", "lru_hits", "urgent_reads", "prefetch_issued", "prefetch_cancelled",
             "prefetch_promoted", "prefetch_used", "prefetch_wasted", "pin_waits", "bytes", "io_wait_ns",
             "forced_invalidations", "prefill_requests", "prefill_lru_hits", "prefill_demand_misses",
             "prefill_demand_bytes"]


class Deadlock(RuntimeError):
    pass


class Op:
    """One expert read (io_sched.h:168-181)."""
    __slots__ = ("layer", "eid", "slot", "prev_eid", "is_prefetch", "promoted", "cancelled", "resolved",
                 "started", "completed", "total", "done")

    def __init__(self, layer, eid, slot, prev_eid, is_prefetch, total):
        self.layer, self.eid, self.slot, self.prev_eid = layer, eid, slot, prev_eid
        self.is_prefetch, self.total = is_prefetch, total
        self.promoted = self.cancelled = self.resolved = self.done = False
        self.started = self.completed = 0


class Task:
    """One read: `len(ops)` consecutive experts of tensor t (io_sched.h:183-191)."""
    __slots__ = ("layer", "tensor", "ops", "row_bytes", "is_prefill")

    def __init__(self, layer, tensor, ops, row_bytes):
        self.layer, self.tensor, self.ops, self.row_bytes, self.is_prefill = layer, tensor, ops, row_bytes, False


class Layer:
    def __init__(self):
        self.initialized = False
        self.capacity = 0
        self.row_bytes = []
        self.expert_bytes = DEFAULT_EXPERT_BYTES
        self.eid_to_slot = [-1] * NUM_EXPERTS
        self.slot_to_eid = [-1] * NUM_EXPERTS
        self.order = []                       # slots, LRU first (the reference's linked list)
        self.free = []                        # stack: pop() gives the next free slot
        self.pin = [0] * NUM_EXPERTS
        self.gpu_pinned = []
        self.active = [None] * NUM_EXPERTS
        self.has_snapshot = False
        self.snapshot = set()
        self.last_prefetch = []
        self.pending = []
        self.stats = dict.fromkeys(STAT_KEYS, 0)
        self.content = []


class P1:
    def __init__(self):
        self.layers = [Layer() for _ in range(MAX_LAYERS)]
        self.urgent = deque()
        self.prefetchq = deque()
        self.reader_cb = None                 # called with the layer when an allocation meets a pin

    # -- list helpers (io_sched.cpp:53-107) ------------------------------------------------------
    @staticmethod
    def _remove(L, slot):
        L.order.remove(slot)

    @staticmethod
    def _append_mru(L, slot):
        L.order.append(slot)

    @staticmethod
    def _prepend_lru(L, eid, slot):
        L.eid_to_slot[eid], L.slot_to_eid[slot] = slot, eid
        L.order.insert(0, slot)

    @staticmethod
    def _move_mru(L, slot):
        L.order.remove(slot)
        L.order.append(slot)

    def _insert(self, L, eid, slot):
        if L.eid_to_slot[eid] >= 0:
            self._move_mru(L, L.eid_to_slot[eid])
            return
        L.eid_to_slot[eid], L.slot_to_eid[slot] = slot, eid
        L.order.append(slot)

    def _evict(self, L, slot):
        eid = L.slot_to_eid[slot]
        self._remove(L, slot)
        if eid >= 0:
            L.eid_to_slot[eid] = -1
        L.slot_to_eid[slot] = -1
        L.active[slot] = None
        return eid

    def _clear_table(self, L, pins=True):
        L.eid_to_slot = [-1] * NUM_EXPERTS
        L.slot_to_eid = [-1] * NUM_EXPERTS
        L.order = []
        L.active = [None] * NUM_EXPERTS
        if pins:
            L.pin = [0] * NUM_EXPERTS
            L.gpu_pinned = []

    # -- setup (io_sched.cpp:109-271) -----------------------------------------------------------------
    def layer_init(self, layer, capacity, row_bytes):
        if not 0 <= layer < MAX_LAYERS:
            return
        self.wait_layer_all(layer)
        L = self.layers[layer]
        L.initialized = True
        L.capacity = min(max(capacity, 1), NUM_EXPERTS)
        L.row_bytes = list(row_bytes[:min(max(len(row_bytes), 1), MAX_TENSORS)])
        s = sum(L.row_bytes)
        L.expert_bytes = s if s > 0 else DEFAULT_EXPERT_BYTES
        self._clear_table(L)
        L.free = list(range(L.capacity - 1, -1, -1))
        L.has_snapshot, L.snapshot = False, set()
        L.last_prefetch, L.pending = [], []
        L.stats = dict.fromkeys(STAT_KEYS, 0)
        L.content = [[None] * L.capacity for _ in L.row_bytes]

    def _rebuild(self, L, eids, slots):
        used = set()
        for e, s in zip(eids, slots):
            if 0 <= s < L.capacity and 0 <= e < NUM_EXPERTS:
                used.add(s)
                self._insert(L, e, s)
        L.free = [s for s in range(L.capacity - 1, -1, -1) if s not in used]

    def resize_layer(self, layer, new_capacity, eids, slots, content=None):
        """io_sched.cpp:157-205.  `content` (per tensor, per new slot) is what the caller copied."""
        if not 0 <= layer < MAX_LAYERS:
            return
        self.wait_layer_all(layer)
        L = self.layers[layer]
        L.capacity = min(max(new_capacity, 1), NUM_EXPERTS)
        self._clear_table(L)
        L.has_snapshot, L.snapshot = False, set()
        L.last_prefetch, L.pending = [], []
        self._rebuild(L, eids, slots)
        L.content = content if content is not None else [[None] * L.capacity for _ in L.row_bytes]

    def reset_cache(self, layer):
        """io_sched.cpp:207-231."""
        if not 0 <= layer < MAX_LAYERS:
            return
        self.wait_layer_all(layer)
        L = self.layers[layer]
        self._clear_table(L)
        L.free = list(range(L.capacity - 1, -1, -1))
        L.has_snapshot, L.snapshot = False, set()
        L.last_prefetch, L.pending = [], []

    def reset_stats(self, layer):
        """io_sched.cpp:233-239."""
        if 0 <= layer < MAX_LAYERS:
            self.layers[layer].stats = dict.fromkeys(STAT_KEYS, 0)

    # -- reads (io_sched.cpp:241-349) -------------------------------------------------------------
    def _pop(self, urgent_only=False):
        while self.urgent:
            t = self.urgent.popleft()
            live = False
            for op in t.ops:
                if not op.cancelled:
                    op.started += 1
                    live = True
            if live:
                return t
        if urgent_only:
            return None
        while self.prefetchq:
            t = self.prefetchq.popleft()
            op = t.ops[0]
            if op.cancelled or op.promoted:
                continue
            op.started += 1
            return t
        return None

    def _execute(self, t):
        L = self.layers[t.layer]
        if not t.is_prefill:
            L.stats["bytes"] += t.row_bytes * len(t.ops)
        for op in t.ops:
            if 0 <= op.slot < len(L.content[t.tensor]):
                L.content[t.tensor][op.slot] = op.eid
            op.completed += 1
            if op.completed >= op.total:
                op.done = True

    def _run_one(self, urgent_only=False):
        t = self._pop(urgent_only)
        if t is None:
            raise Deadlock("nothing left to run")
        self._execute(t)

    # -- slot allocation (io_sched.cpp:367-437) -----------------------------------------------------
    def _alloc(self, layer, protect):
        L = self.layers[layer]
        if L.free:
            return L.free.pop(), -1
        counted = False
        while True:
            saw_pin = saw_io = False
            for s in L.order:
                e = L.slot_to_eid[s]
                prot = e >= 0 and e in protect
                pinned = L.pin[s] > 0
                busy = L.active[s] is not None and not L.active[s].done
                if not prot and not pinned and not busy:
                    return s, self._evict(L, s)
                saw_pin |= (not prot) and pinned
                saw_io |= (not prot) and busy
            if not saw_pin and not saw_io:
                for s in L.order:
                    saw_pin |= L.pin[s] > 0
                    saw_io |= L.active[s] is not None and not L.active[s].done
            if saw_pin:
                if not counted:
                    L.stats["pin_waits"] += 1
                    counted = True
                if self.reader_cb is None:
                    raise Deadlock("pinned slots and no reader callback")
                before = list(L.pin)
                self.reader_cb(layer)
                if L.pin == before:        # the reference would call it again forever
                    raise Deadlock("the reader callback released no pin")
                continue
            if saw_io:
                self._run_one()
                continue
            for s in L.order:
                if L.pin[s] == 0 and (L.active[s] is None or L.active[s].done):
                    return s, self._evict(L, s)

    # -- queueing (io_sched.cpp:439-511) ------------------------------------------------------------
    def _tensor_passes(self, L):
        big = [t for t, rb in enumerate(L.row_bytes) if rb > LARGE_ROW]
        small = [t for t, rb in enumerate(L.row_bytes) if rb <= LARGE_ROW]
        return big + small

    def _enqueue_prefetch(self, layer, L, op):
        for t in self._tensor_passes(L):
            self.prefetchq.append(Task(layer, t, [op], L.row_bytes[t]))

    def _enqueue_urgent(self, layer, L, ops, prefill=False):
        if not ops:
            return
        ops = sorted(ops, key=lambda o: o.eid)
        runs, start = [], 0
        for i in range(1, len(ops)):
            if ops[i].eid != ops[i - 1].eid + 1 or i - start >= MAX_RUN:
                runs.append(ops[start:i])
                start = i
        runs.append(ops[start:])
        for t in self._tensor_passes(L):
            for r in runs:
                task = Task(layer, t, list(r), L.row_bytes[t])
                task.is_prefill = prefill
                self.urgent.append(task)

    def _cancel(self, L, op, mark_snapshot):
        """An unstarted prefetch dropped: its slot goes back to the expert it displaced, or to the
        free stack (io_sched.cpp:530-545, 660-677)."""
        op.cancelled = True
        L.stats["prefetch_cancelled"] += 1
        if L.slot_to_eid[op.slot] == op.eid:
            self._remove(L, op.slot)
            L.eid_to_slot[op.eid] = -1
            L.slot_to_eid[op.slot] = -1
            L.active[op.slot] = None
            if 0 <= op.prev_eid < NUM_EXPERTS and L.eid_to_slot[op.prev_eid] < 0:
                self._prepend_lru(L, op.prev_eid, op.slot)
                if mark_snapshot:
                    L.snapshot.add(op.prev_eid)
            else:
                L.free.append(op.slot)

    # -- decode API (io_sched.cpp:513-773) -----------------------------------------------------------
    def start_prefetch(self, layer, preds, max_fetch):
        if not 0 <= layer < MAX_LAYERS or not preds or max_fetch <= 0:
            return
        L = self.layers[layer]
        if not L.initialized:
            return
        for op in L.last_prefetch:
            if op.resolved:
                continue
            op.resolved = True
            if op.started == 0:
                self._cancel(L, op, mark_snapshot=False)
            else:
                L.stats["prefetch_wasted"] += 1
        L.last_prefetch = []
        L.snapshot = {e for e in range(NUM_EXPERTS) if L.eid_to_slot[e] >= 0}
        L.has_snapshot = True
        protect, missing = set(), []
        cap = min(max_fetch, 32)
        for e in preds:
            if not 0 <= e < NUM_EXPERTS:
                continue
            seen = e in protect
            protect.add(e)
            if not seen and L.eid_to_slot[e] < 0 and len(missing) < cap:
                missing.append(e)
        for e in reversed(missing):
            if L.eid_to_slot[e] >= 0:
                continue
            slot, prev = self._alloc(layer, protect)
            self._insert(L, e, slot)
            op = Op(layer, e, slot, prev, True, len(L.row_bytes))
            L.active[slot] = op
            L.last_prefetch.append(op)
            L.stats["prefetch_issued"] += 1
            self._enqueue_prefetch(layer, L, op)

    def step_decode(self, layer, eids):
        """Returns (pending, slots) (io_sched.cpp:614-773)."""
        k = len(eids)
        if not 0 <= layer < MAX_LAYERS or k <= 0:
            return 0, []
        L = self.layers[layer]
        if not L.initialized:
            return 0, []
        L.stats["decode_requests"] += k
        actual = {e for e in eids if 0 <= e < NUM_EXPERTS}
        urgent_ops = []
        if L.last_prefetch:
            for op in L.last_prefetch:
                if op.resolved or op.eid in actual:
                    continue
                op.resolved = True
                if op.started == 0:
                    self._cancel(L, op, mark_snapshot=True)
                else:
                    L.stats["prefetch_wasted"] += 1
            for op in L.last_prefetch:
                if op.resolved or op.eid not in actual:
                    continue
                op.resolved = True
                L.stats["prefetch_used"] += 1
                if op.started == 0:
                    op.promoted = True
                    op.is_prefetch = False
                    L.stats["prefetch_promoted"] += 1
                    urgent_ops.append(op)
                elif not op.done:
                    keep = deque()
                    for t in self.prefetchq:
                        if t.ops[0] is op:
                            self.urgent.append(t)
                        else:
                            keep.append(t)
                    self.prefetchq = keep
            L.last_prefetch = []
        self.prefetchq = deque(t for t in self.prefetchq if not (t.ops[0].cancelled or t.ops[0].promoted))
        for e in eids:
            if not 0 <= e < NUM_EXPERTS:
                continue
            if L.eid_to_slot[e] >= 0:
                if not L.has_snapshot or e in L.snapshot:
                    L.stats["lru_hits"] += 1
            else:
                L.stats["urgent_reads"] += 1
                slot, prev = self._alloc(layer, actual)
                self._insert(L, e, slot)
                op = Op(layer, e, slot, prev, False, len(L.row_bytes))
                L.active[slot] = op
                urgent_ops.append(op)
        L.has_snapshot = False
        self._enqueue_urgent(layer, L, urgent_ops)
        L.pending = []
        slots = []
        for e in eids:
            s = L.eid_to_slot[e]
            self._move_mru(L, s)
            slots.append(s)
            L.pin[s] += 1
            L.gpu_pinned.append(s)
            if L.active[s] is not None and not L.active[s].done:
                L.pending.append(L.active[s])
        return len(L.pending), slots

    def wait_layer_urgent(self, layer):
        """io_sched.cpp:775-827 (the waiting caller drains the URGENT queue)."""
        if not 0 <= layer < MAX_LAYERS:
            return
        L = self.layers[layer]
        if not L.pending:
            return
        while not all(op.done for op in L.pending):
            self._run_one(urgent_only=True)
        L.pending = []

    def wait_layer_all(self, layer):
        """io_sched.cpp:829-856."""
        if not 0 <= layer < MAX_LAYERS:
            return
        self.wait_layer_urgent(layer)
        L = self.layers[layer]
        if not L.initialized:
            return
        while any(L.active[s] is not None and not L.active[s].done and not L.active[s].cancelled
                  for s in range(L.capacity)):
            self._run_one()

    def wait_all(self):
        for l in range(MAX_LAYERS):
            self.wait_layer_all(l)

    def unpin_layer_slots(self, layer):
        """io_sched.cpp:864-876."""
        if not 0 <= layer < MAX_LAYERS:
            return
        L = self.layers[layer]
        for s in L.gpu_pinned:
            if 0 <= s < NUM_EXPERTS and L.pin[s] > 0:
                L.pin[s] -= 1
        L.gpu_pinned = []

    def pin_slots(self, layer, slots):
        if 0 <= layer < MAX_LAYERS:
            for s in slots:
                if 0 <= s < NUM_EXPERTS:
                    self.layers[layer].pin[s] += 1

    def unpin_slots(self, layer, slots):
        if 0 <= layer < MAX_LAYERS:
            for s in slots:
                if 0 <= s < NUM_EXPERTS and self.layers[layer].pin[s] > 0:
                    self.layers[layer].pin[s] -= 1

    def get_slot_pin_count(self, layer, slot):
        if not (0 <= layer < MAX_LAYERS and 0 <= slot < NUM_EXPERTS):
            return 0
        return self.layers[layer].pin[slot]

    def force_invalidate(self, layer, rate, uniform01):
        """io_sched.cpp:907-982; `uniform01()` draws one std::uniform_real_distribution<double>(0, 1)
        value from the caller's generator."""
        if not 0 <= layer < MAX_LAYERS or rate <= 0.0:
            return 0
        L = self.layers[layer]
        if not L.initialized:
            return 0
        chosen = []
        for s in list(L.order):
            if L.pin[s] > 0 or L.slot_to_eid[s] < 0:
                continue
            if rate >= 1.0 or uniform01() < rate:
                chosen.append(s)
        n = 0
        for s in chosen:
            if L.pin[s] > 0 or L.slot_to_eid[s] < 0:
                continue
            a = L.active[s]
            if a is not None and not a.done and not a.cancelled:
                if a.is_prefetch and a.started == 0:
                    a.resolved = True
                    a.cancelled = True
                    L.stats["prefetch_cancelled"] += 1
                else:
                    while not a.done and not a.cancelled:
                        self._run_one()
            if L.pin[s] > 0:
                continue
            e = L.slot_to_eid[s]
            if e < 0:
                continue
            for op in L.last_prefetch:
                if not op.resolved and op.slot == s:
                    op.resolved = True
                    L.stats["prefetch_wasted"] += 1
            self._remove(L, s)
            L.eid_to_slot[e] = -1
            L.slot_to_eid[s] = -1
            L.active[s] = None
            L.snapshot.discard(e)
            if L.content and L.row_bytes[0] > 0:
                L.content[0][s] = SCRUB
            L.free.append(s)
            n += 1
        L.stats["forced_invalidations"] += n
        return n

    def load_sync(self, layer, eids, slots, is_prefill):
        """io_sched.cpp:984-1027."""
        if not 0 <= layer < MAX_LAYERS or not eids:
            return
        self.wait_layer_all(layer)
        L = self.layers[layer]
        if not L.initialized:
            return
        if is_prefill:
            L.stats["prefill_demand_bytes"] += len(eids) * L.expert_bytes
        ops = []
        for e, s in zip(eids, slots):
            op = Op(layer, e, s, -1, False, len(L.row_bytes))
            L.active[s] = op
            ops.append(op)
        self._enqueue_urgent(layer, L, ops, prefill=is_prefill)
        L.pending = ops
        self.wait_layer_urgent(layer)

    def get_lru_state(self, layer):
        """io_sched.cpp:1029-1049: (eids, slots), LRU first."""
        if not 0 <= layer < MAX_LAYERS:
            return [], []
        self.wait_layer_all(layer)
        L = self.layers[layer]
        return [L.slot_to_eid[s] for s in L.order], list(L.order)

    def set_lru_state(self, layer, eids, slots, add_req=0, add_hits=0, add_miss=0):
        """io_sched.cpp:1051-1094 (pin counts survive)."""
        if not 0 <= layer < MAX_LAYERS:
            return
        self.wait_layer_all(layer)
        L = self.layers[layer]
        L.stats["prefill_requests"] += add_req
        L.stats["prefill_lru_hits"] += add_hits
        L.stats["prefill_demand_misses"] += add_miss
        self._clear_table(L, pins=False)
        L.has_snapshot = False
        L.last_prefetch, L.pending = [], []
        self._rebuild(L, eids, slots)

    def get_layer_stats(self, layer):
        if not 0 <= layer < MAX_LAYERS:
            return dict.fromkeys(STAT_KEYS, 0)
        return dict(self.layers[layer].stats)

    def get_total_stats(self, num_layers=48):
        """io_sched.cpp:1104-1131: layers 1 .. num_layers - 1."""
        tot = dict.fromkeys(STAT_KEYS, 0)
        for l in range(1, min(num_layers, MAX_LAYERS)):
            L = self.layers[l]
            if L.initialized:
                for k in STAT_KEYS:
                    tot[k] += L.stats[k]
        return tot


# -- std::mt19937_64 and std::uniform_real_distribution<double>(0, 1) as libstdc++ computes them --
class MT64:
    """The 64-bit Mersenne Twister of C++11 ([rand.predef]: mt19937_64), for force_invalidate's
    draws; `uniform()` is libstdc++'s generate_canonical<double, 53> over one 64-bit draw."""
    N, M = 312, 156
    MATRIX = 0xB5026F5AA96619E9
    UPPER, LOWER = 0xFFFFFFFF80000000, 0x7FFFFFFF
    MASK = (1 << 64) - 1

    def __init__(self, seed=5489):
        self.mt = [0] * self.N
        self.mt[0] = seed & self.MASK
        for i in range(1, self.N):
            self.mt[i] = (6364136223846793005 * (self.mt[i - 1] ^ (self.mt[i - 1] >> 62)) + i) & self.MASK
        self.idx = self.N

    def _twist(self):
        mt = self.mt
        for i in range(self.N):
            x = (mt[i] & self.UPPER) | (mt[(i + 1) % self.N] & self.LOWER)
            xa = x >> 1
            if x & 1:
                xa ^= self.MATRIX
            mt[i] = mt[(i + self.M) % self.N] ^ xa
        self.idx = 0

    def __call__(self):
        if self.idx >= self.N:
            self._twist()
        x = self.mt[self.idx]
        self.idx += 1
        x ^= (x >> 29) & 0x5555555555555555
        x ^= (x << 17) & 0x71D67FFFEDA60000
        x ^= (x << 37) & 0xFFF7EEE000000000
        x ^= x >> 43
        return x & self.MASK

    def uniform(self):
        r = float(self()) / 18446744073709551616.0
        return r if r < 1.0 else 0.9999999999999999
