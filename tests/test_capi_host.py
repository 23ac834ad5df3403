"""The C-ABI library without a GPU: it loads, exports every declared symbol, and its host slot
table (the expert_io.c entry points on accounting-only layers) reproduces the golden traces
written by the reference's own expert_io.c."""
import ctypes
import re

import numpy as np
import pytest

from conftest import ROOT
from moe_offload import _lib
from sched_replay import TokenMixin, load, replay

HEADER = ROOT / "include" / "moe_offload.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:c|moe)_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    names = declared_symbols()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing
    # the ctypes table covers exactly the header
    assert sorted(_lib.SIGNATURES) == names


def test_q2_blob_bytes_match_layout():
    from moe_offload import q2format
    L = _lib.lib()
    for h, i in [(2048, 512), (256, 128), (2560, 640)]:
        assert L.moe_q2_expert_bytes(h, i, 64) == q2format.expert_bytes(h, i)
    assert q2format.expert_bytes(2048, 512) == 983_040
    assert q2format.expert_bytes(2560, 640) == 1_228_800 + 307_200  # codes + fp16 scale/bias


class CLayer:
    """One accounting-only layer of the product library (no copies: null stores/pools)."""

    def __init__(self, layer, cap, expert_bytes=1_536_000):
        self.L, self.layer, self.cap = _lib.lib(), layer, cap
        self.slot_buf = (ctypes.c_uint32 * 16)()
        z = (ctypes.c_uint64 * 9)()
        rb = (ctypes.c_uint64 * 9)(expert_bytes, *([0] * 8))
        self.L.c_layer_init(layer, -1, cap, z, rb, z, ctypes.addressof(self.slot_buf))
        _lib.check_error("c_layer_init")

    def step(self, ids):
        a = (ctypes.c_uint32 * len(ids))(*ids)
        n = self.L.c_layer_step_decode_ex(self.layer, a, len(ids), 1)
        _lib.check(n, "step")
        return list(self.slot_buf[:len(ids)]), n

    def prefetch(self, preds, cap):
        if len(preds) == 12:
            self.L.c_layer_start_prefetch12(self.layer, cap, *preds)
        else:
            a = (ctypes.c_int32 * max(1, len(preds)))(*preds)
            self.L.c_layer_start_prefetch(self.layer, a, len(preds), cap)
        _lib.check_error("prefetch")

    def state(self):
        e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int()
        self.L.c_layer_get_lru_state(self.layer, e, s, ctypes.byref(c))
        return [list(e[:c.value]), list(s[:c.value])]

    def set_state(self, e, s, r, h, m):
        n = len(e)
        self.L.c_layer_set_lru_state(self.layer, (ctypes.c_int32 * max(n, 1))(*e), (ctypes.c_int32 * max(n, 1))(*s),
                                     n, r, h, m)
        _lib.check_error("set_state")

    def load_sync(self, e, s):
        n = len(e)
        self.L.c_layer_load_sync(self.layer, (ctypes.c_int32 * n)(*e), (ctypes.c_int32 * n)(*s), n, 1)
        _lib.check_error("load_sync")

    def stats(self):
        o = (ctypes.c_uint64 * 18)()
        self.L.c_layer_get_stats(self.layer, o)
        return list(o)


def test_host_table_reproduces_reference_layer_traces(lru_traces):
    for scen in lru_traces["scenarios"]:
        L = CLayer(40, scen["capacity"])
        for op in scen["ops"]:
            if op["op"] == "prefetch":
                L.prefetch(op["preds"], op["cap"])
            elif op["op"] == "step":
                slots, n = L.step(op["ids"])
                assert slots == op["slots"] and n == op["n_miss"], scen["name"]
            elif op["op"] == "set_state":
                L.set_state(op["eids"], op["slots"], *op["add"])
            elif op["op"] == "load_sync":
                L.load_sync(op["eids"], op["slots"])
            assert L.stats() == op["stats"], (scen["name"], op["op"])
            if "state" in op:
                assert L.state() == op["state"]
        assert L.state() == scen["final_state"]


def test_host_table_reproduces_reference_stack_traces(lru_traces):
    lib = _lib.lib()
    for stk in lru_traces["stacks"]:
        n_layers = stk["n_layers"]
        layers = {int(l): CLayer(int(l), c) for l, c in stk["capacities"].items()}
        for op in stk["ops"]:
            L = layers[op["layer"]]
            if op["op"] == "prefetch":
                L.prefetch(op["preds"], op["cap"])
            else:
                slots, n = L.step(op["ids"])
                assert slots == op["slots"] and n == op["n_miss"]
        for l, st in stk["layer_stats"].items():
            assert layers[int(l)].stats() == st
        out = (ctypes.c_uint64 * 6)()
        lib.c_get_decode_totals(n_layers, out)
        assert list(out) == stk["totals"]
        for l in layers:
            lib.c_layer_reset_stats(l)


def test_out_of_range_layer_is_ignored_and_bad_input_reported():
    lib = _lib.lib()
    out = (ctypes.c_uint64 * 18)(*range(18))
    lib.c_layer_get_stats(99, out)            # silently ignored, as in the reference
    assert list(out) == list(range(18))
    assert lib.c_layer_step_decode10(-1, *range(10)) == 0
    L = CLayer(41, 16)
    a = (ctypes.c_uint32 * 10)(*([600] + list(range(9))))
    assert lib.c_layer_step_decode_ex(41, a, 10, 1) == -1
    with pytest.raises(_lib.NativeError, match="out of range"):
        _lib.check_error("x")
    b = (ctypes.c_uint32 * 17)(*range(17))
    assert lib.c_layer_step_decode_ex(41, b, 17, 1) == -1     # k > 16
    lib.c_clear_error()
    assert L.stats()[0] == 0                                    # rejected calls changed nothing


def test_stamp_renormalisation_keeps_order():
    """Long runs relabel recency stamps; the decisions must not change.  Drive one layer with
    many steps against the oracle's linked-list restatement (cheap proxy for clock wrap)."""
    from oracle import lru as olru
    rng = np.random.default_rng(9)
    L = CLayer(42, 20)
    O = olru.CLru(42, 20)
    for t in range(3000):
        if t % 3 == 0:
            preds = rng.choice(80, size=12, replace=False).tolist()
            L.prefetch(preds, 3)
            O.prefetch(preds, 3)
        ids = rng.choice(80, size=10, replace=False).tolist()
        s1, n1 = L.step(ids)
        s2, m2 = O.step(ids)
        assert s1 == s2 and n1 == len(m2)
    assert L.state() == [list(v) for v in O.get_state()]
    assert L.stats()[:16] == O.stats()[:16]


class ProductSched(TokenMixin):
    """The product library's expert-cache ABI (host tables, accounting-only layers) in the shape
    the scheduler replay expects (tests/sched_replay.py)."""

    def __init__(self):
        super().__init__()
        self.L = _lib.lib()
        self.layers = {}

    def init(self, l, cap):
        self.layers[l] = CLayer(l, cap)

    def reset_stats(self, l):
        self.L.c_layer_reset_stats(l)

    def reset_cache(self, l):
        self.L.c_layer_reset_cache(l)

    def accounting(self, on):
        self.L.c_set_io_accounting(1 if on else 0)

    def begin(self):
        self.L.c_begin_decode_token(0)

    def end(self):
        o = (ctypes.c_uint64 * 10)()
        self.L.c_end_decode_token(o)
        return list(o)

    def sched(self, l, ids, preds, nxt, cap, flags):
        k = len(ids) if ids is not None else 0
        ia = (ctypes.c_int32 * max(k, 1))(*(ids or []))
        npred = len(preds) if preds is not None else 0
        pa = (ctypes.c_int32 * max(npred, 1))(*(preds or []))
        n = self.L.c_layer_decode_step_sched(l, ia if ids is not None else None, k,
                                             pa if preds is not None else None, npred, nxt, cap, flags)
        _lib.check(n, "decode_step_sched")
        self.L.c_layer_wait_demand(l)
        slots = list(self.layers[l].slot_buf[:min(k, 16)]) if (l in self.layers and ids is not None) else []
        return n, slots

    def step(self, l, ids):
        slots, n = self.layers[l].step(ids)
        return n, slots

    def prefetch(self, l, preds, cap):
        self.layers[l].prefetch(preds, cap)

    def stats(self, l):
        return self.layers[l].stats()

    def state(self, l):
        return self.layers[l].state()

    def set_state(self, l, e, s, add):
        self.layers[l].set_state(e, s, *add)

    def split(self, l):
        h = (ctypes.c_uint32 * 16)(*([0xFFFFFFFF] * 16))
        m = (ctypes.c_uint32 * 16)(*([0xFFFFFFFF] * 16))
        inv = (ctypes.c_int32 * 16)(*([-7] * 16))
        self.L.c_layer_get_split_inds(l, h, m, inv)
        return [[v for v in h if v != 0xFFFFFFFF], [v for v in m if v != 0xFFFFFFFF], [v for v in inv if v != -7]]

    def totals(self, n_layers):
        o = (ctypes.c_uint64 * 6)()
        self.L.c_get_decode_totals(n_layers, o)
        return list(o)


def test_host_scheduler_entry_point_reproduces_reference_traces():
    """c_layer_decode_step_sched / c_layer_get_split_inds / per-token accounting of the product
    against the traces of the reference's cpp/third_party/expert_io.c."""
    for sc in load()["scenarios"]:
        assert replay(sc, ProductSched()) > 50, sc["name"]
    assert _lib.last_error() == ""


def test_scheduler_entry_point_input_rules():
    lib = _lib.lib()
    L = CLayer(43, 16)
    ids = (ctypes.c_int32 * 10)(*range(10))
    # layer 0 (resident) is never stepped: only the prefetch of next_layer happens
    assert lib.c_layer_decode_step_sched(0, ids, 10, ids, 10, 43, 3, 0) == 0
    assert L.stats()[0] == 0 and L.stats()[5] == 3 * 1_536_000
    # prefetch_cap 0 prefetches nothing (the published entry point would take 32)
    before = L.stats()
    assert lib.c_layer_decode_step_sched(0, None, 0, ids, 10, 43, 0, 0) == 0
    assert L.stats() == before
    # a repeated id is rejected and changes nothing
    bad = (ctypes.c_int32 * 10)(*([1] + list(range(1, 10))))
    assert lib.c_layer_decode_step_sched(43, bad, 10, None, 0, -1, 0, 0) == -1
    lib.c_clear_error()
    assert L.stats() == before
    # k > 16 is cut to 16, as in the reference
    many = (ctypes.c_int32 * 20)(*range(100, 120))
    assert lib.c_layer_decode_step_sched(43, many, 20, None, 0, -1, 0, 0) == 16
    assert L.stats()[0] == 16


def test_set_format9_validates_roles_and_sizes():
    """c_layer_set_format9 accepts the reference's 9 tensors in any order given their roles, and
    rejects a missing / repeated role or a tensor whose bytes per expert do not fit its role (host
    logic only: the pool addresses are never dereferenced)."""
    from moe_offload import _lib
    L = _lib.lib()
    H, I = 2560, 640
    size = {0: I * H // 4, 1: I * H // 64 * 2, 2: I * H // 64 * 2}         # per projection: w, s, b
    order = [6, 0, 3, 7, 8, 1, 2, 4, 5]
    rb = [size[r % 3] for r in order]
    u64 = ctypes.c_uint64 * 9
    layer = 60
    L.c_layer_init(layer, -1, 16, u64(*[0] * 9), u64(*rb), u64(*[0x10000 * (t + 1) for t in range(9)]), 0)
    L.c_clear_error()
    try:
        assert L.c_layer_set_format9(layer, H, I, 64, (ctypes.c_int32 * 9)(*order), 1) == 0
        bad = list(order)
        bad[1] = bad[0]                                                  # a role named twice
        assert L.c_layer_set_format9(layer, H, I, 64, (ctypes.c_int32 * 9)(*bad), 1) == -1
        assert "each of the 9 tensors once" in _lib.last_error()
        L.c_clear_error()
        swapped = list(order)
        swapped[0], swapped[5] = swapped[5], swapped[0]                  # a weight where a scale belongs
        assert L.c_layer_set_format9(layer, H, I, 64, (ctypes.c_int32 * 9)(*swapped), 1) == -1
        assert "bytes per expert" in _lib.last_error()
        L.c_clear_error()
        assert L.c_layer_set_format9(layer, H, 600, 64, (ctypes.c_int32 * 9)(*order), 1) == -1   # not 64k
        L.c_clear_error()
    finally:
        L.c_layer_init(layer, -1, 16, None, None, None, 0)
        L.c_clear_error()


# ---- the ctypes table against the header, argument by argument --------------------------------

_FN_PTRS = {"moe_p1_reader_fn", "moe_p1_uniform_fn"}
_C_KINDS = {"void": None, "float": "f32", "double": "f64", "int": "i32", "unsigned": "i32", "uint32_t": "i32",
            "int32_t": "i32", "uint64_t": "i64", "int64_t": "i64", "size_t": "i64", "uint16_t": "i16"}


def _c_kind(decl):
    """Kind of one C parameter or return type: 'ptr', 'f32', 'f64', 'i16', 'i32', 'i64' or None (void)."""
    decl = decl.strip()
    words = decl.replace("*", " * ").replace("[", " [ ").split()
    if "*" in words or "[" in words or any(w in _FN_PTRS for w in words):
        return "ptr"
    words = [w for w in words if w not in ("const", "struct")]
    return _C_KINDS[words[0]]


def _py_kind(t):
    if t is None:
        return None
    if t in (ctypes.c_void_p, ctypes.c_char_p) or issubclass(t, (ctypes._Pointer, ctypes._CFuncPtr)):
        return "ptr"
    if t in (ctypes.c_float, ctypes.c_double):
        return "f32" if t is ctypes.c_float else "f64"
    return {2: "i16", 4: "i32", 8: "i64"}[ctypes.sizeof(t)]


def header_declarations():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    out = {}
    for m in re.finditer(r"([A-Za-z_][A-Za-z0-9_ *]*?)\s*\b((?:c|moe)_[a-z0-9_]+)\s*\(([^;{()]*)\)\s*;", text):
        ret, name, params = m.group(1), m.group(2), m.group(3).strip()
        plist = [] if params in ("", "void") else [p for p in params.split(",")]
        out[name] = (_c_kind(ret), [_c_kind(p) for p in plist])
    return out


def test_ctypes_signatures_match_the_header():
    """Every entry point's ctypes restype and argtypes have the header's count and kinds (pointer,
    16/32/64-bit integer, float, double): a mismatch would pass wrong values without an error."""
    decls = header_declarations()
    assert sorted(decls) == declared_symbols()
    bad = []
    for name, (ret, args) in decls.items():
        pret, pargs = _lib.SIGNATURES[name]
        got = (_py_kind(pret), [_py_kind(a) for a in pargs])
        if got != (ret, args):
            bad.append((name, (ret, args), got))
    assert not bad, bad


def test_stack_descriptor_layout_matches_the_header():
    """moe_stack_desc: the ctypes structure has the header's fields in order with the same kinds."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    body = re.search(r"typedef struct moe_stack_desc\s*\{(.*?)\}\s*moe_stack_desc\s*;", text, flags=re.S).group(1)
    fields = []
    for line in body.split(";"):
        line = re.sub(r"//[^\n]*", "", line).strip()
        if not line:
            continue
        # "int a, b, c" declares several fields of one type
        m = re.match(r"((?:const\s+)?[A-Za-z_0-9]+\s*\**)\s*(.*)", line)
        typ, rest = m.group(1), m.group(2)
        for nm in rest.split(","):
            nm = nm.strip()
            stars = nm.count("*")
            fields.append((nm.lstrip("*").strip(), _c_kind(typ + "*" * stars)))
    got = [(n, _py_kind(t)) for n, t in _lib.StackDesc._fields_]
    assert got == fields
