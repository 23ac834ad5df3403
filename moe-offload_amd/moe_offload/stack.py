"""Stacked routed-expert decode (the 48-layer workload) on one MI355X.

Each layer l has an fp16 router W_l [E, H], Q2 g64 SwitchGLU experts (inter I) and an fp16
RMSNorm after it (builder-defined glue; the reference mixes hyper-connections there,
`mlx-qwen38/loader.py:61,992`):

    x_0 = token hidden state (fp16)
    ids_l, scores_l      = router(x_l; W_l)                       (loader.py:903-908)
    pred_{l+1}           = top-m(W_{l+1} . x_l)                    (loader.py:950-958)
    h_l                  = x_l + sum_j scores_j SwitchGLU_{ids_j}(x_l)   (fp32)
    x_{l+1}              = RMSNorm_l(h_l)  (fp16, eps 1e-6; fused into the next router)

Layer 0's experts are resident in HBM (the reference pins them, loader.py:1059-1060);
layers 1..L-1 keep `capacity` slots in HBM, fed from a pinned host expert store.  The slot
tables follow the reference's call order per token: prefetch(1) after layer 0, then step(l)
followed by prefetch(l+1) (loader.py:920-977).

Two drivers:
  mode="device"  slot tables live on the GPU; a layer is router -> slot step -> staging kernel
                 -> gate/up -> down with no host round trip; next-layer prefetch (table update +
                 staging) runs on a side stream and joins before the next layer's step.  A whole
                 token can be captured into one HIP graph.
  mode="host"    the reference's shape: one device->host read of the ids per layer, the host
                 slot table (expert_io.c ABI), DMA copies on the library's copy stream.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib, q2format
from .loader import FileExpertStore, HostExpertStore, compute_layer_capacities


@dataclass
class StackConfig:
    n_layers: int = 48
    hidden: int = 2048
    n_exp: int = 512
    top_k: int = 10
    inter: int = 512
    group: int = 64
    budget_pct: float | None = 20.0
    budget_gb: float | None = None
    prefetch: bool = True
    top_m: int = 12
    prefetch_cap: int = 3
    eps: float = 1e-6
    seed: int = 0
    layer_base: int = 0          # first C-ABI layer index used (tables are global to the library)
    stage_ctas: int = 2          # staging blocks per copied expert (enough to fill PCIe; more
                                 # only floods the L2 miss queues with slow host reads)
    pf_stage_ctas: int = 3       # the same for the prefetch copies (0: stage_ctas); they run
                                 # alone on the link more often than the demand copies do
    resident: bool = False       # every layer's experts in HBM (no slot tables, no staging)
    routed_glu: bool = True      # resident: the router writes logits, gate/up selects (no hand-off)
    fused_tables: bool = True    # device mode: the router's last block runs the slot-table step
                                 # and the next layer's prefetch (no separate table launches)
    sched: bool = False          # the C++ runner's scheduler variant (cpp/src/engine.cpp:700-730,
                                 # cpp/third_party/expert_io.c:1094-1394): host mode makes one
                                 # c_layer_decode_step_sched call per layer; device mode tables
                                 # take the variant's decisions
    split: bool = False          # host mode with sched: hit experts run before the misses land
    store_file: str | None = None  # layers 1.. read their misses from this blob file
                                 # (q2format.write_blob_file) instead of a pinned host store;
                                 # device mode: the tables publish their misses to the library's
                                 # feeder thread (c_layer_publish_dev), io="exact", fused tables
    io_threads: int = 8          # reader threads of the file tier
    io_direct: bool = False      # file tier: O_DIRECT reads (page cache bypassed)
    io: str = "exact"            # file tier cache: "exact" (expert_io.c's, c_layer_*) or "p1" (the
                                 # C++ runner's P1 I/O scheduler, moe_p1_*: cancel/promote, pins)
    native_host: bool = False    # host mode: the per-layer loop runs in the library
                                 # (moe_stack_token_host) instead of Python


def effective_fetch_cap(prefetch_cap: int, top_m: int) -> int:
    """Most experts one prefetch call fetches: cap if 0 < cap < 32 else 32
    (expert_io.c:545), bounded by the number of predictions."""
    cap = prefetch_cap if 0 < prefetch_cap < 32 else 32
    return min(cap, top_m)


def random_blobs(n_exp: int, hidden: int, inter: int, group: int, gen: torch.Generator, device,
                 scale_std: float = 0.02) -> torch.Tensor:
    """Synthetic Q2 experts as blobs, generated on the GPU: codes ~ U{0..3} (uniform random
    bytes), scale ~ N(0, scale_std) fp16, bias = -1.5 * scale."""
    o = q2format.blob_offsets(hidden, inter, group)
    blobs = torch.empty((n_exp, o["bytes"]), dtype=torch.uint8, device=device)
    code_bytes = o["gate_sb"]
    blobs[:, :code_bytes] = torch.randint(0, 256, (n_exp, code_bytes), dtype=torch.uint8, device=device,
                                          generator=gen)
    n_pairs = (o["bytes"] - code_bytes) // 4
    s = (torch.randn((n_exp, n_pairs), device=device, generator=gen) * scale_std).half()
    b = (-1.5 * s.float()).half()
    sb = torch.stack([s, b], dim=-1).contiguous().view(torch.uint8).view(n_exp, n_pairs * 4)
    blobs[:, code_bytes:] = sb
    return blobs


class DecodeStack:
    def __init__(self, cfg: StackConfig = StackConfig(), mode: str = "device", device="cuda"):
        assert mode in ("device", "host")
        self.cfg, self.mode = cfg, mode
        self.device = torch.device(device)
        c = cfg
        L = _lib.lib()
        self.L = L
        self.blob_bytes = q2format.expert_bytes(c.hidden, c.inter, c.group)
        caps = compute_layer_capacities(budget_gb=c.budget_gb, budget_pct=c.budget_pct, num_layers=c.n_layers,
                                        num_experts=c.n_exp, expert_bytes=self.blob_bytes)
        self.capacities = caps
        self.file_device = False
        gen = torch.Generator(device=self.device)
        gen.manual_seed(c.seed)
        dev = self.device
        self.router_w = (torch.randn((c.n_layers, c.n_exp, c.hidden), device=dev, generator=gen) * 0.02).half()
        self.norm_w = (1.0 + 0.1 * torch.randn((c.n_layers, c.hidden), device=dev, generator=gen)).half()
        # layer 0: every expert resident
        self.pool0 = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, dev)
        self.pools, self.slot_inds = {}, {}
        if c.resident:
            # all layers resident: pools hold every expert and slot == expert id
            self.store = None
            self.full_pools = [self.pool0] + [random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, dev)
                                              for _ in range(1, c.n_layers)]
            self._init_buffers()
            return
        self.full_pools = None
        self.p1 = None
        self.mirror_ids = True
        if c.io not in ("exact", "p1"):
            raise ValueError(f"io={c.io!r}: 'exact' or 'p1'")
        if c.io == "p1" and c.store_file is None:
            raise ValueError("io='p1' reads from a file: set store_file")
        self.file_device = c.store_file is not None and mode == "device"
        if c.store_file is not None:
            # layers 1..: misses read from a blob file by the reader threads
            if self.file_device and (c.io != "exact" or not c.fused_tables or c.sched):
                raise ValueError("a device-driven file-backed stack takes io='exact', fused tables, no sched")
            L.c_io_init(c.io_threads)
            L.c_io_set_direct(int(c.io_direct))
            L.c_io_clear_fault()                     # the library-wide fault word starts clean
            self.store = FileExpertStore({l: c.store_file for l in range(1, c.n_layers)})
            if self.store.blob_bytes != self.blob_bytes:
                raise ValueError(f"{c.store_file}: blobs of {self.store.blob_bytes} bytes, the stack's are {self.blob_bytes}")
        else:
            # layers 1..: pinned host store
            self.store = HostExpertStore(c.n_layers, c.n_exp, self.blob_bytes, first_layer=1)
        for l in range(1, c.n_layers):
            if c.store_file is None:
                blobs = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, dev)
                self.store.tensor(l).copy_(blobs)
                del blobs
            self.pools[l] = torch.zeros((caps[l], self.blob_bytes), dtype=torch.uint8, device=dev)
            self.slot_inds[l] = torch.zeros(16, dtype=torch.int32, device=dev)
        torch.cuda.synchronize()
        L.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        u64 = ctypes.c_uint64 * 9
        if c.io == "p1":
            self.p1 = L.moe_p1_create()
            L.moe_p1_init(self.p1, c.io_threads)
            L.moe_p1_set_compute_stream(self.p1, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            for l in range(1, c.n_layers):
                L.moe_p1_layer_init(self.p1, self.cidx(l), self.store.fds[l], caps[l], 1,
                                    u64(self.store.headers[l]["data_offset"], *[0] * 8), u64(self.blob_bytes, *[0] * 8),
                                    u64(self.pools[l].data_ptr(), *[0] * 8), self.slot_inds[l].data_ptr())
            _lib.check_error("moe_p1_layer_init")
            self._init_buffers()
            return
        for l in range(1, c.n_layers):
            li = self.cidx(l)
            if c.store_file is not None:
                fd, base = self.store.fds[l], self.store.headers[l]["data_offset"]
            else:
                fd, base = -1, self.store.layer_ptr(l)
            L.c_layer_init(li, fd, caps[l], u64(base, *[0] * 8), u64(self.blob_bytes, *[0] * 8),
                           u64(self.pools[l].data_ptr(), *[0] * 8), self.slot_inds[l].data_ptr())
            _lib.check(L.c_layer_set_format(li, c.hidden, c.inter, c.group), "set_format")
            if mode == "device":
                _lib.check(L.c_layer_set_device_mode(li, 1), "set_device_mode")
            if c.sched:
                _lib.check(L.c_layer_set_sched(li, 1), "set_sched")
        _lib.check_error("c_layer_init")
        self._init_buffers()

    def _init_buffers(self):
        # per-layer outputs / workspaces (fixed addresses, so a token can be graph-captured)
        c, L, dev = self.cfg, self.L, self.device
        k = c.top_k
        self.ids = torch.zeros((c.n_layers, k), dtype=torch.int32, device=dev)
        self.logits = torch.zeros((c.n_layers, c.n_exp), dtype=torch.float32, device=dev)
        self.scores = torch.zeros((c.n_layers, k), dtype=torch.float16, device=dev)
        self.pred = torch.zeros((c.n_layers, max(c.top_m, 1)), dtype=torch.int32, device=dev)
        self.xs = torch.zeros((c.n_layers + 1, c.hidden), dtype=torch.float16, device=dev)
        self.hs = torch.zeros((c.n_layers, c.hidden), dtype=torch.float32, device=dev)
        self.h_ws = torch.zeros((c.top_k * c.inter,), dtype=torch.float16, device=dev)
        self.router_ws = [torch.zeros(int(L.moe_router_workspace_bytes(c.n_exp)), dtype=torch.uint8, device=dev)
                          for _ in range(c.n_layers)]
        self.side = torch.cuda.Stream(device=dev)
        self.ev_pred = [torch.cuda.Event() for _ in range(c.n_layers)]
        self.ev_pref = [torch.cuda.Event() for _ in range(c.n_layers)]
        self.ev_copy = [torch.cuda.Event() for _ in range(c.n_layers)]
        self.ev_demand = [torch.cuda.Event() for _ in range(c.n_layers)]
        self.graph = None
        self._host_sel = []
        self.token_io = False
        self.last_token_io: list[int] | None = None
        if c.native_host and self.mode == "host" and not c.resident and self.p1 is None and not c.sched:
            self._init_native()

    def _init_native(self):
        """Pinned host mirrors for the router's ids / predictions and the runner's descriptor."""
        c, L = self.cfg, self.L
        k, m = c.top_k, max(c.top_m, 1)
        ids_p, pred_p = L.c_host_alloc(c.n_layers * k * 4), L.c_host_alloc(c.n_layers * m * 4)
        if not ids_p or not pred_p:
            raise _lib.NativeError(f"pinned id buffers: {_lib.last_error()}")
        self._host_sel = [ids_p, pred_p]
        self.ids_host = np.ctypeslib.as_array(ctypes.cast(ids_p, ctypes.POINTER(ctypes.c_int32)), shape=(c.n_layers, k))
        self.pred_host = np.ctypeslib.as_array(ctypes.cast(pred_p, ctypes.POINTER(ctypes.c_int32)),
                                               shape=(c.n_layers, m))
        self._ws_flat = torch.zeros(c.n_layers * self.router_ws[0].numel(), dtype=torch.uint8, device=self.device)
        self.desc = _lib.StackDesc(
            n_layers=c.n_layers, layer_base=c.layer_base, hidden=c.hidden, n_exp=c.n_exp, top_k=k, top_m=c.top_m,
            inter=c.inter, group=c.group, prefetch=int(c.prefetch), prefetch_cap=c.prefetch_cap, eps=c.eps,
            xs=self.xs.data_ptr(), hs=self.hs.data_ptr(), router_w=self.router_w.data_ptr(),
            norm_w=self.norm_w.data_ptr(), scores=self.scores.data_ptr(), ids0=self.ids[0].data_ptr(),
            ids_host=ids_p, pred_host=pred_p, router_ws=self._ws_flat.data_ptr(),
            router_ws_bytes=self.router_ws[0].numel(), pool0=self.pool0.data_ptr(), blob_bytes=self.blob_bytes,
            h_ws=self.h_ws.data_ptr())

    # C-ABI layer index of stack layer l
    def cidx(self, l: int) -> int:
        return self.cfg.layer_base + l

    def reset_caches(self):
        if self.cfg.resident:
            return
        if self.p1 is not None:
            for l in range(1, self.cfg.n_layers):
                self.L.moe_p1_unpin_layer_slots(self.p1, self.cidx(l))
                self.L.moe_p1_reset_cache(self.p1, self.cidx(l))
            _lib.check_error("p1 reset_cache")
            return
        for l in range(1, self.cfg.n_layers):
            self.L.c_layer_reset_cache(self.cidx(l))
        if self.file_device:
            torch.cuda.synchronize()                 # no staging kernel of an earlier token still runs
            self.L.c_io_clear_fault()
        _lib.check_error("reset_cache")

    def set_token_accounting(self, on: bool):
        """Per-token I/O accounting (cpp/third_party/expert_io.c:98-111,1002-1038): with it on,
        decode_token opens a token (c_begin_decode_token) before its work and reads the token's 10
        counters (c_end_decode_token: LRU hits, misses, prefetch loads / hits / wasted, demand and
        prefetch reloads within 16 / 64 tokens of the eviction, bytes copied) into last_token_io
        after it, at the cost of one host synchronisation per token.  Device-driven tables count
        on the GPU, host tables in the library, with the same rules.  The library's accounting
        switch and token numbering are process-wide, as the reference's are."""
        if self.cfg.resident or self.p1 is not None:
            raise ValueError("per-token accounting needs the expert_io.c slot tables (not resident, io='exact')")
        self.L.c_set_io_accounting(1 if on else 0)
        _lib.check_error("set_io_accounting")
        self.token_io = bool(on)
        self.last_token_io = None

    def reset_stats(self):
        if self.cfg.resident:
            return
        if self.p1 is not None:
            for l in range(1, self.cfg.n_layers):
                self.L.moe_p1_reset_stats(self.p1, self.cidx(l))
            return
        for l in range(1, self.cfg.n_layers):
            self.L.c_layer_reset_stats(self.cidx(l))

    def layer_stats(self, l: int) -> list[int]:
        if self.p1 is not None:                      # the 16 P1LayerStats fields (io_sched.h:23-44)
            o = (ctypes.c_uint64 * 16)()
            self.L.moe_p1_get_layer_stats(self.p1, self.cidx(l), o)
            return list(o)
        o = (ctypes.c_uint64 * 18)()
        self.L.c_layer_get_stats(self.cidx(l), o)
        return list(o)

    # ---- one token ---------------------------------------------------------------------------
    def _router(self, l: int, tables: bool = False):
        c = self.cfg
        wn = self.router_w[l + 1] if (c.prefetch and l + 1 < c.n_layers) else None
        x_in = self.xs[0] if l == 0 else None
        h_in = None if l == 0 else self.hs[l - 1]
        if tables:
            step_layer = self.cidx(l) if l >= 1 else -1
            pf_layer = self.cidx(l + 1) if wn is not None else -1
            rc = self.L.c_router_tables_dev(step_layer, pf_layer, c.prefetch_cap,
                                            h_in.data_ptr() if h_in is not None else None,
                                            self.norm_w[l - 1].data_ptr() if l > 0 else None, c.eps,
                                            x_in.data_ptr() if x_in is not None else None,
                                            self.xs[l].data_ptr() if l > 0 else None,
                                            self.router_w[l].data_ptr(), wn.data_ptr() if wn is not None else None,
                                            c.hidden, c.n_exp, c.top_k, c.top_m if wn is not None else 0,
                                            self.router_ws[l].data_ptr(), self.ids[l].data_ptr(),
                                            self.scores[l].data_ptr(), self.pred[l].data_ptr(),
                                            torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, "router_tables")
            return
        rc = self.L.moe_router(h_in.data_ptr() if h_in is not None else None,
                               self.norm_w[l - 1].data_ptr() if l > 0 else None, c.eps,
                               x_in.data_ptr() if x_in is not None else None,
                               self.xs[l].data_ptr() if l > 0 else None,
                               self.router_w[l].data_ptr(), wn.data_ptr() if wn is not None else None,
                               c.hidden, c.n_exp, c.top_k, c.top_m if wn is not None else 0,
                               self.router_ws[l].data_ptr(), self.ids[l].data_ptr(), self.scores[l].data_ptr(),
                               self.pred[l].data_ptr(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "router")

    def _layer_routed(self, l: int):
        """Resident layer with the selection inside gate/up: logits -> gate/up (selects the
        top-k itself, writes ids/scores) -> down."""
        c = self.cfg
        stream = torch.cuda.current_stream().cuda_stream
        x_in = self.xs[0] if l == 0 else None
        h_in = None if l == 0 else self.hs[l - 1]
        _lib.check(self.L.moe_router_logits(h_in.data_ptr() if h_in is not None else None,
                                            self.norm_w[l - 1].data_ptr() if l > 0 else None, c.eps,
                                            x_in.data_ptr() if x_in is not None else None,
                                            self.xs[l].data_ptr() if l > 0 else None, self.router_w[l].data_ptr(),
                                            c.hidden, c.n_exp, self.logits[l].data_ptr(), stream), "router_logits")
        pool = self.full_pools[l].data_ptr()
        _lib.check(self.L.moe_q2_gate_up_routed(self.xs[l].data_ptr(), self.logits[l].data_ptr(), c.n_exp, c.top_k,
                                                pool, self.blob_bytes, c.hidden, c.inter, c.group,
                                                self.ids[l].data_ptr(), self.scores[l].data_ptr(),
                                                self.h_ws.data_ptr(), stream), "gate_up_routed")
        _lib.check(self.L.moe_q2_down(self.h_ws.data_ptr(), pool, self.blob_bytes, c.n_exp, self.ids[l].data_ptr(),
                                      self.scores[l].data_ptr(), c.top_k, c.hidden, c.inter, c.group,
                                      self.xs[l].data_ptr(), self.hs[l].data_ptr(), 0, stream), "down")

    def _glu(self, l: int):
        c = self.cfg
        stream = torch.cuda.current_stream().cuda_stream
        L = self.L
        if l == 0 or self.mode == "device" or c.resident:
            # device-driven layers are ordered by the stream alone (no copy/read events)
            if l == 0 or c.resident:
                pool = (self.full_pools[l] if c.resident else self.pool0).data_ptr()
                n_slots, slots = c.n_exp, self.ids[l].data_ptr()
            else:
                pool, n_slots, slots = self.pools[l].data_ptr(), self.capacities[l], self.slot_inds[l].data_ptr()
            rc = L.moe_q2_switch_glu(self.xs[l].data_ptr(), pool, self.blob_bytes, n_slots, slots,
                                     self.scores[l].data_ptr(), c.top_k, c.hidden, c.inter, c.group,
                                     self.xs[l].data_ptr(), self.h_ws.data_ptr(), self.hs[l].data_ptr(), 0, stream)
        else:
            rc = L.c_layer_switch_glu(self.cidx(l), self.xs[l].data_ptr(), self.scores[l].data_ptr(),
                                      self.xs[l].data_ptr(), self.h_ws.data_ptr(), self.hs[l].data_ptr(), 0,
                                      c.top_k, stream)
        _lib.check(rc, "switch_glu")

    def decode_token_device(self):
        """Device-driven token: no host synchronisation; reads xs[0], writes xs[n_layers].

        Main stream, layer l: router(l) -> [join prefetch table(l)] -> slot step(l) ->
        [join prefetch copies(l)] -> demand copies(l) -> gate/up -> down.
        Side stream: prefetch table(l+1) as soon as router(l) has produced the prediction;
        prefetch copies(l+1) once the demand copies of layer l are queued ahead of them.

        The PCIe link is the bottleneck of this workload, so the order is chosen to keep it
        busy: demand copies first (they gate this layer's GEMV), prefetch copies next, running
        under this layer's GEMV and the next layer's router and step.  The demand copies of a
        layer wait for its prefetch copies because both may target the same slot."""
        c = self.cfg
        main = torch.cuda.current_stream()
        for l in range(c.n_layers):
            if c.resident:
                if c.routed_glu:
                    self._layer_routed(l)
                else:
                    self._router(l)
                    self._glu(l)
                continue
            if c.fused_tables:
                self._layer_fused(l, main)
                continue
            self._router(l)
            if l >= 1:
                if c.prefetch:
                    main.wait_event(self.ev_pref[l])       # table of prefetch(l) updated
                _lib.check(self.L.c_layer_step_decode_dev(self.cidx(l), self.ids[l].data_ptr(), c.top_k, -1,
                                                          main.cuda_stream), "step_dev")
            if c.prefetch and l + 1 < c.n_layers:
                self.ev_pred[l].record(main)
                self.side.wait_event(self.ev_pred[l])
                _lib.check(self.L.c_layer_start_prefetch_dev(self.cidx(l + 1), self.pred[l].data_ptr(), c.top_m,
                                                             c.prefetch_cap, -1, self.side.cuda_stream),
                           "prefetch_dev")
                self.ev_pref[l + 1].record(self.side)
            if l >= 1:
                if c.prefetch:
                    main.wait_event(self.ev_copy[l])       # prefetch copies(l) landed
                _lib.check(self.L.c_layer_stage_dev(self.cidx(l), 0, c.stage_ctas, main.cuda_stream), "stage_demand")
            if c.prefetch and l + 1 < c.n_layers:
                self.ev_demand[l].record(main)
                self.side.wait_event(self.ev_demand[l])
                _lib.check(self.L.c_layer_stage_dev(self.cidx(l + 1), 1, c.pf_stage_ctas or c.stage_ctas,
                                                    self.side.cuda_stream), "stage_prefetch")
                self.ev_copy[l + 1].record(self.side)
            self._glu(l)
        _lib.check(self.L.moe_rmsnorm(self.hs[c.n_layers - 1].data_ptr(), self.norm_w[c.n_layers - 1].data_ptr(),
                                      c.eps, c.hidden, self.xs[c.n_layers].data_ptr(), main.cuda_stream), "rmsnorm")

    def demand_overlaps_prefetch(self, l: int) -> bool:
        """Whether layer l's demand copies may be queued before its prefetch copies have landed.

        A demand miss takes the oldest unprotected slot; the experts the last prefetch fetched
        are the newest entries of the table (nothing touches it between that prefetch and this
        step), so they are reached only after every older unprotected entry: at least
        capacity - fetched - top_k of them, which covers the at most top_k misses when
        capacity >= 2 top_k + fetched.  Then no demand copy targets a slot a prefetch copy
        is still writing, and the join can move from before the demand copies to before the
        GEMV that reads the prefetched slots (it then overlaps the demand copies).  `fetched`
        is the most one prefetch can fetch: the cap as the table applies it (a cap outside
        1..31 means 32, expert_io.c:545), and never more than the predictions it is given."""
        c = self.cfg
        return self.capacities[l] >= 2 * c.top_k + effective_fetch_cap(c.prefetch_cap, c.top_m)

    def _layer_fused(self, l: int, main):
        """One layer of the device-driven token with the table work inside the router:
        main: router + step(l) + prefetch table(l+1) -> demand copies(l) -> [join prefetch
        copies(l)] -> gate/up -> down (the join goes before the demand copies when the pool is
        too small for demand_overlaps_prefetch);  side: prefetch copies(l+1) after the demand
        copies of layer l (demand first: they gate this layer's GEMV)."""
        c = self.cfg
        self._router(l, tables=True)
        pf = c.prefetch and l + 1 < c.n_layers
        if self.file_device:                           # the misses go to the feeder's readers now
            if l >= 1:
                _lib.check(self.L.c_layer_publish_dev(self.cidx(l), 0, main.cuda_stream), "publish_demand")
            if pf:
                _lib.check(self.L.c_layer_publish_dev(self.cidx(l + 1), 1, main.cuda_stream), "publish_prefetch")
        if l >= 1:
            early = c.prefetch and self.demand_overlaps_prefetch(l)
            if c.prefetch and not early:
                main.wait_event(self.ev_copy[l])
            _lib.check(self.L.c_layer_stage_dev(self.cidx(l), 0, c.stage_ctas, main.cuda_stream), "stage_demand")
        if pf:
            self.ev_demand[l].record(main)
            self.side.wait_event(self.ev_demand[l])
            _lib.check(self.L.c_layer_stage_dev(self.cidx(l + 1), 1, c.pf_stage_ctas or c.stage_ctas,
                                                self.side.cuda_stream), "stage_prefetch")
            self.ev_copy[l + 1].record(self.side)
        if l >= 1 and c.prefetch and self.demand_overlaps_prefetch(l):
            main.wait_event(self.ev_copy[l])           # the GEMV reads the prefetched slots
        self._glu(l)

    def decode_token_host(self):
        """Reference-shaped token: one device->host read of (ids, pred) per layer."""
        c = self.cfg
        L = self.L
        main = torch.cuda.current_stream()
        L.c_set_compute_stream(ctypes.c_void_p(main.cuda_stream))
        if c.sched:
            return self._decode_token_sched(main)
        for l in range(c.n_layers):
            self._router(l)
            if l == 0:
                self._glu(0)
                if c.prefetch and c.n_layers > 1:
                    p = self.pred[0, :c.top_m].tolist()
                    L.c_layer_start_prefetch(self.cidx(1), (ctypes.c_int32 * c.top_m)(*p), c.top_m, c.prefetch_cap)
                continue
            sel = torch.cat([self.ids[l], self.pred[l, :c.top_m]]).tolist()      # the one sync per layer
            ids, pred = sel[:c.top_k], sel[c.top_k:]
            n = L.c_layer_step_decode_ex(self.cidx(l), (ctypes.c_uint32 * c.top_k)(*ids), c.top_k, 1)
            _lib.check(n, "step")
            self._glu(l)                                  # waits for this layer's copies on the GPU
            if c.prefetch and l + 1 < c.n_layers:
                L.c_layer_start_prefetch(self.cidx(l + 1), (ctypes.c_int32 * c.top_m)(*pred), c.top_m,
                                         c.prefetch_cap)
        _lib.check_error("decode_token_host")
        _lib.check(L.moe_rmsnorm(self.hs[c.n_layers - 1].data_ptr(), self.norm_w[c.n_layers - 1].data_ptr(),
                                 c.eps, c.hidden, self.xs[c.n_layers].data_ptr(), main.cuda_stream), "rmsnorm")

    def decode_token_p1(self):
        """The C++ runner's `--io p1` token (cpp/src/engine.cpp:572-610): per cached layer, end
        the layer's last GPU reader and unpin its slots, step_decode, wait for the urgent reads if
        any are pending, the SwitchGLU over the slot ids the scheduler wrote, mark the reader,
        then queue the next layer's prefetch."""
        c, L, P = self.cfg, self.L, self.p1
        main = torch.cuda.current_stream()
        for l in range(c.n_layers):
            self._router(l)
            if l == 0:
                self._glu(0)
                if c.prefetch and c.n_layers > 1:
                    p = self.pred[0, :c.top_m].tolist()
                    L.moe_p1_start_prefetch(P, self.cidx(1), (ctypes.c_int32 * c.top_m)(*p), c.top_m,
                                            c.prefetch_cap)
                continue
            sel = torch.cat([self.ids[l], self.pred[l, :c.top_m]]).tolist()      # the one sync per layer
            ids, pred = sel[:c.top_k], sel[c.top_k:]
            li = self.cidx(l)
            L.moe_p1_unpin_layer_slots(P, li)           # the layer's last reader ended before that sync
            n = L.moe_p1_step_decode(P, li, (ctypes.c_uint32 * c.top_k)(*ids), c.top_k, None)
            _lib.check(n, "p1 step_decode")
            if n > 0:
                L.moe_p1_wait_layer_urgent(P, li)
            rc = L.moe_q2_switch_glu(self.xs[l].data_ptr(), self.pools[l].data_ptr(), self.blob_bytes,
                                     self.capacities[l], self.slot_inds[l].data_ptr(), self.scores[l].data_ptr(),
                                     c.top_k, c.hidden, c.inter, c.group, self.xs[l].data_ptr(),
                                     self.h_ws.data_ptr(), self.hs[l].data_ptr(), 0, main.cuda_stream)
            _lib.check(rc, "switch_glu")
            _lib.check(L.moe_p1_mark_read(P, li, ctypes.c_void_p(main.cuda_stream)), "p1 mark_read")
            if c.prefetch and l + 1 < c.n_layers:
                L.moe_p1_start_prefetch(P, self.cidx(l + 1), (ctypes.c_int32 * c.top_m)(*pred), c.top_m,
                                        c.prefetch_cap)
        _lib.check_error("decode_token_p1")
        _lib.check(L.moe_rmsnorm(self.hs[c.n_layers - 1].data_ptr(), self.norm_w[c.n_layers - 1].data_ptr(),
                                 c.eps, c.hidden, self.xs[c.n_layers].data_ptr(), main.cuda_stream), "rmsnorm")

    def _decode_token_sched(self, main):
        """The runner's decode loop (cpp/src/engine.cpp:545-560,700-730): after the resident
        layer 0 a prefetch-only call for layer 1, then per cached layer one
        c_layer_decode_step_sched(l, ids, k, pred(l+1), m, l+1, cap, flags) -- step of l and
        prefetch of l+1 in one call -- and the layer's SwitchGLU; with split, the hit experts
        run first and the missed ones after their copies."""
        c, L = self.cfg, self.L
        m = c.top_m
        pf_cap = c.prefetch_cap if c.prefetch else 0
        stream = main.cuda_stream
        for l in range(c.n_layers):
            self._router(l)
            if l == 0:
                self._glu(0)
                if c.prefetch and c.n_layers > 1:
                    p = self.pred[0, :m].tolist()
                    _lib.check(L.c_layer_decode_step_sched(0, None, 0, (ctypes.c_int32 * m)(*p), m, self.cidx(1),
                                                           pf_cap, 0), "sched prefetch")
                continue
            sel = torch.cat([self.ids[l], self.pred[l, :m]]).tolist()      # the one sync per layer
            ids, pred = sel[:c.top_k], sel[c.top_k:]
            last = l + 1 >= c.n_layers or not c.prefetch
            flags = (4 if c.split else 0) | (2 if last else 0)
            n = L.c_layer_decode_step_sched(self.cidx(l), (ctypes.c_int32 * c.top_k)(*ids), c.top_k,
                                            None if last else (ctypes.c_int32 * m)(*pred), 0 if last else m,
                                            -1 if last else self.cidx(l + 1), pf_cap, flags)
            _lib.check(n, "decode_step_sched")
            if c.split and 0 < n < c.top_k:
                for part in (0, 1):
                    _lib.check(L.c_layer_switch_glu_split(self.cidx(l), part, self.xs[l].data_ptr(),
                                                          self.scores[l].data_ptr(), self.xs[l].data_ptr(),
                                                          self.h_ws.data_ptr(), self.hs[l].data_ptr(), stream),
                               "switch_glu_split")
            else:
                self._glu(l)
        _lib.check_error("decode_token_sched")
        _lib.check(L.moe_rmsnorm(self.hs[c.n_layers - 1].data_ptr(), self.norm_w[c.n_layers - 1].data_ptr(),
                                 c.eps, c.hidden, self.xs[c.n_layers].data_ptr(), stream), "rmsnorm")

    def check_io(self):
        """Raise if a device-driven file-backed layer's staging failed (a read error or a wait past
        its limit): the slot kept its old bytes, so outputs since then are wrong until
        reset_caches().  Reads the library's host-memory fault word (no GPU synchronisation: it
        covers the staging kernels that have run)."""
        if self.file_device and self.L.c_io_fault():
            torch.cuda.synchronize()
            raise _lib.NativeError(f"file tier: staging failed (table status by layer {self.table_status()}: 16 a read "
                                   "failed, 17 a wait timed out); reset_caches() before decoding on")

    def decode_token(self, x0: torch.Tensor | None = None) -> torch.Tensor:
        self.check_io()                              # a fault of an earlier token
        if x0 is not None:
            self.xs[0].copy_(x0)
        if self.token_io:
            self.L.c_begin_decode_token(0)
        if self.mode == "device" or self.cfg.resident:
            if self.graph is not None:
                self.graph.replay()
            else:
                self.decode_token_device()
        elif self.p1 is not None:
            self.decode_token_p1()
        elif self._host_sel:
            stream = torch.cuda.current_stream()
            _lib.check(self.L.moe_stack_token_host(ctypes.byref(self.desc), ctypes.c_void_p(stream.cuda_stream)),
                       "moe_stack_token_host")
            if self.mirror_ids:                      # the device copies the Python drivers keep
                self.ids[1:].copy_(torch.from_numpy(self.ids_host[1:]), non_blocking=True)
                self.pred[:, :self.pred_host.shape[1]].copy_(torch.from_numpy(self.pred_host), non_blocking=True)
        else:
            self.decode_token_host()
        if self.token_io:
            out = (ctypes.c_uint64 * 10)()
            self.L.c_end_decode_token(out)           # waits for the token's table work
            _lib.check_error("end_decode_token")
            self.last_token_io = list(out)
        return self.xs[self.cfg.n_layers]

    def table_status(self) -> dict[int, int]:
        """Nonzero status words of the device-driven tables (blocks): 1 / 2 rejected ids, 16 a
        file read failed, 17 a file-backed staging wait timed out."""
        if self.mode != "device" or self.cfg.resident:
            return {}
        st = {l: self.L.c_layer_table_status(self.cidx(l)) for l in range(1, self.cfg.n_layers)}
        return {l: v for l, v in st.items() if v}

    def capture_graph(self):
        """Capture one device-driven token into a HIP graph (replayed by decode_token)."""
        assert self.mode == "device"
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.decode_token_device()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = g

    def decode_totals(self) -> list[int]:
        """(hits, prefetch hits, misses, requests, demand bytes, prefetch bytes) over the cached
        layers; with the P1 scheduler: (lru_hits, prefetch_used, urgent_reads, decode_requests, bytes
        read, 0)."""
        if self.cfg.resident:
            return [0] * 6
        if self.p1 is not None:
            t = (ctypes.c_uint64 * 16)()
            self.L.moe_p1_get_total_stats(self.p1, self.cidx(self.cfg.n_layers), t)
            return [t[1], t[6], t[2], t[0], t[9], 0]
        o = (ctypes.c_uint64 * 6)()
        self.L.c_get_decode_totals(self.cidx(self.cfg.n_layers), o)
        return list(o)

    def close(self):
        torch.cuda.synchronize()
        self.graph = None
        for ptr in self._host_sel:
            self.L.c_host_free(ptr)
        self._host_sel = []
        if self.cfg.resident:
            self.full_pools = None
            return
        if self.p1 is not None:
            self.L.moe_p1_wait_all(self.p1)
            self.L.moe_p1_destroy(self.p1)
            self.p1 = None
        else:
            self.L.c_sync_copies()
            for l in range(1, self.cfg.n_layers):
                self.L.c_layer_init(self.cidx(l), -1, 16, None, None, None, 0)
        self.store.close()
        if self.cfg.store_file is not None:
            self.L.c_io_set_direct(0)

    def expert_blob(self, l: int, e: int) -> np.ndarray:
        """Expert e of layer l as a blob in the standard layout (q2format), from its pool (layer 0,
        resident stacks) or the host store."""
        c = self.cfg
        if l == 0 or c.resident:
            return (self.full_pools[l] if c.resident else self.pool0)[e].cpu().numpy()
        return self.store.view(l)[e]

    # algorithmic bytes of the routed experts touched per token (the roofline numerator)
    def routed_bytes_per_token(self) -> int:
        return self.cfg.n_layers * self.cfg.top_k * self.blob_bytes

    def router_bytes_per_token(self) -> int:
        c = self.cfg
        per = c.n_exp * c.hidden * 2
        return c.n_layers * per + (c.n_layers - 1) * per * int(c.prefetch)
