"""P1 I/O scheduler with its slot pools in HBM (reads staged in pinned memory, copied by DMA).

* the golden traces of the reference's io_sched.cpp replay call for call with the 9 slot pools and
  the slot ids in device memory (no reader threads): slots, pending counts, counters, pins and the
  bytes every HBM slot row holds;
* 8 reader threads, 4 layers, forced invalidations and next-layer prefetches, with the GPU as the
  reader: every step's slots are checked on the device against the file's rows right after
  wait_layer_urgent, the layer's reader is marked with moe_p1_mark_read, and the scheduler's own
  reader wait (no callback) waits for that event before it reuses a pinned slot.
"""
from __future__ import annotations

import ctypes
import gzip
import json
import os
import random
from pathlib import Path

import numpy as np
import pytest

from p1_replay import ProductAdapter, decode_content, make_file, replay, row_pattern

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

HERE = Path(__file__).resolve().parent


class DeviceAdapter(ProductAdapter):
    """ProductAdapter whose slot pools and slot ids live in HBM."""

    def _alloc(self, layer, cap):
        if layer in self.bufs:
            self.retired.append(self.bufs[layer])
        self.bufs[layer] = [torch.full((cap, rb), 0xCD, dtype=torch.uint8, device="cuda") for rb in self.rb]
        self.slot_inds[layer] = torch.zeros(16, dtype=torch.int32, device="cuda")

    def _ptrs(self, layer):
        return (ctypes.c_uint64 * 9)(*[b.data_ptr() for b in self.bufs[layer]])

    def layer_init(self, l, cap):
        self._alloc(l, cap)
        u64 = ctypes.c_uint64 * 9
        self.L.moe_p1_layer_init(self.h, l, self.fd, cap, len(self.rb), u64(*self.offs[l]), u64(*self.rb),
                                 self._ptrs(l), self.slot_inds[l].data_ptr())

    def resize_buffers(self, layer, cap, old_slots):
        new = [torch.full((cap, rb), 0xCD, dtype=torch.uint8, device="cuda") for rb in self.rb]
        if old_slots:
            idx = torch.tensor(old_slots, dtype=torch.long, device="cuda")
            for t in range(len(self.rb)):
                new[t][:len(old_slots)] = self.bufs[layer][t][idx]
        torch.cuda.synchronize()
        self.retired.append(self.bufs[layer])
        self.bufs[layer] = new

    def resize(self, l, cap, eids, slots, old_slots):
        self.resize_buffers(l, cap, old_slots)
        from p1_replay import _i32
        self.L.moe_p1_resize_layer(self.h, l, cap, self._ptrs(l), self.slot_inds[l].data_ptr(), _i32(eids),
                                   _i32(slots), len(eids))

    def step(self, l, eids):
        n, slots = super().step(l, eids)
        torch.cuda.synchronize()
        assert self.slot_inds[l][:len(eids)].cpu().tolist() == slots
        return n, slots

    def content(self, layer):
        torch.cuda.synchronize()
        return decode_content([b.cpu().numpy() for b in self.bufs[layer]], layer, self.n_exp, self.rb)


def test_golden_traces_with_hbm_pools(tmp_path):
    g = json.load(gzip.open(HERE / "golden" / "p1_traces.json.gz", "rt"))
    path = tmp_path / "experts.bin"
    offs = make_file(path, g["layers"], g["n_exp"], g["row_bytes"])
    fd = os.open(path, os.O_RDONLY)
    try:
        for tr in g["traces"][:20]:
            print(f"p1 hbm trace seed {tr['seed']}", flush=True)
            ad = DeviceAdapter(fd, offs, g["n_exp"], g["row_bytes"], threads=0)
            try:
                got = replay(ad, tr)
            finally:
                torch.cuda.synchronize()
                ad.close()
            for i, (want, have) in enumerate(zip(tr["expect"], got)):
                assert have == want, f"seed {tr['seed']} call {i} {tr['ops'][i]}"
    finally:
        os.close(fd)


def test_threaded_readers_with_gpu_readers(tmp_path):
    from moe_offload import _lib
    L = _lib.lib()
    N_EXP, ROW = 32, [100_352, 256, 256, 100_352, 256, 256, 100_352, 256, 256]
    layers, cap, k = [1, 2, 3, 4], 12, 4
    path = tmp_path / "experts.bin"
    offs = make_file(path, layers, N_EXP, ROW)
    fd = os.open(path, os.O_RDONLY)
    # the file's rows on the device, to check slots where they are read
    want = {l: [torch.from_numpy(np.stack([row_pattern(l, e, t, rb) for e in range(N_EXP)])).cuda()
                for t, rb in enumerate(ROW)] for l in layers}
    pools = {l: [torch.full((cap, rb), 0xCD, dtype=torch.uint8, device="cuda") for rb in ROW] for l in layers}
    sinds = {l: torch.zeros(16, dtype=torch.int32, device="cuda") for l in layers}
    h = L.moe_p1_create()
    L.moe_p1_init(h, 8)
    stream = torch.cuda.current_stream().cuda_stream
    L.moe_p1_set_compute_stream(h, ctypes.c_void_p(stream))
    u64 = ctypes.c_uint64 * 9
    mt = L.moe_p1_mt64_create(99)
    draw = ctypes.cast(L.moe_p1_mt64_uniform, ctypes.c_void_p)
    rng = random.Random(5)
    bad = torch.zeros((), dtype=torch.int64, device="cuda")
    try:
        for l in layers:
            L.moe_p1_layer_init(h, l, fd, cap, 9, u64(*offs[l]), u64(*ROW), u64(*[p.data_ptr() for p in pools[l]]),
                                sinds[l].data_ptr())
        for step in range(60):
            for l in layers:
                if step % 5 == 2:
                    L.moe_p1_force_invalidate(h, l, 0.3, draw, mt)
                eids = rng.sample(range(N_EXP), k)
                n = L.moe_p1_step_decode(h, l, (ctypes.c_uint32 * k)(*eids), k, None)
                assert n >= 0, _lib.last_error()
                if n > 0:
                    L.moe_p1_wait_layer_urgent(h, l)
                # the GPU reader: compares the routed slots (ids read from device memory) with the file
                sl = sinds[l][:k].long()
                ev = torch.tensor(eids, dtype=torch.long, device="cuda")
                for t in range(9):
                    bad += (pools[l][t][sl] != want[l][t][ev]).sum()
                _lib.check(L.moe_p1_mark_read(h, l, ctypes.c_void_p(stream)), "mark_read")
                if l + 1 in pools:
                    pred = rng.sample(range(N_EXP), 6)
                    L.moe_p1_start_prefetch(h, l + 1, (ctypes.c_int32 * 6)(*pred), 6, 3)
        L.moe_p1_wait_all(h)
        torch.cuda.synchronize()
        assert int(bad) == 0
        tot = (ctypes.c_uint64 * 16)()
        L.moe_p1_get_total_stats(h, 5, tot)
        assert tot[0] == 60 * 4 * k and tot[2] > 0 and tot[3] > 0 and tot[11] > 0
        assert tot[4] + tot[7] + tot[6] == tot[3]
        assert _lib.last_error() == ""
    finally:
        torch.cuda.synchronize()
        L.moe_p1_destroy(h)
        L.moe_p1_mt64_destroy(mt)
        os.close(fd)
