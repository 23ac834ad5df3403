"""On-disk tier on the GPU: cached layers whose misses are read from a file by the reader threads
(one read per tensor and run of consecutive experts, into pinned bounce buffers) and copied to the
HBM slot pools (the reference reads its shard the same way, `mlx-qwen38/expert_io.c:113-276`).

Blob file: 40 decode steps (capacity 16 over 64 experts) then an 8-token prefill.  Reference
shard read in place (9 tensors, bf16 scales, hidden 2560 / inter 640): decode steps with
prefetches, 1 and 8 reader threads, page cache and O_DIRECT, with host- and device-driven tables
(the latter through the feeder thread and the waiting staging kernels).  Slot decisions and counters match
the oracle LRU, every slot holds the expert the table names, outputs match the fp64 oracle within
1e-2 x RMS.
"""
import ctypes

import numpy as np
import pytest

from helpers import (H, I, K, assert_close_rms, expert_fn, experts_bf16, experts_np, oracle_moe, role_arrays,
                     write_reference_shard)
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_EXP, CAP, LAYER = 64, 16, 34


def _state(L, layer):
    e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
    L.c_layer_get_lru_state(layer, e, s, ctypes.byref(c))
    return list(e[:c.value]), list(s[:c.value])


def test_file_backed_layer(tmp_path):
    from moe_offload import _lib, q2format, synth
    from moe_offload.loader import CachedSwitchGLU, FileExpertStore
    dev = torch.device("cuda:0")
    mlx, blobs = experts_np(N_EXP, H, I, seed=17)
    path = tmp_path / "layer34.q2blob"
    q2format.write_blob_file(path, blobs, H, I)
    store = FileExpertStore({LAYER: str(path)})
    mod = CachedSwitchGLU(store, LAYER, CAP, H, I)
    ora = olru.CLru(LAYER, CAP, expert_bytes=blobs.shape[1])
    ora.reset_stats()
    L = _lib.lib()
    try:
        ids_seq = synth.expert_id_stream(40, K, N_EXP, seed=21)
        xs = synth.hidden_states(40, H, seed=22)
        rng = np.random.default_rng(23)
        for t, ids in enumerate(ids_seq):
            ids = [int(v) for v in ids]
            sc = rng.random(K).astype(np.float16)
            out = mod.forward_combined(torch.from_numpy(xs[t]).to(dev), ids, torch.from_numpy(sc).to(dev))
            slots, _ = ora.step(ids)
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots, t
            if t in (0, 17, 39):
                want = oracle_moe(xs[t], np.array(ids), sc, mlx)
                assert_close_rms(out.cpu().numpy(), want, 1e-2, f"step {t}")
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()

        # prefill through the file-backed layer (loads go through c_layer_load_sync)
        n_tok = 8
        pids = np.stack([rng.choice(N_EXP, K, replace=False) for _ in range(n_tok)]).astype(np.int32)
        px = synth.hidden_states(n_tok, H, seed=24)
        e0, s0 = ora.get_state()
        plan = q2.prefill_plan(pids.reshape(-1), e0, s0, CAP)
        y = mod(torch.from_numpy(px).to(dev)[None], torch.from_numpy(pids).to(dev)[None])
        torch.cuda.synchronize()
        yh = y[0].reshape(n_tok * K, H).cpu().numpy().astype(np.float64)
        flat = pids.reshape(-1)
        for e in sorted(set(flat.tolist()))[:6]:
            pairs = np.nonzero(flat == e)[0]
            want = q2.switch_glu_expert(px[pairs // K].astype(np.float64), *expert_fn(mlx)(e), bits=2, group=64)
            assert_close_rms(yh[pairs], want, 1e-2, f"prefill expert {e}")
        for _, _, le, ls in plan["chunks"]:
            if le:
                ora.load_sync(le, ls, 1)
        ora.set_state(*plan["new_lru"], plan["add_req"], plan["add_hits"], plan["add_misses"])
        assert _state(L, LAYER) == ora.get_state()
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        pool = mod.pool.cpu().numpy()
        for e, s in zip(*ora.get_state()):
            assert np.array_equal(pool[s], blobs[e]), (e, s)
        assert _lib.last_error() == ""
    finally:
        mod.close()
        store.close()


@pytest.mark.parametrize("threads,direct", [(1, 0), (8, 0), (8, 1)])
def test_reference_shard_read_in_place(tmp_path, threads, direct):
    from moe_offload import _lib
    from moe_offload.loader import CachedSwitchGLU, ShardExpertStore
    Hs, Is, Es, cap, layer = 2560, 640, 40, 12, 35
    print(f"shard in place: threads={threads} direct={direct}", flush=True)
    mlx = experts_bf16(Es, Hs, Is, seed=31)
    write_reference_shard(tmp_path / f"experts-{layer:02d}.safetensors", layer, mlx)
    want_rows = role_arrays(mlx)
    dev = torch.device("cuda:0")
    L = _lib.lib()
    L.c_io_init(threads)
    L.c_io_set_direct(direct)
    store = ShardExpertStore(tmp_path, layers=[layer])
    mod = None
    try:
        mod = CachedSwitchGLU(store, layer, cap)
        assert (mod.hidden, mod.inter) == (Hs, Is)
        assert L.c_io_threads() == threads
        print(f"O_DIRECT in use: {L.c_layer_io_direct(layer)}", flush=True)
        if not direct:
            assert L.c_layer_io_direct(layer) == 0
        lay = store.layout[layer]
        ora = olru.CLru(layer, cap, expert_bytes=mod.blob_bytes)
        ora.reset_stats()
        rng = np.random.default_rng(32)
        f = lambda e: tuple((p[0][e], p[1][e], p[2][e]) for p in mlx)
        for t in range(16):
            ids = [int(v) for v in rng.choice(Es, K, replace=False)]
            x = rng.standard_normal(Hs).astype(np.float16)
            sc = rng.dirichlet(np.ones(K)).astype(np.float16)
            out = mod.forward_combined(torch.from_numpy(x).to(dev), ids, torch.from_numpy(sc).to(dev))
            slots, _ = ora.step(ids)
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots, t
            if t in (0, 9, 15):
                want = q2.moe_combine(x.astype(np.float64), np.array(ids), sc.astype(np.float64), f, bits=2, group=64,
                                      sdtype="bf16")
                assert_close_rms(out.cpu().numpy(), want, 1e-2, f"step {t}")
            if t % 3 == 1:                       # prefetch 3 of 12 predicted experts for the next step
                pred = [int(v) for v in rng.choice(Es, 12, replace=False)]
                mod.start_prefetch(pred, 3)
                ora.prefetch(pred, 3)
        mod.wait_prefetch()
        torch.cuda.synchronize()
        L.c_sync_copies()
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        for e, sl in zip(*ora.get_state()):
            for t, r in enumerate(lay["roles"]):
                assert np.array_equal(mod.pools[t][sl].cpu().numpy(), want_rows[r][e]), (e, sl, t)
        assert _lib.last_error() == ""
    finally:
        if mod is not None:
            mod.close()
        L.c_io_set_direct(0)
        L.c_io_init(8)
        store.close()


@pytest.mark.parametrize("threads,direct", [(8, 0), (2, 1)])
def test_reference_shard_read_in_place_device_driven(tmp_path, threads, direct):
    """The same shard bound in place with device-driven tables: each decode step and prefetch
    publishes its misses to the feeder thread (c_layer_step_decode_dev / c_layer_start_prefetch_dev
    with staging), which reads the 9 tensors of each expert into its bounce entry; the staging
    kernels copy every tensor into its pool.  Slots, counters, pool rows and outputs as host-driven."""
    from moe_offload import _lib
    from moe_offload.loader import CachedSwitchGLU, ShardExpertStore
    Hs, Is, Es, cap, layer = 2560, 640, 40, 12, 38
    print(f"shard in place, device-driven: threads={threads} direct={direct}", flush=True)
    mlx = experts_bf16(Es, Hs, Is, seed=51)
    write_reference_shard(tmp_path / f"experts-{layer:02d}.safetensors", layer, mlx)
    want_rows = role_arrays(mlx)
    dev = torch.device("cuda:0")
    L = _lib.lib()
    L.c_io_init(threads)
    L.c_io_set_direct(direct)
    store = ShardExpertStore(tmp_path, layers=[layer])
    mod = None
    try:
        mod = CachedSwitchGLU(store, layer, cap)
        _lib.check(L.c_layer_set_device_mode(layer, 1), "device_mode")
        stream = torch.cuda.current_stream().cuda_stream
        lay = store.layout[layer]
        ora = olru.CLru(layer, cap, expert_bytes=mod.blob_bytes)
        ora.reset_stats()
        rng = np.random.default_rng(52)
        f = lambda e: tuple((p[0][e], p[1][e], p[2][e]) for p in mlx)
        y = torch.empty(Hs, dtype=torch.float32, device=dev)
        for t in range(16):
            ids = [int(v) for v in rng.choice(Es, K, replace=False)]
            x = rng.standard_normal(Hs).astype(np.float16)
            sc = rng.dirichlet(np.ones(K)).astype(np.float16)
            xt, sct = torch.from_numpy(x).to(dev), torch.from_numpy(sc).to(dev)
            it = torch.tensor(ids, dtype=torch.int32, device=dev)
            _lib.check(L.c_layer_step_decode_dev(layer, it.data_ptr(), K, 0, stream), "step_dev")
            _lib.check(L.c_layer_switch_glu(layer, xt.data_ptr(), sct.data_ptr(), None, mod._h_ws.data_ptr(),
                                            y.data_ptr(), 0, K, stream), "switch_glu")
            slots, _ = ora.step(ids)
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots, t
            assert L.c_layer_table_status(layer) == 0, t
            if t in (0, 9, 15):
                want = q2.moe_combine(x.astype(np.float64), np.array(ids), sc.astype(np.float64), f, bits=2, group=64,
                                      sdtype="bf16")
                assert_close_rms(y.cpu().numpy(), want, 1e-2, f"step {t}")
            if t % 3 == 1:                       # prefetch 3 of 12 predicted experts for the next step
                pred = [int(v) for v in rng.choice(Es, 12, replace=False)]
                pt = torch.tensor(pred, dtype=torch.int32, device=dev)
                _lib.check(L.c_layer_start_prefetch_dev(layer, pt.data_ptr(), 12, 3, 0, stream), "prefetch_dev")
                ora.prefetch(pred, 3)
        torch.cuda.synchronize()
        assert L.c_layer_table_status(layer) == 0
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        for e, sl in zip(*ora.get_state()):
            for tt, r in enumerate(lay["roles"]):
                assert np.array_equal(mod.pools[tt][sl].cpu().numpy(), want_rows[r][e]), (e, sl, tt)
        assert _lib.last_error() == ""
    finally:
        if mod is not None:
            L.c_layer_set_device_mode(layer, 0)
            mod.close()
        L.c_io_set_direct(0)
        L.c_io_init(8)
        store.close()


@pytest.mark.parametrize("mode", ["host", "device"])
def test_reference_shard_in_pinned_host_memory(tmp_path, mode):
    """HostShardStore: the shard's 9 tensors read whole into pinned memory (one read per tensor by
    the reader threads); a layer bound to it decodes with host- or device-driven staging."""
    from moe_offload import _lib
    from moe_offload.loader import CachedSwitchGLU, HostShardStore
    Hs, Is, Es, cap = 2560, 640, 40, 12
    layer = 36 if mode == "host" else 37
    print(f"host shard store: mode={mode}", flush=True)
    mlx = experts_bf16(Es, Hs, Is, seed=41)
    write_reference_shard(tmp_path / f"experts-{layer:02d}.safetensors", layer, mlx)
    want_rows = role_arrays(mlx)
    dev = torch.device("cuda:0")
    L = _lib.lib()
    store = HostShardStore(tmp_path, layers=[layer], threads=4)
    mod = None
    try:
        lay = store.layout[layer]
        for t, r in enumerate(lay["roles"]):
            assert np.array_equal(store.tensor(layer, t), want_rows[r]), t
        mod = CachedSwitchGLU(store, layer, cap)
        stream = torch.cuda.current_stream().cuda_stream
        if mode == "device":
            _lib.check(L.c_layer_set_device_mode(layer, 1), "device_mode")
        ora = olru.CLru(layer, cap, expert_bytes=mod.blob_bytes)
        ora.reset_stats()
        rng = np.random.default_rng(42)
        f = lambda e: tuple((p[0][e], p[1][e], p[2][e]) for p in mlx)
        y = torch.empty(Hs, dtype=torch.float32, device=dev)
        for t in range(12):
            ids = [int(v) for v in rng.choice(Es, K, replace=False)]
            x = rng.standard_normal(Hs).astype(np.float16)
            sc = rng.dirichlet(np.ones(K)).astype(np.float16)
            xt, sct = torch.from_numpy(x).to(dev), torch.from_numpy(sc).to(dev)
            if mode == "host":
                out = mod.forward_combined(xt, ids, sct)
            else:
                it = torch.tensor(ids, dtype=torch.int32, device=dev)
                _lib.check(L.c_layer_step_decode_dev(layer, it.data_ptr(), K, 0, stream), "step_dev")
                _lib.check(L.c_layer_stage_dev(layer, 0, 2, stream), "stage_dev")
                _lib.check(L.c_layer_switch_glu(layer, xt.data_ptr(), sct.data_ptr(), None, mod._h_ws.data_ptr(),
                                                y.data_ptr(), 0, K, stream), "switch_glu")
                out = y
            slots, _ = ora.step(ids)
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots, t
            if t in (0, 11):
                want = q2.moe_combine(x.astype(np.float64), np.array(ids), sc.astype(np.float64), f, bits=2, group=64,
                                      sdtype="bf16")
                assert_close_rms(out.cpu().numpy(), want, 1e-2, f"step {t}")
        torch.cuda.synchronize()
        for e, sl in zip(*ora.get_state()):
            for tt, r in enumerate(lay["roles"]):
                assert np.array_equal(mod.pools[tt][sl].cpu().numpy(), want_rows[r][e]), (e, sl, tt)
        assert _lib.last_error() == ""
    finally:
        if mod is not None:
            if mode == "device":
                L.c_layer_set_device_mode(layer, 0)
            mod.close()
        store.close()


@pytest.mark.parametrize("kind", ["file", "pinned"])
def test_reference_shard_prefill(tmp_path, kind):
    """Prefill through a layer bound to the reference's shard (9 tensors, bf16 scales, 2560 x 640):
    the grouped kernels read the 9 pools; outputs, LRU state, counters and pool contents follow
    the oracle's prefill plan after a few decode steps.  file: the chunk loads are reads of the
    shard by the reader threads; pinned: the shard in pinned host memory, the chunk loads one CU
    copy kernel over the 9 tensors."""
    from moe_offload import _lib
    from moe_offload.loader import CachedSwitchGLU, HostShardStore, ShardExpertStore
    Hs, Is, Es, cap = 2560, 640, 40, 16
    layer = 38 if kind == "file" else 39
    print(f"reference shard prefill: store={kind}", flush=True)
    mlx = experts_bf16(Es, Hs, Is, seed=51)
    write_reference_shard(tmp_path / f"experts-{layer:02d}.safetensors", layer, mlx)
    want_rows = role_arrays(mlx)
    dev = torch.device("cuda:0")
    L = _lib.lib()
    L.c_io_init(8)
    if kind == "file":
        store = ShardExpertStore(tmp_path, layers=[layer])
    else:
        store = HostShardStore(tmp_path, layers=[layer], threads=4)
    mod = None
    try:
        mod = CachedSwitchGLU(store, layer, cap)
        ora = olru.CLru(layer, cap, expert_bytes=mod.blob_bytes)
        ora.reset_stats()
        rng = np.random.default_rng(52)
        for t in range(5):
            ids = [int(v) for v in rng.choice(Es, K, replace=False)]
            x = rng.standard_normal(Hs).astype(np.float16)
            mod.forward_combined(torch.from_numpy(x).to(dev), ids, torch.ones(K, dtype=torch.float16, device=dev))
            ora.step(ids)
        n_tok = 12
        pids = np.stack([rng.choice(Es, K, replace=False) for _ in range(n_tok)]).astype(np.int32)
        px = rng.standard_normal((n_tok, Hs)).astype(np.float16)
        e0, s0 = ora.get_state()
        plan = q2.prefill_plan(pids.reshape(-1), e0, s0, cap)
        _lib.check(L.c_timing_begin(4096), "timing_begin")
        y = mod(torch.from_numpy(px).to(dev)[None], torch.from_numpy(pids).to(dev)[None])
        torch.cuda.synchronize()
        ms, nk = (ctypes.c_double * 11)(), (ctypes.c_int * 11)()
        _lib.check(L.c_timing_end(ms, nk), "timing_end")
        n_loads = sum(1 for _, _, le, _ in plan["chunks"] if le)
        assert n_loads > 0
        # kind 3: staging kernels -- the pinned store's chunk loads, none for the file's reads
        assert (nk[3] >= n_loads) if kind == "pinned" else (nk[3] == 0), (kind, nk[3], n_loads)
        yh = y[0].reshape(n_tok * K, Hs).cpu().numpy().astype(np.float64)
        flat = pids.reshape(-1)
        f = lambda e: tuple((p[0][e], p[1][e], p[2][e]) for p in mlx)
        for e in sorted(set(flat.tolist()))[:8]:
            pairs = np.nonzero(flat == e)[0]
            want = q2.switch_glu_expert(px[pairs // K].astype(np.float64), *f(e), bits=2, group=64, sdtype="bf16")
            assert_close_rms(yh[pairs], want, 1e-2, f"prefill expert {e}")
        for _, _, le, ls in plan["chunks"]:
            if le:
                ora.load_sync(le, ls, 1)
        ora.set_state(*plan["new_lru"], plan["add_req"], plan["add_hits"], plan["add_misses"])
        assert _state(L, layer) == ora.get_state()
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        lay = store.layout[layer]
        for e, sl in zip(*ora.get_state()):
            for tt, r in enumerate(lay["roles"]):
                assert np.array_equal(mod.pools[tt][sl].cpu().numpy(), want_rows[r][e]), (e, sl, tt)
        assert _lib.last_error() == ""
    finally:
        if mod is not None:
            mod.close()
        store.close()
