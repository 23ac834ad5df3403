"""GPU parity of the stacked decode with the on-disk tier: 6 layers at the full per-layer shapes
whose misses are read from a blob file by the reader threads (host-driven tables).

* every layer matches the oracle given the GPU's own input to that layer (teacher forcing), with
  the experts taken from the file;
* the id/prediction stream replayed through the oracle LRU in the reference's call order
  (loader.py:920-977) gives the same slots and counters;
* 1 reader thread with O_DIRECT and 8 threads through the page cache give bit-identical tokens;
* device-driven tables (the misses published to the library's feeder thread, staged by a kernel
  that waits for each read) give bit-identical tokens, slots and counters, eager and replayed
  from a HIP graph, through the page cache and with O_DIRECT; a truncated file and a staging
  wait past its (tiny) time limit are reported in the table status instead of hanging;
* the same stack on the P1 I/O scheduler (the C++ runner's `--io p1`: its own slot decisions, reads
  by 6 reader threads straight into HBM slot rows) gives bit-identical tokens too (the slots differ,
  the experts and their bytes do not), with the scheduler's counters consistent.
"""
import ctypes

import numpy as np
import pytest

from helpers import assert_close_rms
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, N_TOK = 6, 10


def _run(path, layer_base, threads, direct, io="exact", mode="host", graph=False):
    from moe_offload.stack import DecodeStack, StackConfig
    print(f"file stack: io={io} threads={threads} direct={direct} mode={mode} graph={graph}", flush=True)
    cfg = StackConfig(n_layers=N_LAYERS, seed=6, layer_base=layer_base, store_file=str(path), io_threads=threads,
                      io_direct=direct, io=io)
    st = DecodeStack(cfg, mode=mode)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(98)
    xs = torch.randn((N_TOK, cfg.hidden), device="cuda", generator=gen).half()
    rec = []
    for t in range(N_TOK):
        if graph and t == 1:                          # token 0 eager, the rest replayed
            st.capture_graph()
        st.decode_token(xs[t])
        torch.cuda.synchronize()
        if mode == "device":
            assert st.table_status() == {}, t
        rec.append({"ids": st.ids.cpu().numpy().copy(), "scores": st.scores.cpu().numpy().copy(),
                    "pred": st.pred.cpu().numpy().copy(), "xs": st.xs.cpu().numpy().copy(),
                    "hs": st.hs.cpu().numpy().copy(),
                    "slots": {l: st.slot_inds[l][:cfg.top_k].cpu().numpy().copy() for l in range(1, N_LAYERS)}})
    stats = {l: st.layer_stats(l) for l in range(1, N_LAYERS)}
    return st, rec, stats


def test_file_backed_stack(tmp_path):
    from moe_offload import q2format
    from moe_offload.stack import StackConfig, random_blobs
    c = StackConfig()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    blobs = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, "cuda").cpu().numpy()
    path = tmp_path / "layer.q2blob"
    q2format.write_blob_file(path, blobs, c.hidden, c.inter)
    st, rec, stats = _run(path, 50, 8, False)
    try:
        W = st.router_w.float().cpu().numpy().astype(np.float16)
        NW = st.norm_w.cpu().numpy()
        pool0 = st.pool0.cpu().numpy()
        for t in (0, N_TOK - 1):
            r = rec[t]
            for l in range(N_LAYERS):
                x = r["xs"][l]
                if l > 0:
                    want_x = q2.round_to(q2.rmsnorm(r["hs"][l - 1].astype(np.float64), NW[l - 1], c.eps), "f16")
                    assert np.array_equal(x.astype(np.float64), want_x), (t, l)
                ids, sc, _ = q2.route(q2.router_logits(x, W[l], "f16")[None], c.top_k, "f16")
                assert r["ids"][l].tolist() == ids[0].astype(np.int64).tolist(), (t, l)
                src = pool0 if l == 0 else blobs
                experts = lambda e: q2format.from_blob(src[e], c.hidden, c.inter, c.group)
                want = q2.moe_combine(x.astype(np.float64), ids[0], sc[0], experts, bits=2, group=64)
                assert_close_rms(r["hs"][l].astype(np.float64) - x.astype(np.float64), want, 1e-2, f"t{t} l{l}")
        layers = {l: olru.CLru(30 + l, st.capacities[l], expert_bytes=st.blob_bytes) for l in range(1, N_LAYERS)}
        for L in layers.values():
            L.reset_stats()
        for t in range(N_TOK):
            r = rec[t]
            layers[1].prefetch(r["pred"][0].tolist(), c.prefetch_cap)
            for l in range(1, N_LAYERS):
                slots, _ = layers[l].step(r["ids"][l].tolist())
                assert slots == r["slots"][l].tolist(), (t, l)
                if l + 1 < N_LAYERS:
                    layers[l + 1].prefetch(r["pred"][l].tolist(), c.prefetch_cap)
        for l in range(1, N_LAYERS):
            assert layers[l].stats() == stats[l], l
        for l in range(1, N_LAYERS):                  # every slot holds the expert its table names
            e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
            st.L.c_layer_get_lru_state(st.cidx(l), e, s, ctypes.byref(n))
            pool = st.pools[l].cpu().numpy()
            for i in range(n.value):
                assert np.array_equal(pool[s[i]], blobs[e[i]]), (l, e[i], s[i])
    finally:
        st.close()
    st2, rec2, stats2 = _run(path, 56, 1, True)
    try:
        for t in range(N_TOK):
            assert np.array_equal(rec2[t]["xs"], rec[t]["xs"]), t
            for l in range(1, N_LAYERS):
                assert np.array_equal(rec2[t]["slots"][l], rec[t]["slots"][l]), (t, l)
        assert stats2 == stats
    finally:
        st2.close()


@pytest.mark.parametrize("threads", [0, 6])
def test_p1_scheduler_stack_gives_the_same_tokens(tmp_path, threads):
    from moe_offload import q2format
    from moe_offload.stack import StackConfig, random_blobs
    c = StackConfig()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    blobs = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, "cuda").cpu().numpy()
    path = tmp_path / "layer.q2blob"
    q2format.write_blob_file(path, blobs, c.hidden, c.inter)
    st, rec, _ = _run(path, 50, 8, False)
    st.close()
    p1, prec, _ = _run(path, 0, threads, False, io="p1")
    try:
        for t in range(N_TOK):
            assert np.array_equal(prec[t]["xs"], rec[t]["xs"]), t
            assert np.array_equal(prec[t]["ids"], rec[t]["ids"]), t
        for l in range(1, N_LAYERS):                 # every routed slot held its expert's bytes
            pool = p1.pools[l].cpu().numpy()
            for j, s in enumerate(prec[-1]["slots"][l]):
                assert np.array_equal(pool[s], blobs[prec[-1]["ids"][l][j]]), (l, j)
        tot = p1.decode_totals()
        assert tot[3] == N_TOK * (N_LAYERS - 1) * p1.cfg.top_k
        for l in range(1, N_LAYERS):
            s16 = p1.layer_stats(l)
            assert s16[0] == N_TOK * p1.cfg.top_k
            assert s16[4] + s16[6] + s16[7] <= s16[3]     # cancelled + used + wasted <= issued
        from moe_offload import _lib
        assert _lib.last_error() == ""
    finally:
        p1.close()


def _blob_file(tmp_path, name="layer.q2blob"):
    from moe_offload import q2format
    from moe_offload.stack import StackConfig, random_blobs
    c = StackConfig()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(77)
    blobs = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, "cuda").cpu().numpy()
    path = tmp_path / name
    q2format.write_blob_file(path, blobs, c.hidden, c.inter)
    return path, blobs


@pytest.mark.parametrize("graph,threads,direct", [(False, 8, False), (True, 8, False), (True, 1, True)])
def test_device_driven_file_stack_matches_host_driven(tmp_path, graph, threads, direct):
    path, blobs = _blob_file(tmp_path)
    st, rec, stats = _run(path, 50, 8, False)
    st.close()
    dv, drec, dstats = _run(path, 44, threads, direct, mode="device", graph=graph)
    try:
        for t in range(N_TOK):
            assert np.array_equal(drec[t]["xs"], rec[t]["xs"]), t
            assert np.array_equal(drec[t]["ids"], rec[t]["ids"]), t
            for l in range(1, N_LAYERS):
                assert np.array_equal(drec[t]["slots"][l], rec[t]["slots"][l]), (t, l)
        assert dstats == stats
        for l in range(1, N_LAYERS):                  # every slot holds the expert its table names
            e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
            dv.L.c_layer_get_lru_state(dv.cidx(l), e, s, ctypes.byref(n))
            pool = dv.pools[l].cpu().numpy()
            for i in range(n.value):
                assert np.array_equal(pool[s[i]], blobs[e[i]]), (l, e[i], s[i])
    finally:
        dv.close()


def test_device_driven_file_stack_reports_failed_reads_and_timeouts(tmp_path):
    import os

    from moe_offload.stack import DecodeStack, StackConfig
    from moe_offload import _lib
    path, blobs = _blob_file(tmp_path)
    cfg = StackConfig(n_layers=3, seed=6, layer_base=40, store_file=str(path))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    x = torch.randn(cfg.hidden, device="cuda", generator=gen).half()
    # every expert past the first 8 lies beyond the end of the file: its read comes up short
    from moe_offload import q2format
    hdr = q2format.read_blob_header(str(path))
    short = tmp_path / "short.q2blob"
    with open(path, "rb") as f, open(short, "wb") as g:
        g.write(f.read(hdr["data_offset"] + 8 * hdr["blob_bytes"]))
    assert os.path.getsize(short) < os.path.getsize(path)
    print("file stack: truncated file", flush=True)
    st = DecodeStack(StackConfig(n_layers=3, seed=6, layer_base=40, store_file=str(short)), mode="device")
    try:
        st.decode_token(x)
        torch.cuda.synchronize()
        assert 16 in st.table_status().values()
    finally:
        st.close()
    # a wait limit far below one read's time: the cold layer's demand entries time out.  The fault
    # is sticky (the next token raises, the status stays 17) until reset_caches; the tokens after
    # it -- whose reads start only once the timed-out token's late reads have ended, though they
    # reuse the same bounce entries -- leave every slot holding the expert its table names.
    print("file stack: 1 us staging wait", flush=True)
    st = DecodeStack(cfg, mode="device")
    try:
        st.L.c_io_set_feed_timeout_us(1)
        st.decode_token(x)
        torch.cuda.synchronize()
        assert st.table_status().get(1) == 17
        assert st.L.c_io_fault() == 17
        st.L.c_io_set_feed_timeout_us(0)
        with pytest.raises(_lib.NativeError, match="staging failed"):
            st.decode_token(x)
        assert st.table_status().get(1) == 17
        st.reset_caches()
        assert st.table_status() == {} and st.L.c_io_fault() == 0
        gen.manual_seed(6)
        xs = torch.randn((3, cfg.hidden), device="cuda", generator=gen).half()
        for t in range(3):
            st.decode_token(xs[t])
            torch.cuda.synchronize()
            assert st.table_status() == {}, t
        for l in range(1, cfg.n_layers):
            e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
            st.L.c_layer_get_lru_state(st.cidx(l), e, s, ctypes.byref(n))
            assert n.value > 0
            pool = st.pools[l].cpu().numpy()
            for i in range(n.value):
                assert np.array_equal(pool[s[i]], blobs[e[i]]), (l, e[i], s[i])
    finally:
        st.L.c_io_set_feed_timeout_us(0)
        st.close()


def test_device_driven_file_layer_stages_only_published_lists(tmp_path):
    """Staging a file-backed device layer's list that a table operation changed since its last
    publication is refused on the host (it would copy the previous list's entries)."""
    from moe_offload import _lib
    from moe_offload.stack import DecodeStack, StackConfig
    path, blobs = _blob_file(tmp_path)
    st = DecodeStack(StackConfig(n_layers=2, seed=6, layer_base=46, store_file=str(path)), mode="device")
    try:
        L, li = st.L, st.cidx(1)
        s = torch.cuda.current_stream().cuda_stream
        ids = torch.arange(10, dtype=torch.int32, device="cuda")
        assert L.c_layer_step_decode_dev(li, ids.data_ptr(), 10, -1, s) == 0
        L.c_clear_error()
        assert L.c_layer_stage_dev(li, 0, 2, s) == -1 and "publication" in _lib.last_error()
        L.c_clear_error()
        assert L.c_layer_publish_dev(li, 0, s) == 0
        assert L.c_layer_stage_dev(li, 0, 2, s) == 0
        torch.cuda.synchronize()
        assert st.table_status() == {}
        pool = st.pools[1].cpu().numpy()
        slots = st.slot_inds[1][:10].cpu().numpy()
        for j, sl in enumerate(slots):                # a cold table: all ten missed and were read
            assert np.array_equal(pool[sl], blobs[j]), j
    finally:
        st.close()


def test_device_driven_file_stack_exits_cleanly_without_close(tmp_path):
    """A process that ends with a device-driven file stack still open (the feeder thread polling its
    pinned mailboxes) exits with status 0: the feeder stops before the runtime's teardown."""
    import os
    import subprocess
    import sys
    path, _ = _blob_file(tmp_path)
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = (
        "import sys, torch\n"
        f"sys.path[:0] = [{root!r}, {os.path.join(root, 'moe-offload_amd')!r}]\n"
        "from moe_offload.stack import DecodeStack, StackConfig\n"
        f"st = DecodeStack(StackConfig(n_layers=3, seed=6, layer_base=40, store_file={str(path)!r}), mode='device')\n"
        "st.decode_token(torch.randn(st.cfg.hidden, device='cuda').half())\n"
        "torch.cuda.synchronize()\n"
        "assert st.table_status() == {}\n"
        "print('token done', flush=True)\n"
    )
    print("file stack: child process exits without close()", flush=True)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-2000:])
    assert "token done" in r.stdout
