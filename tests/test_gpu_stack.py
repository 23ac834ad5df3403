"""GPU parity of the stacked decode (6 layers at the full per-layer shapes).

* the device-driven and host-driven drivers give bit-identical ids, slots and outputs;
* every layer matches the oracle given the GPU's own input to that layer (teacher forcing):
  router ids/scores/prediction exact, RMSNorm exact, SwitchGLU + residual within 1e-2 x RMS;
* the per-layer id/prediction stream replayed through the oracle LRU in the reference's call
  order (prefetch(1) after layer 0, then step(l), prefetch(l+1); loader.py:920-977) gives the
  same slots and counters as the library;
* the table work fused into the router and the separate table kernels agree; a graph replay
  equals eager execution;
* the host-driven loop run natively (moe_stack_token_host) equals the Python host driver bit for
  bit (ids, predictions, slots, outputs, counters).
"""
import numpy as np
import pytest

from helpers import assert_close_rms
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, N_TOK = 6, 12


def run_stack(mode, layer_base, graph=False, fused=True, native=False, token_io=False):
    from moe_offload.stack import DecodeStack, StackConfig
    cfg = StackConfig(n_layers=N_LAYERS, seed=5, layer_base=layer_base, fused_tables=fused, native_host=native)
    st = DecodeStack(cfg, mode=mode)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(99)
    xs = torch.randn((N_TOK, cfg.hidden), device="cuda", generator=gen).half()
    rec = []
    if graph:
        st.capture_graph()
    if token_io:
        st.set_token_accounting(True)
    try:
        for t in range(N_TOK):
            st.decode_token(xs[t])
            torch.cuda.synchronize()
            rec.append({"ids": st.ids.cpu().numpy().copy(), "scores": st.scores.cpu().numpy().copy(),
                        "pred": st.pred.cpu().numpy().copy(), "xs": st.xs.cpu().numpy().copy(),
                        "hs": st.hs.cpu().numpy().copy(), "io": st.last_token_io,
                        "slots": {l: st.slot_inds[l][:cfg.top_k].cpu().numpy().copy() for l in range(1, N_LAYERS)}})
    finally:
        if token_io:
            st.set_token_accounting(False)
    stats = {l: st.layer_stats(l) for l in range(1, N_LAYERS)}
    return st, rec, stats


@pytest.fixture(scope="module")
def runs():
    dev_st, dev_rec, dev_stats = run_stack("device", 10)
    host_st, host_rec, host_stats = run_stack("host", 20)
    yield (dev_st, dev_rec, dev_stats), (host_st, host_rec, host_stats)
    dev_st.close()
    host_st.close()


def test_device_and_host_drivers_agree(runs):
    (_, d, ds), (_, h, hs) = runs
    for t in range(N_TOK):
        assert np.array_equal(d[t]["ids"], h[t]["ids"]), f"token {t}"
        assert np.array_equal(d[t]["pred"], h[t]["pred"]), f"token {t}"
        for l in range(1, N_LAYERS):
            assert np.array_equal(d[t]["slots"][l], h[t]["slots"][l]), (t, l)
        assert np.array_equal(d[t]["xs"], h[t]["xs"]), f"token {t}"
    assert ds == hs


def test_layers_match_oracle_teacher_forced(runs):
    from moe_offload import q2format
    (st, rec, _), _ = runs
    c = st.cfg
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
            assert np.array_equal(r["scores"][l].astype(np.float64), sc[0]), (t, l)
            if l + 1 < N_LAYERS:
                p = q2.predict_topm(q2.router_logits(x, W[l + 1], "f16")[None], c.top_m)
                assert r["pred"][l].tolist() == p[0].tolist(), (t, l)
            src = pool0 if l == 0 else st.store.view(l)
            experts = lambda e: q2format.from_blob(src[e], c.hidden, c.inter, c.group)
            want = q2.moe_combine(x.astype(np.float64), ids[0], sc[0], experts, bits=2, group=64)
            assert_close_rms(r["hs"][l].astype(np.float64) - x.astype(np.float64), want, 1e-2, f"t{t} l{l}")


def test_slot_sequence_matches_oracle_lru(runs):
    (st, rec, stats), _ = runs
    c = st.cfg
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


def test_separate_table_launches_match_fused(runs):
    """The router with the table work in its last block and the separate step / prefetch
    kernels take identical decisions."""
    (_, d, ds), _ = runs
    st, u, us = run_stack("device", 0, fused=False)
    try:
        for t in range(N_TOK):
            assert np.array_equal(u[t]["xs"], d[t]["xs"]), f"token {t}"
            for l in range(1, N_LAYERS):
                assert np.array_equal(u[t]["slots"][l], d[t]["slots"][l]), (t, l)
        assert us == ds
    finally:
        st.close()


def test_graph_replay_matches_eager(runs):
    (_, d, _), _ = runs
    st, g, _ = run_stack("device", 40, graph=True)
    try:
        for t in range(N_TOK):
            assert np.array_equal(g[t]["xs"], d[t]["xs"]), f"token {t}"
            for l in range(1, N_LAYERS):
                assert np.array_equal(g[t]["slots"][l], d[t]["slots"][l]), (t, l)
    finally:
        st.close()


def test_router_tables_reject_one_layer_for_step_and_prefetch(runs):
    """The step and the prefetch run in two waves at once; naming one table for both is refused
    before anything is launched."""
    from moe_offload import _lib
    (st, _, _), _ = runs
    c, l = st.cfg, 2
    rc = st.L.c_router_tables_dev(st.cidx(l), st.cidx(l), c.prefetch_cap, st.hs[l - 1].data_ptr(),
                                  st.norm_w[l - 1].data_ptr(), c.eps, None, st.xs[l].data_ptr(),
                                  st.router_w[l].data_ptr(), st.router_w[l + 1].data_ptr(), c.hidden, c.n_exp,
                                  c.top_k, c.top_m, st.router_ws[l].data_ptr(), st.ids[l].data_ptr(),
                                  st.scores[l].data_ptr(), st.pred[l].data_ptr(),
                                  torch.cuda.current_stream().cuda_stream)
    with pytest.raises(_lib.NativeError, match="same layer"):
        _lib.check(rc, "router_tables")


def test_native_host_runner_matches_python_host_driver(runs):
    _, (_, h, hs) = runs
    st, nat, ns = run_stack("host", 30, native=True)
    try:
        assert st._host_sel, "the native runner was not used"
        for t in range(N_TOK):
            assert np.array_equal(nat[t]["ids"], h[t]["ids"]), f"token {t}"
            assert np.array_equal(nat[t]["pred"], h[t]["pred"]), f"token {t}"
            assert np.array_equal(nat[t]["xs"], h[t]["xs"]), f"token {t}"
            for l in range(1, N_LAYERS):
                assert np.array_equal(nat[t]["slots"][l], h[t]["slots"][l]), (t, l)
        assert ns == hs
    finally:
        st.close()


@pytest.mark.parametrize("graph", [False, True])
def test_token_accounting_on_device_tables_matches_host_tables(runs, graph):
    """Per-token I/O accounting (cpp/third_party/expert_io.c:98-111,1002-1038) counted by the
    device-driven tables' kernels equals the host tables' counts for the same token stream
    (eager, and with the token replayed from a HIP graph): every token's 10 counters.  Their sums
    tie to the layers' own counters: LRU hits, prefetch hits and misses are the layers' three
    classes of requests, and the bytes = (misses + prefetch loads) x blob bytes."""
    (_, d, ds), _ = runs
    dst, drec, dstats = run_stack("device", 50, graph=graph, token_io=True)
    hst, hrec, hstats = run_stack("host", 57, token_io=True)
    try:
        assert dstats == ds == hstats                 # the same decisions as without accounting
        for t in range(N_TOK):
            assert np.array_equal(drec[t]["xs"], d[t]["xs"]), f"token {t}"
            assert drec[t]["io"] == hrec[t]["io"], f"token {t}: {drec[t]['io']} vs {hrec[t]['io']}"
        tot = np.array([r["io"] for r in drec], dtype=np.int64).sum(axis=0)
        col = lambda i: sum(v[i] for v in dstats.values())   # noqa: E731
        assert (tot[0], tot[3], tot[1]) == (col(1), col(2), col(3))
        assert tot[0] + tot[3] + tot[1] == col(0)
        assert tot[9] == (tot[1] + tot[2]) * dst.blob_bytes
        assert tot[1] > 0 and tot[2] > 0              # the stream does miss and prefetch
    finally:
        dst.close()
        hst.close()
