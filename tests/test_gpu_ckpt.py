"""GPU parity of the routed-expert decode over a model directory in the reference's own layout
(ckpt.CheckpointStack, OffloadEngine(model_path), CachedSwitchGLU(shard path); loader.py:311,
903-977, 1004-1095): 6 layers x 64 experts at the real layer shape (hidden 2560, inter 640, bf16
scales), the 8-bit group-64 routers read from base-00.safetensors, layer 0 pinned, 16-slot caches,
prefetch top-12 cap 3.

* device-driven tables (eager and graph-replayed) and host-driven tables (pinned store, and the
  shards read in place) give bit-identical tokens, ids, scores and slots;
* the id and prediction streams replayed through the oracle LRU in the reference's call order give
  the same slots and the same 18 counters per layer;
* at sampled (token, layer) points the layer matches the oracle given its own input: the glue
  x = bf16(RMSNorm(h)) bit-exact (one rounding from fp64), the 8-bit router's ids, bf16 scores and
  next-layer prediction bit-exact, the SwitchGLU plus residual within 1e-2 x RMS of fp64;
* CachedSwitchGLU built from a shard path, as the reference builds it, matches the oracle;
  OffloadEngine(model_path) decodes through the directory and reports the reference's keys.
"""
import ctypes

import numpy as np
import pytest

from helpers import assert_close_rms, write_model_dir
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, N_EXP, H, I, N_TOK = 6, 64, 2560, 640, 8


@pytest.fixture(scope="module")
def model_dir(tmp_path_factory):
    root = tmp_path_factory.mktemp("model")
    print("[ckpt] writing the model directory", flush=True)
    experts, routers = write_model_dir(root, N_LAYERS, N_EXP, H, I, seed=3)
    return root, experts, routers


def _run(root, mode, graph=False, store="host", layer_base=0):
    from moe_offload.ckpt import CheckpointStack, CkptConfig
    print(f"[ckpt] mode={mode} graph={graph} store={store}", flush=True)
    st = CheckpointStack(root, CkptConfig(store=store, layer_base=layer_base), mode=mode)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(21)
    xs = torch.randn((N_TOK, H), device="cuda", generator=gen)
    st.reset_caches()
    st.reset_stats()
    rec = []
    for t in range(N_TOK):
        if graph and t == 1:
            st.capture_graph()
        st.decode_token(xs[t])
        torch.cuda.synchronize()
        rec.append({"ids": st.ids.cpu().numpy().copy(), "scores": st.scores.cpu().numpy().view(np.uint16).copy(),
                    "pred": st.pred.cpu().numpy().copy(), "xb": st.xb.cpu().numpy().view(np.uint16).copy(),
                    "hs": st.hs.cpu().numpy().copy(),
                    "slots": {l: st.slot_inds[l][:st.cfg.top_k].cpu().numpy().copy() for l in range(1, N_LAYERS)}})
    stats = {l: st.layer_stats(l) for l in range(1, N_LAYERS)}
    return st, rec, stats


def _experts_fn(mlx):
    return lambda e: tuple((w[e], s[e], b[e]) for (w, s, b) in mlx)


def test_checkpoint_stack_matches_oracle(model_dir):
    root, experts, routers = model_dir
    st, rec, stats = _run(root, "device")
    try:
        c = st.cfg
        assert (c.n_layers, c.n_exp, c.hidden, c.inter) == (N_LAYERS, N_EXP, H, I)
        assert all(st.capacities[l] == 16 for l in range(1, N_LAYERS))
        assert st.table_status() == {}
        W = {l: q2.dequantize(*routers[l], 8, 64, "bf16") for l in range(N_LAYERS)}
        for t in (0, N_TOK - 1):
            r = rec[t]
            for l in range(N_LAYERS):
                x = q2.to_f64(r["xb"][l], "bf16")
                if l > 0:
                    want_xb = q2.round_bf16_once(q2.rmsnorm(r["hs"][l - 1].astype(np.float64), 1.0, c.eps))
                    assert np.array_equal(r["xb"][l], want_xb), (t, l)
                logits = q2.round_to(x @ W[l].T, "bf16")
                ids, sc, _ = q2.route(logits[None], c.top_k, "bf16")
                assert r["ids"][l].tolist() == ids[0].astype(np.int64).tolist(), (t, l)
                assert np.array_equal(q2.to_f64(r["scores"][l], "bf16"), sc[0]), (t, l)
                if l + 1 < N_LAYERS:
                    want_p = q2.predict_topm(q2.round_to(x @ W[l + 1].T, "bf16")[None], c.top_m)
                    assert r["pred"][l].tolist() == want_p[0].tolist(), (t, l)
                xf = x.astype(np.float16).astype(np.float64)   # the experts' fp16 copy of x
                want = q2.moe_combine(xf, ids[0], sc[0], _experts_fn(experts[l]), bits=2, group=64, sdtype="bf16")
                assert_close_rms(r["hs"][l].astype(np.float64) - xf, want, 1e-2, f"t{t} l{l}")
        lay = {l: olru.CLru(20 + l, st.capacities[l], expert_bytes=st.blob_bytes) for l in range(1, N_LAYERS)}
        for L in lay.values():
            L.reset_cache()
            L.reset_stats()
        for t in range(N_TOK):
            r = rec[t]
            lay[1].prefetch(r["pred"][0].tolist(), c.prefetch_cap)
            for l in range(1, N_LAYERS):
                slots, _ = lay[l].step(r["ids"][l].tolist())
                assert slots == r["slots"][l].tolist(), (t, l)
                if l + 1 < N_LAYERS:
                    lay[l + 1].prefetch(r["pred"][l].tolist(), c.prefetch_cap)
        for l in range(1, N_LAYERS):
            assert lay[l].stats() == stats[l], l
        for l in range(1, N_LAYERS):                   # every slot row holds its expert's 9 tensors
            e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
            st.L.c_layer_get_lru_state(st.cidx(l), e, s, ctypes.byref(n))
            lay_l = st.store.layout[l]
            for t_i, role in enumerate(lay_l["roles"]):
                pool = st.pools[l][t_i].cpu().numpy()
                arr = experts[l][role // 3][role % 3]
                for i in range(n.value):
                    assert np.array_equal(pool[s[i]], np.ascontiguousarray(arr[e[i]]).view(np.uint8).ravel()), (l, role)
    finally:
        st.close()


def test_checkpoint_stack_drivers_agree(model_dir):
    root, _, _ = model_dir
    runs = {}
    for key, kw in (("device", dict(mode="device")), ("graph", dict(mode="device", graph=True)),
                    ("host", dict(mode="host")), ("file", dict(mode="host", store="file"))):
        st, rec, stats = _run(root, **kw)
        st.close()
        runs[key] = (rec, stats)
    ref_rec, ref_stats = runs["device"]
    for key, (rec, stats) in runs.items():
        assert stats == ref_stats, key
        for t in range(N_TOK):
            for f in ("ids", "scores", "pred", "xb"):
                assert np.array_equal(rec[t][f], ref_rec[t][f]), (key, t, f)
            for l in range(1, N_LAYERS):
                assert np.array_equal(rec[t]["slots"][l], ref_rec[t]["slots"][l]), (key, t, l)


def test_cached_switch_glu_from_shard_path(model_dir):
    """CachedSwitchGLU(path, layer, capacity), the reference's construction (loader.py:311,
    1045-1046): decode steps read their misses from the shard in place and match the oracle."""
    from moe_offload.loader import CachedSwitchGLU
    root, experts, _ = model_dir
    layer = 2
    mod = CachedSwitchGLU(root / f"experts-{layer:02d}.safetensors", layer, 16)
    try:
        assert (mod.hidden, mod.inter, mod.group) == (H, I, 64)
        rng = np.random.default_rng(5)
        for t in range(4):
            ids = rng.choice(N_EXP, 10, replace=False)
            x = rng.standard_normal(H).astype(np.float16)
            out = mod(torch.from_numpy(x).cuda().reshape(1, 1, H), torch.from_numpy(ids).reshape(1, 1, 10))
            torch.cuda.synchronize()
            got = out.reshape(10, H).float().cpu().numpy()
            f = _experts_fn(experts[layer])
            for j, e in enumerate(ids):
                want = q2.switch_glu_expert(x.astype(np.float64), *f(int(e)), bits=2, group=64, sdtype="bf16")
                assert_close_rms(got[j].astype(np.float64), want, 1e-2, f"t{t} e{e}")
        st = mod.get_layer_stats()
        assert st["decode_requests"] == 40 and st["decode_demand_misses"] > 0
    finally:
        mod.close()


def test_offload_engine_over_model_directory(model_dir, tmp_path):
    from moe_offload.loader import OffloadEngine
    root, _, _ = model_dir
    eng = OffloadEngine(model_path=root, budget_pct=20.0)
    try:
        assert eng.model.cfg.n_layers == N_LAYERS and eng.total_cached_slots == 16 * (N_LAYERS - 1)
        assert eng.layer0_pinned_bytes == N_EXP * 1_536_000
        res = eng.generate_greedy("hello", max_new_tokens=16, reset_cache_before=True, reset_stats_before=True)
        for key in ("decode_tok_per_s", "prompt_effective_hit_rate", "first_window_tok_per_s", "steady_window_tok_per_s",
                    "step_latencies_ms"):
            assert key in res
        stats = eng.collect_stats(16)
        assert stats["decode_aggregate"]["total_requests"] == 16 * (N_LAYERS - 1) * 10
    finally:
        eng.close()
    with pytest.raises(FileNotFoundError):
        OffloadEngine(model_path=tmp_path / "no-model")


def test_resident_checkpoint_stack_equals_cached(model_dir):
    """Every layer in HBM (the 8-bit router's logits, gate/up selecting the experts itself, down)
    gives the cached device-driven stack's tokens bit for bit, eager and graph-replayed: the same
    selection code, the same weights, the same kernels' arithmetic."""
    from moe_offload.ckpt import CheckpointStack, CkptConfig
    root, _, _ = model_dir
    st, rec, _ = _run(root, "device")
    st.close()
    for graph in (False, True):
        rs = CheckpointStack(root, CkptConfig(), mode="device", resident=True)
        try:
            gen = torch.Generator(device="cuda")
            gen.manual_seed(21)
            xs = torch.randn((N_TOK, H), device="cuda", generator=gen)
            for t in range(N_TOK):
                if graph and t == 1:
                    rs.capture_graph()
                rs.decode_token(xs[t])
                torch.cuda.synchronize()
                assert np.array_equal(rs.ids.cpu().numpy(), rec[t]["ids"]), (graph, t)
                assert np.array_equal(rs.scores.cpu().numpy().view(np.uint16), rec[t]["scores"]), (graph, t)
                assert np.array_equal(rs.xb.cpu().numpy().view(np.uint16), rec[t]["xb"]), (graph, t)
        finally:
            rs.close()


def test_synthetic_checkpoint_resident_and_cached_agree():
    """The synthetic source (the checkpoint's shapes generated on the GPU, for 48-layer measurements):
    cached (16-slot pools fed from pinned host memory) and resident stacks built from the same seed
    give bit-identical tokens, and a sampled layer matches the oracle given its own input."""
    from moe_offload.ckpt import CheckpointStack, CkptConfig, SyntheticCheckpoint
    n_layers, E, Hs, Is = 4, 64, 1024, 320
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    xs = torch.randn((4, Hs), device="cuda", generator=gen)
    out = {}
    for resident in (False, True):
        st = CheckpointStack(cfg=CkptConfig(), synthetic=SyntheticCheckpoint(n_layers, E, Hs, Is, seed=9),
                             resident=resident)
        try:
            rec = []
            for t in range(4):
                st.decode_token(xs[t])
                torch.cuda.synchronize()
                rec.append((st.ids.cpu().numpy().copy(), st.xb.cpu().numpy().copy(), st.hs.cpu().numpy().copy(),
                            st.scores.cpu().numpy().view(np.uint16).copy()))
            if resident:                              # oracle at layer 2 of the last token
                l = 2
                ids, xb, hs, sc = rec[-1]
                codes, scales, biases = (a.cpu().numpy() for a in st.routers[l])
                W = q2.dequantize(codes.view(np.uint32), scales.view(np.uint16), biases.view(np.uint16), 8, 64, "bf16")
                x = q2.to_f64(xb[l].view(np.uint16), "bf16")
                want_i, want_s, _ = q2.route(q2.round_to(x @ W.T, "bf16")[None], 10, "bf16")
                assert ids[l].tolist() == want_i[0].astype(np.int64).tolist()
                assert np.array_equal(q2.to_f64(sc[l], "bf16"), want_s[0])
                t9 = [t.cpu().numpy() for t in st.full[l][0]]
                shapes = [(Is, Hs), (Is, Hs), (Hs, Is)]
                mlx = []
                for p, (o, i_) in enumerate(shapes):
                    w = t9[3 * p].view(np.uint32).reshape(E, o, i_ // 16)
                    s_ = t9[3 * p + 1].view(np.uint16).reshape(E, o, i_ // 64)
                    b_ = t9[3 * p + 2].view(np.uint16).reshape(E, o, i_ // 64)
                    mlx.append((w, s_, b_))
                xf = x.astype(np.float16).astype(np.float64)
                want = q2.moe_combine(xf, want_i[0], want_s[0], _experts_fn(mlx), bits=2, group=64, sdtype="bf16")
                assert_close_rms(hs[l].astype(np.float64) - xf, want, 1e-2, "synthetic layer 2")
            out[resident] = rec
        finally:
            st.close()
    for t in range(4):
        for a, b in zip(out[False][t], out[True][t]):
            assert np.array_equal(a, b), t
