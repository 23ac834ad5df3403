"""OffloadEngine (loader.py:1004-1343), the engine the reference's bench and server drive, over a
4-layer stack: generate_greedy's keys and windows, collect_stats against the per-layer counters and
the decode totals (_snapshot_decode_totals, loader.py:1120-1123), set_prefetch turning prefetch
hits off, reset_stats / reset_caches, with a pinned host store (device- and host-driven) and with
the on-disk tier (device-driven: the feeder thread)."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, K = 4, 10


def _check_run(eng, out, n_tok):
    assert out["decode_tokens"] == n_tok and len(out["step_latencies_ms"]) == n_tok
    assert out["first_window_tokens"] + out["steady_window_tokens"] == n_tok
    for key in ("prompt_pure_lru_hit_rate", "prompt_effective_hit_rate", "first_window_pure_hit_rate",
                "steady_window_effective_hit_rate"):
        assert 0.0 <= out[key] <= 1.0, key
    assert out["prompt_pure_lru_hit_rate"] <= out["prompt_effective_hit_rate"]
    assert out["decode_tok_per_s"] > 0


def _engine_checks(eng):
    n_tok = 12
    eng.reset_caches()
    eng.reset_stats()
    t0 = eng._snapshot_decode_totals()
    assert t0 == (0, 0, 0, 0, 0, 0)
    out = eng.generate_greedy("hello", max_new_tokens=n_tok)
    _check_run(eng, out, n_tok)
    tot = eng._snapshot_decode_totals()
    st = eng.collect_stats(n_tok)
    agg = st["decode_aggregate"]
    assert len(st["per_layer"]) == N_LAYERS - 1
    assert agg["total_requests"] == tot[3] == n_tok * (N_LAYERS - 1) * K
    assert (agg["lru_hits"], agg["prefetch_hits"], agg["demand_misses"]) == tot[:3]
    assert agg["lru_hits"] + agg["prefetch_hits"] + agg["demand_misses"] == agg["total_requests"]
    assert (agg["demand_bytes_read"], agg["prefetch_bytes_read"]) == tot[4:6]
    assert agg["demand_bytes_read"] == agg["demand_misses"] * eng.model.blob_bytes
    assert out["prompt_effective_hit_rate"] == pytest.approx(agg["effective_hit_rate"], abs=1e-4)
    assert st["budget_summary"]["total_cached_slots"] == sum(eng.capacities.values())
    # prefetch off: no prefetch hits or bytes from here on
    eng.set_prefetch(False)
    eng.reset_stats()
    out2 = eng.generate_greedy("hello again", max_new_tokens=8)
    _check_run(eng, out2, 8)
    tot2 = eng._snapshot_decode_totals()
    assert tot2[1] == 0 and tot2[5] == 0 and tot2[3] == 8 * (N_LAYERS - 1) * K
    assert eng.collect_stats(8)["budget_summary"]["prefetch_cap"] == 0
    if eng.model.mode == "device":
        assert eng.model.table_status() == {}


@pytest.mark.parametrize("mode", ["device", "host"])
def test_engine_pinned_store(mode):
    from moe_offload.loader import OffloadEngine
    print(f"engine: pinned store, mode={mode}", flush=True)
    eng = OffloadEngine(n_layers=N_LAYERS, mode=mode, seed=3)
    try:
        _engine_checks(eng)
    finally:
        eng.close()


def test_engine_on_disk_tier(tmp_path):
    from moe_offload import q2format
    from moe_offload.loader import OffloadEngine
    from moe_offload.stack import StackConfig, random_blobs
    c = StackConfig()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(7)
    blobs = random_blobs(c.n_exp, c.hidden, c.inter, c.group, gen, "cuda").cpu().numpy()
    path = tmp_path / "experts.q2blob"
    q2format.write_blob_file(path, blobs, c.hidden, c.inter)
    print("engine: on-disk tier, device-driven", flush=True)
    eng = OffloadEngine(n_layers=N_LAYERS, mode="device", seed=3, store_file=str(path))
    try:
        _engine_checks(eng)
        for l in range(1, N_LAYERS):                # every slot holds the expert its table names
            import ctypes
            e, s, n = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
            eng.model.L.c_layer_get_lru_state(eng.model.cidx(l), e, s, ctypes.byref(n))
            pool = eng.model.pools[l].cpu().numpy()
            for i in range(n.value):
                assert np.array_equal(pool[s[i]], blobs[e[i]]), (l, e[i], s[i])
    finally:
        eng.close()
