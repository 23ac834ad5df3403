"""GPU parity of the 48-layer decode stack at its full size: 48 layers, hidden 2048, 512 experts,
top-10, inter 512, 102-slot pools (20% cache) with layer 0 pinned, misses staged from the pinned
host store, next-layer prefetch top-12 cap 3, 128 tokens, device-driven tables, graph replay.

* every layer's id and prediction stream, replayed through the oracle LRU in the reference's call
  order (prefetch(1) after layer 0, then step(l) and prefetch(l+1); loader.py:920-977), gives
  the same slots at every (token, layer) and the same 18 counters per layer and decode totals;
* at 10 sampled (token, layer) points the layer matches the oracle given the GPU's own input to
  it (teacher forcing): RMSNorm and router ids / scores / prediction bit-exact, SwitchGLU plus
  residual within 1e-2 x RMS of the fp64 oracle.
"""
import numpy as np
import pytest

from helpers import assert_close_rms
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, N_TOK = 48, 128
SAMPLES = [(0, 0), (0, 1), (0, 47), (19, 9), (37, 30), (64, 24), (90, 5), (90, 46), (127, 23), (127, 47)]


@pytest.fixture(scope="module")
def full_run():
    from moe_offload.stack import DecodeStack, StackConfig
    cfg = StackConfig(n_layers=N_LAYERS, seed=11, layer_base=0)
    print("[c3-full] building the 48-layer stack", flush=True)
    st = DecodeStack(cfg, mode="device")
    try:
        assert all(st.capacities[l] == 102 for l in range(1, N_LAYERS))
        gen = torch.Generator(device="cuda")
        gen.manual_seed(2024)
        xs = torch.randn((N_TOK, cfg.hidden), device="cuda", generator=gen).half()
        st.reset_caches()
        st.reset_stats()
        st.capture_graph()
        want_tok = {t for t, _ in SAMPLES}
        ids, pred, slots, keep = [], [], [], {}
        for t in range(N_TOK):
            st.decode_token(xs[t])
            ids.append(st.ids.cpu().numpy().copy())
            pred.append(st.pred.cpu().numpy().copy())
            slots.append(np.stack([st.slot_inds[l][:cfg.top_k].cpu().numpy() for l in range(1, N_LAYERS)]))
            if t in want_tok:
                keep[t] = (st.xs.cpu().numpy().copy(), st.hs.cpu().numpy().copy(), st.scores.cpu().numpy().copy())
            if t % 32 == 31:
                print(f"[c3-full] {t + 1} tokens decoded", flush=True)
        stats = {l: st.layer_stats(l) for l in range(1, N_LAYERS)}
        totals = st.decode_totals()
        yield st, np.stack(ids), np.stack(pred), np.stack(slots), keep, stats, totals
    finally:
        st.close()


def test_full_stack_slots_and_counters_match_oracle_lru(full_run):
    st, ids, pred, slots, _, stats, totals = full_run
    c = st.cfg
    lay = {l: olru.CLru(l, st.capacities[l], expert_bytes=st.blob_bytes) for l in range(1, N_LAYERS)}
    for L in lay.values():
        L.reset_cache()
        L.reset_stats()
    misses = 0
    for t in range(N_TOK):
        lay[1].prefetch(pred[t, 0].tolist(), c.prefetch_cap)
        for l in range(1, N_LAYERS):
            got, pairs = lay[l].step(ids[t, l].tolist())
            misses += len(pairs)
            assert got == slots[t, l - 1].tolist(), (t, l)
            if l + 1 < N_LAYERS:
                lay[l + 1].prefetch(pred[t, l].tolist(), c.prefetch_cap)
    for l in range(1, N_LAYERS):
        assert lay[l].stats() == stats[l], l
    want_tot = [0] * 6
    for l in range(1, N_LAYERS):
        s = stats[l]
        for i, w in enumerate((1, 2, 3, 0, 4, 5)):
            want_tot[i] += s[w]
    assert totals == want_tot
    assert misses > 47 * 102                 # far beyond the cold start: the pools turned over


def test_full_stack_layers_match_oracle_teacher_forced(full_run):
    from moe_offload import q2format
    st, ids, pred, _, keep, _, _ = full_run
    c = st.cfg
    W = st.router_w.cpu().numpy()
    NW = st.norm_w.cpu().numpy()
    for t, l in SAMPLES:
        xs, hs, scores = keep[t]
        x = xs[l]
        if l > 0:
            want_x = q2.round_to(q2.rmsnorm(hs[l - 1].astype(np.float64), NW[l - 1], c.eps), "f16")
            assert np.array_equal(x.astype(np.float64), want_x), (t, l)
        want_i, want_s, _ = q2.route(q2.router_logits(x, W[l], "f16")[None], c.top_k, "f16")
        assert ids[t, l].tolist() == want_i[0].astype(np.int64).tolist(), (t, l)
        assert np.array_equal(scores[l].astype(np.float64), want_s[0]), (t, l)
        if l + 1 < N_LAYERS:
            want_p = q2.predict_topm(q2.router_logits(x, W[l + 1], "f16")[None], c.top_m)
            assert pred[t, l].tolist() == want_p[0].tolist(), (t, l)
        if l == 0:
            blobs = {int(e): st.pool0[int(e)].cpu().numpy() for e in want_i[0]}
        else:
            view = st.store.view(l)
            blobs = {int(e): view[int(e)] for e in want_i[0]}
        experts = lambda e: q2format.from_blob(blobs[int(e)], c.hidden, c.inter, c.group)
        want = q2.moe_combine(x.astype(np.float64), want_i[0], want_s[0], experts, bits=2, group=64)
        assert_close_rms(hs[l].astype(np.float64) - x.astype(np.float64), want, 1e-2, f"t{t} l{l}")
        print(f"[c3-full] token {t} layer {l}: oracle parity ok", flush=True)
