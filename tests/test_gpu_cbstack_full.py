"""GPU parity of the codebook-expert (Nemotron-style) decode stack at its full size: 40 layers,
240 experts, top-9, hidden 3072, non-gated inter 1536 (squared ReLU), 2-bit codebook experts,
a 4 GiB HBM expert cache over the layers fed from the pinned host store, Zipf(1.0) routing,
64 tokens, device-driven tables, graph replay.

* every layer's id stream replayed through the oracle LRU (the reference's expert_io.c decode
  step) gives the same slots at every (token, layer) and the same 18 counters per layer;
* at 8 sampled (token, layer) points the layer matches the fp64 oracle given the GPU's own input
  (teacher forcing): RMSNorm exact, expert sum + residual within 1e-3 x RMS (bf16 h as stored).
"""
import numpy as np
import pytest

from helpers import assert_close_rms
from oracle import codebook as cbo
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_LAYERS, N_TOK = 40, 64
SAMPLES = [(0, 0), (0, 39), (13, 7), (31, 20), (40, 33), (50, 1), (63, 12), (63, 38)]


@pytest.fixture(scope="module")
def full_run():
    from moe_offload.cbstack import CbStackConfig, CodebookStack, zipf_routing
    cfg = CbStackConfig(n_layers=N_LAYERS, seed=7, layer_base=0)
    print("[c5-full] building the 40-layer codebook stack", flush=True)
    st = CodebookStack(cfg)
    try:
        ids, sc = zipf_routing(N_TOK, N_LAYERS, cfg.n_exp, cfg.top_k, cfg.zipf_s, seed=9)
        gen = torch.Generator(device="cuda")
        gen.manual_seed(31)
        xs = torch.randn((N_TOK, cfg.hidden), device="cuda", generator=gen).half()
        st.capture_graph()
        want_tok = {t for t, _ in SAMPLES}
        slots, keep = [], {}
        for t in range(N_TOK):
            st.decode_token(xs[t], torch.from_numpy(ids[t]).cuda(), torch.from_numpy(sc[t]).cuda())
            slots.append(np.stack([s[:cfg.top_k].cpu().numpy() for s in st.slot_inds]))
            if t in want_tok:
                keep[t] = (st.xs.cpu().numpy().copy(), st.hs.cpu().numpy().copy())
            if t % 16 == 15:
                print(f"[c5-full] {t + 1} tokens decoded", flush=True)
        stats = [st.layer_stats(l) for l in range(N_LAYERS)]
        yield st, ids, sc, np.stack(slots), keep, stats
    finally:
        st.close()


def test_full_codebook_stack_slots_and_counters_match_oracle_lru(full_run):
    st, ids, _, slots, _, stats = full_run
    # 4 GiB over 40 layers of 2,433,024-byte experts: 44 slots per layer
    assert st.capacity == (4 << 30) // (N_LAYERS * st.blob_bytes) == 44
    lay = [olru.CLru(l, st.capacity, expert_bytes=st.blob_bytes) for l in range(N_LAYERS)]
    for L in lay:
        L.reset_cache()
        L.reset_stats()
    misses = 0
    for t in range(N_TOK):
        for l in range(N_LAYERS):
            got, pairs = lay[l].step([int(v) for v in ids[t, l]])
            misses += len(pairs)
            assert got == slots[t, l].tolist(), (t, l)
    for l in range(N_LAYERS):
        assert lay[l].stats() == stats[l], l
    assert misses > N_LAYERS * 44              # beyond the cold start: the pools turned over


def test_full_codebook_layers_match_oracle_teacher_forced(full_run):
    from moe_offload import cbformat
    st, ids, sc, _, keep, _ = full_run
    c = st.cfg
    grid = cbformat.grid()
    nw = st.norm_w.cpu().numpy()
    for t, l in SAMPLES:
        xs, hs = keep[t]
        x = xs[l]
        if l > 0:
            want_x = q2.round_to(q2.rmsnorm(hs[l - 1].astype(np.float64), nw[l - 1], c.eps), "f16")
            assert np.array_equal(x.astype(np.float64), want_x), (t, l)
        view = st.store.view(l)
        experts = lambda e: cbformat.from_blob(view[int(e)], c.hidden, c.inter)
        want = cbo.moe_combine(x.astype(np.float64), ids[t, l], sc[t, l], experts, grid, h_bf16=True)
        assert_close_rms(hs[l].astype(np.float64) - x.astype(np.float64), want, 1e-3, f"t{t} l{l}")
        print(f"[c5-full] token {t} layer {l}: oracle parity ok", flush=True)
