"""GPU parity of the prefill grouped GEMM (MFMA) and of prefill through a cached layer.

* prefill chunk shape (512 tokens x top-10 of 512 experts, long-tailed tokens per expert, max 62):
  the per-(token, k) SwitchGLU outputs of the grouped kernels against the fp64 oracle on every
  row of a subset of experts (the longest segment, single-row segments, random ones), within
  1e-2 x RMS per expert; the score-weighted combine against numpy on the same rows.
* the reference's own prefill_qproj test shapes (test_prefill_qproj.py:28-30: cache of 102
  slots, D=1024 -> O=384, (rows, experts) pairs) through the grouped down projection, with its
  criterion max|err| <= 0.02 x max|ref| per row, and the 1e-2 x RMS bar.
* a cached layer (102 slots): multi-chunk and single-chunk prefill give oracle outputs, the LRU
  state and counters of the oracle's prefill plan applied to the C LRU restatement, and decode
  afterwards makes the same slot decisions as that oracle.
* a row naming an out-of-range token computes from zeros; rows naming an out-of-range output
  row or slot are not written; the other rows are unaffected.
"""
import ctypes

import numpy as np
import pytest

from helpers import E, H, I, K, assert_close_rms, expert_fn, experts_np
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def experts(dev):
    mlx, blobs = experts_np(E, H, I, seed=11)
    return mlx, blobs, torch.from_numpy(blobs).to(dev)


def _oracle_rows(mlx, xs, rows_tok, e):
    """fp64 SwitchGLU of expert e on the given token rows -> [n, H]."""
    return q2.switch_glu_expert(xs[rows_tok].astype(np.float64), *expert_fn(mlx)(e), bits=2, group=64)


def _check_experts(y, ids, xs, mlx, chosen, k):
    flat = ids.reshape(-1)
    for e in chosen:
        pairs = np.nonzero(flat == e)[0]
        want = _oracle_rows(mlx, xs, pairs // k, e)
        assert_close_rms(y[pairs].astype(np.float64), want, 1e-2, f"expert {e} ({pairs.size} rows)")


def test_grouped_prefill_chunk_matches_oracle(dev, experts):
    from moe_offload import ops, prefill, synth
    mlx, _, pool = experts
    ids, scores = synth.prefill_routing(512, K, E)
    xs = synth.hidden_states(512, H, seed=12)
    row_tok, row_out, seg_start, seg_slot = prefill.resident_plan(ids, K)
    counts = np.diff(seg_start)
    assert counts.max() == 62 and seg_slot.size == 496
    t = lambda a: torch.from_numpy(a).to(dev)
    y = ops.q2_grouped_switch_glu(t(xs), t(row_tok), t(seg_start), pool, H, I, row_out=t(row_out),
                                  n_out_rows=ids.size, seg_slot=t(seg_slot))
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    rng = np.random.default_rng(3)
    longest = int(seg_slot[np.argmax(counts)])
    singles = [int(e) for e in seg_slot[counts == 1][:3]]
    chosen = [longest] + singles + [int(e) for e in rng.choice(seg_slot, 20, replace=False)]
    _check_experts(yh, ids, xs, mlx, chosen, K)

    # gate/up over one-tile segments (the same rows, each keeping its expert's slot): bit-identical h
    h_e = ops.q2_grouped_gate_up(t(xs), t(row_tok), t(seg_start), pool, H, I, seg_slot=t(seg_slot))
    seg_t, slot_t = prefill.tile_segments(seg_start, seg_slot)
    assert slot_t.size == int(np.sum((counts + 15) // 16))
    h_t = ops.q2_grouped_gate_up(t(xs), t(row_tok), t(seg_t), pool, H, I, seg_slot=t(slot_t))
    assert torch.equal(h_e, h_t)

    comb = ops.pair_combine(y, t(scores)).cpu().numpy()
    want = (yh.reshape(512, K, H).astype(np.float32) * scores.astype(np.float32)[..., None]).astype(np.float64)
    want = want.sum(axis=1)
    np.testing.assert_allclose(comb, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def test_grouped_down_reference_qproj_shapes(dev):
    """test_prefill_qproj.py:28-30,66-70: W [102, 384, 1024] 2-bit g64, rows sorted by slot."""
    from moe_offload import ops, q2format, synth
    cap, D, O = 102, 1024, 384
    shapes = [(63, 19), (190, 55), (404, 102), (128, 33), (99, 26), (22, 9), (73, 25), (372, 102),
              (61, 17), (80, 25), (587, 102), (246, 39), (64, 16), (2000, 90), (5, 2), (1500, 102)]
    gate, up, down = synth.q2_experts(cap, O, D, seed=21, scale_std=0.05)
    pool = torch.from_numpy(q2format.to_blobs(gate, up, down, O, D)).to(dev)
    rng = np.random.default_rng(0)
    for rows, ne in shapes:
        idx = np.sort(np.concatenate([np.arange(ne), rng.integers(0, ne, rows - ne)])).astype(np.int64)
        x = rng.standard_normal((rows, D)).astype(np.float16)
        seg = np.searchsorted(idx, np.arange(ne + 1)).astype(np.int32)
        y = ops.q2_grouped_down(torch.from_numpy(x).to(dev), torch.from_numpy(seg).to(dev), pool, O, D)
        got = y.cpu().numpy().astype(np.float64)
        want = np.empty((rows, O))
        for u in range(ne):
            r0, r1 = seg[u], seg[u + 1]
            want[r0:r1] = q2.qmatvec(x[r0:r1].astype(np.float64), down[0][u], down[1][u], down[2][u], 2, 64)
        err = np.abs(got - want).max(axis=1)
        assert (err <= 0.02 * np.abs(want).max()).all(), (rows, ne)
        assert_close_rms(got, want, 1e-2, f"rows={rows} experts={ne}")


def test_grouped_skips_out_of_range_rows(dev, experts):
    from moe_offload import ops, synth
    mlx, _, pool = experts
    xs = synth.hidden_states(4, H, seed=13)
    # segments: expert 5 (rows 0-2), slot 9999 (row 3, skipped), expert 7 (rows 4-5), empty, expert 8 (row 6)
    row_tok = np.array([0, 1, 77, 2, 3, 0, 1], np.int32)        # row 2 names token 77: zeros
    row_out = np.array([0, 1, 2, 3, 4, 99, 6], np.int32)        # row 5 writes row 99: skipped
    seg = np.array([0, 3, 4, 6, 6, 7], np.int32)
    slot = np.array([5, 9999, 7, 3, 8], np.int32)
    t = lambda a: torch.from_numpy(a).to(dev)
    y = torch.full((8, H), 7.0, dtype=torch.float16, device=dev)
    ops.q2_grouped_switch_glu(t(xs), t(row_tok), t(seg), pool, H, I, row_out=t(row_out), n_out_rows=8,
                              seg_slot=t(slot), out=y)
    yh = y.cpu().numpy().astype(np.float64)
    for r, (tok, e) in {0: (0, 5), 1: (1, 5), 4: (3, 7), 6: (1, 8)}.items():
        assert_close_rms(yh[r], _oracle_rows(mlx, xs, np.array([tok]), e)[0], 1e-2, f"row {r}")
    assert (yh[2] == 0.0).all()
    for r in (3, 5, 7):
        assert (yh[r] == 7.0).all(), f"row {r} was written"


def _lru_state(L, layer):
    e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
    L.c_layer_get_lru_state(layer, e, s, ctypes.byref(c))
    return list(e[:c.value]), list(s[:c.value])


@pytest.mark.parametrize("n_tok", [64, 8])
def test_cached_layer_prefill(dev, experts, n_tok):
    """Warm the LRU by decode, prefill n_tok tokens (64: four chunks, 8: one), then decode."""
    from moe_offload import _lib, synth
    from moe_offload.loader import CachedSwitchGLU, HostExpertStore
    mlx, blobs, _ = experts
    layer, cap = (30 if n_tok == 64 else 31), 102
    store = HostExpertStore(layer + 1, E, blobs.shape[1], first_layer=layer)
    store.view(layer)[:] = blobs
    mod = CachedSwitchGLU(store, layer, cap, H, I)
    ora = olru.CLru(layer, cap, expert_bytes=blobs.shape[1])
    ora.reset_stats()
    L = _lib.lib()
    try:
        stream_ids = synth.expert_id_stream(40, K, E, seed=9)
        for ids in stream_ids[:20]:
            mod.step([int(v) for v in ids])
            ora.step([int(v) for v in ids])
        ids, _ = synth.prefill_routing(n_tok, K, E, seed=14)
        xs = synth.hidden_states(n_tok, H, seed=15)
        e0, s0 = ora.get_state()
        assert _lru_state(L, layer) == (e0, s0)
        plan = q2.prefill_plan(ids.reshape(-1), e0, s0, cap)
        assert (len(plan["chunks"]) > 1) == (n_tok == 64)

        y = mod(torch.from_numpy(xs).to(dev)[None], torch.from_numpy(ids).to(dev)[None])
        torch.cuda.synchronize()
        assert tuple(y.shape) == (1, n_tok, K, H)
        yh = y[0].reshape(n_tok * K, H).cpu().numpy()
        rng = np.random.default_rng(5)
        uniq = np.unique(ids)
        _check_experts(yh, ids, xs, mlx, [int(e) for e in rng.choice(uniq, 12, replace=False)], K)

        for _, _, le, ls in plan["chunks"]:
            if le:
                ora.load_sync(le, ls, 1)
        ora.set_state(*plan["new_lru"], plan["add_req"], plan["add_hits"], plan["add_misses"])
        assert _lru_state(L, layer) == ora.get_state()
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        # every slot holds the expert the table says it holds
        pool = mod.pool.cpu().numpy()
        for e, s in zip(*ora.get_state()):
            assert np.array_equal(pool[s], blobs[e]), (e, s)

        for ids in stream_ids[20:]:
            mod.step([int(v) for v in ids])
            slots, _ = ora.step([int(v) for v in ids])
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        assert _lib.last_error() == ""
    finally:
        mod.close()
        store.close()


@pytest.mark.parametrize("hidden,inter", [(384, 192), (1024, 320), (128, 768), (2560, 64), (2048, 576), (384, 512),
                                          (2048, 512)])
def test_grouped_gate_up_and_down_odd_contractions(dev, hidden, inter):
    """Contraction lengths off the 256-wide chunk grid (K = 384, 192, 320, 128, 64) take the
    per-chunk scale/bias loads; multiples of 256 from 512 up (1024, 768, 2560) take the
    four-chunk blocks; gate/up at K = 2048 and down at K = 512 take the whole-K forms, here also
    with a last slice only partly in range (inter 576: half of a 128-row gate/up slice; hidden
    384: half of a 256-row down slice); all against the fp64 oracle."""
    from moe_offload import ops, q2format, synth
    n_exp, rows_per = 6, [1, 17, 40, 3, 64, 9]
    gate, up, down = synth.q2_experts(n_exp, hidden, inter, seed=hidden + inter, scale_std=0.05)
    pool = torch.from_numpy(q2format.to_blobs(gate, up, down, hidden, inter)).to(dev)
    rng = np.random.default_rng(hidden)
    n_rows = sum(rows_per)
    x = rng.standard_normal((n_rows, hidden)).astype(np.float16)
    seg = np.concatenate([[0], np.cumsum(rows_per)]).astype(np.int32)
    row_tok = np.arange(n_rows, dtype=np.int32)
    h = ops.q2_grouped_gate_up(torch.from_numpy(x).to(dev), torch.from_numpy(row_tok).to(dev),
                               torch.from_numpy(seg).to(dev), pool, hidden, inter)
    y = ops.q2_grouped_down(h, torch.from_numpy(seg).to(dev), pool, hidden, inter)
    h_got, y_got = h.cpu().numpy().astype(np.float64), y.cpu().numpy().astype(np.float64)
    for u in range(n_exp):
        r0, r1 = seg[u], seg[u + 1]
        xg = x[r0:r1].astype(np.float64)
        g = q2.qmatvec(xg, gate[0][u], gate[1][u], gate[2][u], 2, 64)
        v = q2.qmatvec(xg, up[0][u], up[1][u], up[2][u], 2, 64)
        want_h = g / (1.0 + np.exp(-g)) * v
        # h is stored in fp16: one ulp at the largest |h| on top of the 1% of RMS
        bound = 1e-2 * np.sqrt(np.mean(want_h ** 2)) + np.abs(want_h).max() * 2.0 ** -10
        err = np.abs(h_got[r0:r1] - want_h).max()
        assert err <= bound, f"gate/up expert {u} K={hidden}: max|err| {err:.3e} > {bound:.3e}"
        want_y = q2.qmatvec(h_got[r0:r1].astype(np.float16).astype(np.float64), down[0][u], down[1][u],
                            down[2][u], 2, 64)
        assert_close_rms(y_got[r0:r1], want_y, 1e-2, f"down expert {u} K={inter}")
