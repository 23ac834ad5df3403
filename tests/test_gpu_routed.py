"""GPU: the resident path's split router (moe_router_logits + moe_q2_gate_up_routed, the selection
inside gate/up's blocks) selects exactly what moe_router selects (ids, order, scores; loader.py:
903-908) and computes exactly moe_q2_gate_up's h; the resident stack gives bit-identical tokens
either way, eager and graph-replayed."""
import numpy as np
import pytest

from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _pool(n_exp, hidden, inter, seed):
    from moe_offload import q2format, synth
    gate, up, down = synth.q2_experts(n_exp, hidden, inter, seed=seed)
    return torch.from_numpy(q2format.to_blobs(gate, up, down, hidden, inter)).cuda()


def _both(L, w, hidden, inter, n_exp, k, pool, x=None, h=None, nw=None):
    from moe_offload import _lib, ops
    s = torch.cuda.current_stream().cuda_stream
    xa = x if h is None else torch.empty(hidden, dtype=torch.float16, device="cuda")
    ids_a, sc_a, _ = ops.router(w, k, x=x, h=h, norm_w=nw, eps=1e-6, x_out=None if h is None else xa)
    h_a = ops.q2_gate_up(xa, pool, ids_a, hidden, inter)
    logits = torch.empty(n_exp, dtype=torch.float32, device="cuda")
    xb = torch.empty(hidden, dtype=torch.float16, device="cuda") if h is not None else None
    _lib.check(L.moe_router_logits(h.data_ptr() if h is not None else None, nw.data_ptr() if nw is not None else None,
                                   1e-6, x.data_ptr() if x is not None else None, xb.data_ptr() if xb is not None else None,
                                   w.data_ptr(), hidden, n_exp, logits.data_ptr(), s), "router_logits")
    xg = x if x is not None else xb
    ids_b = torch.empty(k, dtype=torch.int32, device="cuda")
    sc_b = torch.empty(k, dtype=torch.float16, device="cuda")
    h_b = torch.empty(k * inter, dtype=torch.float16, device="cuda")
    _lib.check(L.moe_q2_gate_up_routed(xg.data_ptr(), logits.data_ptr(), n_exp, k, pool.data_ptr(), pool.shape[1],
                                       hidden, inter, 64, ids_b.data_ptr(), sc_b.data_ptr(), h_b.data_ptr(), s),
               "gate_up_routed")
    torch.cuda.synchronize()
    if xb is not None:
        assert torch.equal(xa, xb), "RMSNorm output"
    return (ids_a, sc_a, h_a), (ids_b, sc_b, h_b), logits


@pytest.mark.parametrize("n_exp,hidden,inter,k", [(512, 2048, 512, 10), (100, 512, 256, 8), (1024, 1024, 128, 16),
                                                  (16, 256, 128, 4), (64, 2048, 64, 1)])
def test_routed_matches_router_and_gate_up(n_exp, hidden, inter, k):
    from moe_offload import _lib, synth
    L = _lib.lib()
    pool = _pool(n_exp, hidden, inter, seed=n_exp + k)
    w = torch.from_numpy(synth.router_weight(n_exp, hidden, seed=3)).cuda()
    rng = np.random.default_rng(hidden + k)
    nw = torch.from_numpy((1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)).cuda()
    for t in range(12):
        if t % 2 == 0:
            x = torch.from_numpy(rng.standard_normal(hidden).astype(np.float16)).cuda()
            a, b, logits = _both(L, w, hidden, inter, n_exp, k, pool, x=x)
            want = q2.router_logits(x.cpu().numpy(), w.cpu().numpy(), "f16")
        else:
            h = torch.from_numpy((rng.standard_normal(hidden) * (1 + t)).astype(np.float32)).cuda()
            a, b, logits = _both(L, w, hidden, inter, n_exp, k, pool, h=h, nw=nw)
            xn = q2.round_to(q2.rmsnorm(h.cpu().numpy().astype(np.float64), nw.cpu().numpy(), 1e-6), "f16")
            want = q2.router_logits(xn, w.cpu().numpy(), "f16")
        assert np.array_equal(logits.cpu().numpy().astype(np.float64), want), f"token {t}: logits"
        assert torch.equal(a[0], b[0]), f"token {t}: ids {a[0].tolist()} vs {b[0].tolist()}"
        assert torch.equal(a[1], b[1]), f"token {t}: scores"
        assert torch.equal(a[2].view(-1), b[2]), f"token {t}: h"


def test_routed_selection_ties():
    """Hand-built equal gates at the k boundary: the higher id wins, as in moe_router."""
    from moe_offload import _lib, synth
    L = _lib.lib()
    n_exp, hidden, inter, k = 512, 2048, 512, 10
    pool = _pool(n_exp, hidden, inter, seed=7)
    w = synth.router_weight(n_exp, hidden, seed=3)
    x = synth.hidden_states(1, hidden, seed=4)[0]
    w[:, :] = 0
    w[:, 0] = np.float16(0.01) * (np.arange(n_exp) % 7).astype(np.float16)   # many exact ties
    x[0] = np.float16(1.0)
    a, b, _ = _both(L, torch.from_numpy(w).cuda(), hidden, inter, n_exp, k, pool, x=torch.from_numpy(x).cuda())
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2].view(-1), b[2])


def test_resident_stack_routed_equals_router_path():
    from moe_offload.stack import DecodeStack, StackConfig
    outs = {}
    for routed in (True, False):
        for graph in (False, True):
            cfg = StackConfig(n_layers=4, seed=5, resident=True, prefetch=False, routed_glu=routed)
            st = DecodeStack(cfg, mode="device")
            gen = torch.Generator(device="cuda")
            gen.manual_seed(11)
            xs = torch.randn((6, cfg.hidden), device="cuda", generator=gen).half()
            if graph:
                st.capture_graph()
            rec = []
            for t in range(6):
                st.decode_token(xs[t])
                torch.cuda.synchronize()
                rec.append((st.ids.cpu().clone(), st.scores.cpu().clone(), st.xs.cpu().clone(), st.hs.cpu().clone()))
            outs[(routed, graph)] = rec
            st.close()
            del st
            torch.cuda.empty_cache()
    ref = outs[(False, False)]
    for key, rec in outs.items():
        for t in range(6):
            for a, b in zip(rec[t], ref[t]):
                assert torch.equal(a, b), f"{key} token {t}"



@pytest.mark.parametrize("n_exp,k,peaks", [(512, 10, {5: 30.0, 200: 25.0}), (16, 16, {3: 30.0}), (100, 12, {99: 40.0})])
def test_peaked_softmax_selects_zero_gates_by_descending_id(n_exp, k, peaks):
    """A router whose softmax rounds all but one or two gates to fp16 zero: the other picks are
    zero-gate experts, whose keys are their ids alone, taken by descending id (down to expert 0,
    whose key equals the padding's, when k = n_exp).  The router's last block and the routed
    gate/up both give the oracle's ids, scores and next-layer predictions (ties of equal logits)."""
    from moe_offload import _lib, ops
    L = _lib.lib()
    hidden, inter = 256, 64
    pool = _pool(n_exp, hidden, inter, seed=n_exp)
    w = np.zeros((n_exp, hidden), np.float16)
    for e, v in peaks.items():
        w[e, 0] = v
    x = np.zeros(hidden, np.float16)
    x[0] = 1.0
    wt, xt = torch.from_numpy(w).cuda(), torch.from_numpy(x).cuda()
    a, b, logits = _both(L, wt, hidden, inter, n_exp, k, pool, x=xt)
    want_i, want_s, _ = q2.route(q2.router_logits(x, w, "f16")[None], k, "f16")
    zero = sorted(e for e in range(n_exp) if e not in peaks)[n_exp - len(peaks) - (k - len(peaks)):]
    assert sorted(e for e in want_i[0].tolist() if e not in peaks) == zero      # the oracle's own rule
    if k == n_exp:
        assert 0 in want_i[0].tolist()
    assert a[0].cpu().numpy().astype(np.int64).tolist() == want_i[0].astype(np.int64).tolist()
    assert np.array_equal(a[1].cpu().numpy().astype(np.float64), want_s[0])
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1]) and torch.equal(a[2].view(-1), b[2])
    m = min(12, n_exp)
    _, _, pred = ops.router(wt, k, x=xt, w_next=wt, m=m)
    want_p = q2.predict_topm(q2.router_logits(x, w, "f16")[None], m)
    assert pred.cpu().numpy().tolist() == want_p[0].tolist()


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_routed_selection_gate_ties_from_distinct_logits(seed):
    """Logits packed into a narrow band of adjacent fp16 values, so that distinct logits round to
    equal fp16 gates around the k boundary and inside the top k: the gate/up blocks first rank by
    logit, and where that ranking and the rule's (gate, then id) can differ they take the rule's
    own selection.  Ids, order and scores are the oracle's, h is moe_q2_gate_up's for those ids."""
    from moe_offload import _lib, ops
    L = _lib.lib()
    n_exp, hidden, inter, k = 512, 2048, 512, 10
    pool = _pool(n_exp, hidden, inter, seed=11)
    rng = np.random.default_rng(seed)
    base = np.float16(0.25 + 0.05 * seed)
    lg = np.full(n_exp, np.float16(-6.0), dtype=np.float16)
    band = rng.choice(n_exp, size=40, replace=False)
    steps = rng.integers(0, 12, size=40)                       # adjacent fp16 values, some repeated
    lg[band] = (base.view(np.uint16) + steps.astype(np.uint16)).view(np.float16)
    logits = torch.from_numpy(lg.astype(np.float32)).cuda()
    x = torch.from_numpy(rng.standard_normal(hidden).astype(np.float16)).cuda()
    ids = torch.empty(k, dtype=torch.int32, device="cuda")
    sc = torch.empty(k, dtype=torch.float16, device="cuda")
    h = torch.empty(k * inter, dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(L.moe_q2_gate_up_routed(x.data_ptr(), logits.data_ptr(), n_exp, k, pool.data_ptr(), pool.shape[1],
                                       hidden, inter, 64, ids.data_ptr(), sc.data_ptr(), h.data_ptr(), s),
               "gate_up_routed")
    torch.cuda.synchronize()
    want_i, want_s, _ = q2.route(lg.astype(np.float64)[None], k, "f16")
    assert ids.cpu().numpy().astype(np.int64).tolist() == want_i[0].astype(np.int64).tolist()
    assert np.array_equal(sc.cpu().numpy().astype(np.float64), want_s[0])
    h_ref = ops.q2_gate_up(x, pool, torch.from_numpy(want_i[0].astype(np.int32)).cuda(), hidden, inter)
    assert torch.equal(h_ref.view(-1), h)
