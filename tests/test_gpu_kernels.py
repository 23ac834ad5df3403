"""GPU parity: router and Q2 SwitchGLU kernels against the CPU oracle (seeded inputs)."""
import numpy as np
import pytest

from helpers import E, H, I, K, assert_close_rms, experts_np, oracle_moe
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    assert torch.cuda.is_available(), "GPU tests need a GPU"
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def layer(dev):
    mlx, blobs = experts_np(E, H, I, seed=1)
    pool = torch.from_numpy(blobs).to(dev)
    return mlx, blobs, pool


def test_router_config_shape_exact(dev):
    """ids (order included), scores and the top-12 prediction are bit-exact vs the oracle."""
    from moe_offload import ops, synth
    w = synth.router_weight(E, H, seed=3)
    wn = synth.router_weight(E, H, seed=5)
    xs = synth.hidden_states(64, H, seed=4)
    wt, wnt = torch.from_numpy(w).to(dev), torch.from_numpy(wn).to(dev)
    for t in range(xs.shape[0]):
        xt = torch.from_numpy(xs[t]).to(dev)
        ids, sc, pred = ops.router(wt, K, x=xt, w_next=wnt, m=12)
        logits = q2.router_logits(xs[t], w, "f16")
        want_i, want_s, _ = q2.route(logits[None], K, "f16")
        want_p = q2.predict_topm(q2.router_logits(xs[t], wn, "f16")[None], 12)
        assert ids.cpu().numpy().astype(np.uint32).tolist() == want_i[0].tolist(), f"token {t}"
        assert sc.cpu().numpy().astype(np.float64).tolist() == want_s[0].tolist(), f"token {t}"
        assert pred.cpu().numpy().tolist() == want_p[0].tolist(), f"token {t}"


def test_router_rmsnorm_prologue_exact(dev):
    from moe_offload import ops, synth
    w = synth.router_weight(E, H, seed=3)
    rng = np.random.default_rng(8)
    nw = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float16)
    wt, nwt = torch.from_numpy(w).to(dev), torch.from_numpy(nw).to(dev)
    for t in range(16):
        h = (rng.standard_normal(H) * (1 + t)).astype(np.float32)
        x_out = torch.empty(H, dtype=torch.float16, device=dev)
        ids, sc, _ = ops.router(wt, K, h=torch.from_numpy(h).to(dev), norm_w=nwt, eps=1e-6, x_out=x_out)
        xn = q2.round_to(q2.rmsnorm(h.astype(np.float64), nw, 1e-6), "f16")
        assert np.array_equal(x_out.cpu().numpy().astype(np.float64), xn)
        want_i, want_s, _ = q2.route(q2.router_logits(xn, w, "f16")[None], K, "f16")
        assert ids.cpu().numpy().tolist() == want_i[0].astype(np.int64).tolist()
        assert np.array_equal(sc.cpu().numpy().astype(np.float64), want_s[0])


@pytest.mark.parametrize("n_exp,hidden,k,m", [(16, 256, 4, 6), (100, 520, 8, 12), (200, 2048, 10, 12),
                                             (1024, 2048, 16, 32), (512, 4096, 10, 12)])
def test_router_shapes_exact(dev, n_exp, hidden, k, m):
    """Expert counts covering 1, 2, 4 and 16 keys per lane in the selection, a hidden size that
    is not a multiple of 512 and one above 2048; both input kinds (x, and h with RMSNorm)."""
    from moe_offload import ops, synth
    w = synth.router_weight(n_exp, hidden, seed=n_exp + hidden)
    wn = synth.router_weight(n_exp, hidden, seed=n_exp + hidden + 1)
    wt, wnt = torch.from_numpy(w).to(dev), torch.from_numpy(wn).to(dev)
    rng = np.random.default_rng(n_exp)
    nw = (1.0 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)
    for t in range(4):
        if t % 2 == 0:
            xn = rng.standard_normal(hidden).astype(np.float16)
            ids, sc, pred = ops.router(wt, k, x=torch.from_numpy(xn).to(dev), w_next=wnt, m=m)
            xn = xn.astype(np.float64)
        else:
            h = (rng.standard_normal(hidden) * (1 + t)).astype(np.float32)
            x_out = torch.empty(hidden, dtype=torch.float16, device=dev)
            ids, sc, pred = ops.router(wt, k, h=torch.from_numpy(h).to(dev), norm_w=torch.from_numpy(nw).to(dev),
                                       eps=1e-6, x_out=x_out, w_next=wnt, m=m)
            xn = q2.round_to(q2.rmsnorm(h.astype(np.float64), nw, 1e-6), "f16")
            assert np.array_equal(x_out.cpu().numpy().astype(np.float64), xn), (n_exp, hidden, t)
        want_i, want_s, _ = q2.route(q2.router_logits(xn, w, "f16")[None], k, "f16")
        want_p = q2.predict_topm(q2.router_logits(xn, wn, "f16")[None], m)
        assert ids.cpu().numpy().astype(np.int64).tolist() == want_i[0].astype(np.int64).tolist(), (n_exp, hidden, t)
        assert np.array_equal(sc.cpu().numpy().astype(np.float64), want_s[0]), (n_exp, hidden, t)
        assert pred.cpu().numpy().tolist() == want_p[0].tolist(), (n_exp, hidden, t)


def test_router_ties_follow_stable_rule(dev):
    """Hand-built ties: equal gates keep ascending id and the higher id wins the k boundary;
    equal predictor logits come out in ascending id."""
    from moe_offload import ops
    w = np.zeros((E, H), np.float16)
    x = np.zeros(H, np.float16)
    x[0] = 1.0
    vals = {7: 2.0, 300: 2.0, 9: 1.5, 400: 1.5, 401: 1.5, 12: 1.0, 13: 1.0, 14: 1.0, 15: 1.0, 16: 1.0,
            17: 1.0, 18: 0.5}
    for e, v in vals.items():
        w[e, 0] = v
    wt = torch.from_numpy(w).to(dev)
    ids, sc, pred = ops.router(wt, K, x=torch.from_numpy(x).to(dev), w_next=wt, m=12)
    logits = q2.router_logits(x, w, "f16")
    want_i, want_s, _ = q2.route(logits[None], K, "f16")
    assert ids.cpu().numpy().tolist() == want_i[0].astype(np.int64).tolist()
    assert pred.cpu().numpy().tolist() == q2.predict_topm(logits[None], 12)[0].tolist()
    assert ids.cpu().numpy().tolist()[-2:] == [7, 300]


def test_switch_glu_config_shape(dev, layer):
    """Weighted SwitchGLU over 10 of 512 experts: max|err| <= 1e-2 x RMS vs the fp64 oracle."""
    from moe_offload import ops, synth
    mlx, blobs, pool = layer
    xs = synth.hidden_states(8, H, seed=11)
    rng = np.random.default_rng(12)
    worst = 0.0
    for t in range(xs.shape[0]):
        inds = rng.choice(E, size=K, replace=False).astype(np.int32)
        sc = rng.dirichlet(np.ones(K)).astype(np.float16)
        y = ops.q2_switch_glu(torch.from_numpy(xs[t]).to(dev), pool, torch.from_numpy(inds).to(dev), H, I,
                              scores=torch.from_numpy(sc).to(dev), residual=torch.from_numpy(xs[t]).to(dev))
        want = oracle_moe(xs[t], inds, sc, mlx, residual=xs[t])
        worst = max(worst, assert_close_rms(y.cpu().numpy(), want, 1e-2, f"token {t}"))
    print(f"worst max|err|/RMS = {worst:.2e}")


def test_switch_glu_per_expert_and_gate_up(dev, layer):
    from moe_offload import ops, synth
    mlx, blobs, pool = layer
    x = synth.hidden_states(1, H, seed=21)[0]
    inds = np.array([5, 511, 0, 17, 256, 3, 4, 100, 200, 300], np.int32)
    xt = torch.from_numpy(x).to(dev)
    slots = torch.from_numpy(inds).to(dev)
    h = ops.q2_gate_up(xt, pool, slots, H, I).view(K, I).float().cpu().numpy()
    y = ops.q2_switch_glu(xt, pool, slots, H, I, per_expert=True).cpu().numpy()
    from helpers import expert_fn
    f = expert_fn(mlx)
    for j, e in enumerate(inds):
        g, u, d = f(int(e))
        gg = q2.qmatvec(x.astype(np.float64), *g, 2, 64)
        uu = q2.qmatvec(x.astype(np.float64), *u, 2, 64)
        hh = q2.silu(gg) * uu
        assert_close_rms(h[j], hh, 4e-3, f"h expert {e}")  # h is stored as fp16
        assert_close_rms(y[j], q2.qmatvec(hh, *d, 2, 64), 1e-2, f"y expert {e}")


@pytest.mark.parametrize("k", [1, 7, 8, 9, 16])
def test_down_every_expert_count(dev, layer, k):
    """The down kernel deals expert j to wave j mod 8 of its block: with k <= 8 some waves have no
    expert, with k = 9..16 some have two, at 16 every wave has two.  Each of its three outputs
    against the fp64 oracle: the weighted sum plus residual, every expert's row, and the weighted
    sum added to a y that already holds values (the second half of a hit/miss split)."""
    from moe_offload import ops, synth
    from helpers import expert_fn
    mlx, blobs, pool = layer
    x = synth.hidden_states(1, H, seed=40 + k)[0]
    rng = np.random.default_rng(41 + k)
    inds = rng.choice(E, size=k, replace=False).astype(np.int32)
    sc = rng.dirichlet(np.ones(k)).astype(np.float16)
    xt, slots, st = torch.from_numpy(x).to(dev), torch.from_numpy(inds).to(dev), torch.from_numpy(sc).to(dev)
    h = ops.q2_gate_up(xt, pool, slots, H, I)
    y = ops.q2_down(h, pool, slots, H, I, scores=st, residual=xt).cpu().numpy()
    assert_close_rms(y, oracle_moe(x, inds, sc, mlx, residual=x), 1e-2, f"k={k} weighted")
    yk = ops.q2_down(h, pool, slots, H, I, per_expert=True).cpu().numpy()
    f = expert_fn(mlx)
    for j, e in enumerate(inds):
        want = q2.switch_glu_expert(x.astype(np.float64), *f(int(e)), bits=2, group=64)
        assert_close_rms(yk[j], want, 1e-2, f"k={k} expert {e}")
    base = np.linspace(-1.0, 1.0, H).astype(np.float32)
    y2 = torch.from_numpy(base.copy()).to(dev)
    ops.q2_down(h, pool, slots, H, I, scores=st, per_expert=2, out=y2)
    got = y2.cpu().numpy().astype(np.float64) - base
    assert_close_rms(got, oracle_moe(x, inds, sc, mlx), 1e-2, f"k={k} added")


def test_switch_glu_golden_fixture_shapes(dev, golden_moe):
    """The reference's own 16-expert fixture (hidden 256, inter 128, top-4): the routed part of
    moe.y_dec / moe.y_pre (golden minus the golden shared-expert output) within the reference's
    gather_qmm tolerance 0.02*max|ref| (test_prefill_qproj.py:106)."""
    from moe_offload import ops, q2format
    d = golden_moe
    bf = lambda n: q2.to_f64(d[n], "bf16")
    def proj(p):
        return (d[f"moe.switch_{p}.weight"], bf(f"moe.switch_{p}.scales").astype(np.float16),
                bf(f"moe.switch_{p}.biases").astype(np.float16))
    g, u, dn = proj("gate"), proj("up"), proj("down")
    # bf16 -> fp16 is exact for these values
    assert np.array_equal(g[1].astype(np.float64), bf("moe.switch_gate.scales"))
    blobs = q2format.to_blobs(g, u, dn, 256, 128)
    pool = torch.from_numpy(blobs).to(dev)
    for suffix in ("dec", "pre"):
        X = bf(f"moe.x_{suffix}").reshape(-1, 256).astype(np.float16)
        IDS = d[f"moe.inds_{suffix}"].reshape(-1, 4).astype(np.int32)
        S = bf(f"moe.scores_{suffix}").reshape(-1, 4).astype(np.float16)
        Y = bf(f"moe.y_{suffix}").reshape(-1, 256) - bf(f"moe.sh_{suffix}").reshape(-1, 256)
        for t in range(X.shape[0]):
            y = ops.q2_switch_glu(torch.from_numpy(X[t]).to(dev), pool, torch.from_numpy(IDS[t]).to(dev), 256, 128,
                                  scores=torch.from_numpy(S[t]).to(dev)).cpu().numpy()
            full = bf(f"moe.y_{suffix}").reshape(-1, 256)[t]
            assert np.abs(y - Y[t]).max() <= 0.02 * np.abs(full).max() + 1e-4


def test_f64_to_f16_single_rounding(dev):
    """The kernels' f64 -> f16 rounding equals numpy's (one round-to-nearest-even) on exact
    ties, values one f64 ulp either side of ties, subnormals, the overflow edge and random
    values."""
    from moe_offload import _lib
    rng = np.random.default_rng(3)
    h = rng.integers(0, 0x7C00, size=20000).astype(np.uint16).view(np.float16).astype(np.float64)
    nxt = np.nextafter(h.astype(np.float16), np.float16(np.inf)).astype(np.float64)
    mid = (h + nxt) / 2
    vals = np.concatenate([h, mid, np.nextafter(mid, np.inf), np.nextafter(mid, -np.inf),
                           rng.standard_normal(20000) * 10.0 ** rng.integers(-9, 5, 20000),
                           [65504.0, 65519.99, 65520.0, 2.0 ** -25, 2.0 ** -24 * 1.5, 0.0, -0.0, 1e-300]])
    vals = np.concatenate([vals, -vals])
    src = torch.from_numpy(vals).to(dev)
    out = torch.empty(vals.size, dtype=torch.int16, device=dev)
    assert _lib.lib().moe_f64_to_f16(src.data_ptr(), out.data_ptr(), vals.size,
                                     torch.cuda.current_stream().cuda_stream) == 0
    got = out.cpu().numpy().view(np.uint16)
    want = vals.astype(np.float16).view(np.uint16)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(vals[i], hex(got[i]), hex(want[i])) for i in bad[:5]]
