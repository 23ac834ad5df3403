"""The numpy oracle against the reference's golden vectors and closed forms (CPU only)."""
import numpy as np
import pytest

from oracle import q2


def _bf(d, name):
    return q2.to_f64(d[name], "bf16")


def _router_w(d, prefix="moe.gate"):
    return q2.dequantize(d[f"{prefix}.weight"], d[f"{prefix}.scales"], d[f"{prefix}.biases"], 8, 64, "bf16")


@pytest.mark.parametrize("xname,iname,sname", [("moe.x_dec", "moe.inds_dec", "moe.scores_dec"),
                                               ("moe.x_pre", "moe.inds_pre", "moe.scores_pre")])
def test_router_ids_exact_against_golden(golden_moe, xname, iname, sname):
    d = golden_moe
    x = _bf(d, xname).reshape(-1, 256)
    logits = q2.round_to(x @ _router_w(d).T, "bf16")
    inds, scores, _ = q2.route(logits, 4, "bf16")
    ref_i = d[iname].reshape(-1, 4)
    assert np.array_equal(inds, ref_i), "router ids and their order must match the fixture exactly"


def test_router_scores_against_golden(golden_moe):
    """scores are bit-exact on 20 of 21 rows; the 21st (prefill row 12) is explained exactly by
    one router logit that MLX's 8-bit quantized matmul rounds one bf16 ulp below the correctly
    rounded value (0.42 ulp from the true dot product): moving that logit by one ulp makes the
    row bit-exact too."""
    d = golden_moe
    W = _router_w(d)
    rows = 0
    for xname, sname in [("moe.x_dec", "moe.scores_dec"), ("moe.x_pre", "moe.scores_pre")]:
        x = _bf(d, xname).reshape(-1, 256)
        logits = q2.round_to(x @ W.T, "bf16")
        _, scores, _ = q2.route(logits, 4, "bf16")
        ref = _bf(d, sname).reshape(-1, 4)
        ok = (scores == ref).all(axis=1)
        rows += int(ok.sum())
        for t in np.nonzero(~ok)[0]:
            assert xname == "moe.x_pre" and t == 12
            l = logits[t].copy()
            l[2] -= 2.0 ** (np.floor(np.log2(abs(l[2]))) - 7)
            _, s2, _ = q2.route(l[None], 4, "bf16")
            assert np.array_equal(s2[0], ref[t])
    assert rows == 20


def test_score_sum_rule_is_sequential(golden_moe):
    """Negative control: one exact sum rounded once reproduces fewer rows than the
    left-to-right rounded sum used by the oracle."""
    d = golden_moe
    x = _bf(d, "moe.x_pre").reshape(-1, 256)
    logits = q2.round_to(x @ _router_w(d).T, "bf16")
    inds, scores, gates = q2.route(logits, 4, "bf16")
    g = np.take_along_axis(gates, inds.astype(np.int64), -1)
    once = q2.round_to(g / q2.round_to(g.sum(-1, keepdims=True), "bf16"), "bf16")
    ref = _bf(d, "moe.scores_pre").reshape(-1, 4)
    assert (scores == ref).all(1).sum() > (once == ref).all(1).sum()


@pytest.mark.parametrize("which", ["nowrite", "write"])
def test_predictor_against_golden(golden_moe, which):
    d = golden_moe
    W = _router_w(d, "pred_next.gate")
    m = _bf(d, f"hc.r1.m_{which}").reshape(-1)
    logits = q2.round_to(m @ W.T, "bf16")
    got = q2.predict_topm(logits[None], 12).ravel()
    assert np.array_equal(got, d[f"pred_next.top12_{which}"].ravel().astype(np.int32))


def _expert(d, e):
    t = lambda p: (d[f"moe.switch_{p}.weight"][e], d[f"moe.switch_{p}.scales"][e], d[f"moe.switch_{p}.biases"][e])
    return t("gate"), t("up"), t("down")


@pytest.mark.parametrize("suffix", ["dec", "pre"])
def test_switch_glu_against_golden(golden_moe, suffix):
    """Routed SwitchGLU + weighted combine + shared expert output vs `moe.y_*`, at the
    reference's own gather_qmm-vs-dequant tolerance (test_prefill_qproj.py:106: 0.02*max|ref|)."""
    d = golden_moe
    X = _bf(d, f"moe.x_{suffix}").reshape(-1, 256)
    I = d[f"moe.inds_{suffix}"].reshape(-1, 4)
    S = _bf(d, f"moe.scores_{suffix}").reshape(-1, 4)
    SH = _bf(d, f"moe.sh_{suffix}").reshape(-1, 256)
    Y = _bf(d, f"moe.y_{suffix}").reshape(-1, 256)
    out = np.stack([q2.moe_combine(X[t], I[t], S[t], lambda e: _expert(d, e), bits=2, group=64,
                                   sdtype="bf16", act_dtype="bf16") + SH[t] for t in range(len(X))])
    err = np.abs(q2.round_to(out, "bf16") - Y).max()
    assert err <= 0.02 * np.abs(Y).max()
    # negative control: dropping the bias term breaks the match by a wide margin
    def no_bias(e):
        return tuple((w, s, np.zeros_like(b)) for (w, s, b) in _expert(d, e))
    bad = np.stack([q2.moe_combine(X[t], I[t], S[t], no_bias, bits=2, group=64, sdtype="bf16")
                    + SH[t] for t in range(len(X))])
    assert np.abs(bad - Y).max() > 5 * 0.02 * np.abs(Y).max()


def test_codes_pack_roundtrip_and_lsb_first():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 4, size=(3, 64)).astype(np.uint8)
    w = q2.pack_codes(q, 2)
    assert w.shape == (3, 4)
    assert np.array_equal(q2.unpack_codes(w, 2), q)
    # code j sits at bits 2j..2j+1: a word with only code 0 == 3 is the integer 3
    one = np.zeros((1, 16), np.uint8)
    one[0, 0] = 3
    assert q2.pack_codes(one, 2)[0, 0] == 3
    one[0, 0], one[0, 15] = 0, 1
    assert q2.pack_codes(one, 2)[0, 0] == 1 << 30


def test_dequant_closed_form():
    # W = s*q + b: for codes 0..3 in every group, the dequantised row is s*[0,1,2,3,...] + b
    q = np.tile(np.arange(4, dtype=np.uint8), 32)[None]          # 1 row, 128 inputs, 2 groups
    w = q2.pack_codes(q, 2)
    s = np.array([[0.5, -2.0]], np.float16)
    b = np.array([[1.0, 0.25]], np.float16)
    W = q2.dequantize(w, s, b, 2, 64)
    want = np.concatenate([0.5 * np.tile(np.arange(4), 16) + 1.0, -2.0 * np.tile(np.arange(4), 16) + 0.25])
    assert np.array_equal(W[0], want)
    # qmatvec == brute-force double loop
    rng = np.random.default_rng(1)
    x = rng.standard_normal(128)
    y = q2.qmatvec(x, w, s, b, 2, 64)
    assert np.isclose(y[0], sum(x[i] * want[i] for i in range(128)))


def test_topk_tie_rule_bruteforce():
    """Stable ascending order: equal values keep ascending index; at the k boundary the higher
    index wins; the predictor emits descending values, equal values in ascending index."""
    v = np.array([1.0, 3.0, 2.0, 3.0, 2.0, 0.5])
    assert q2.topk_ascending(v, 3).tolist() == [4, 1, 3]           # 2.0@4 beats 2.0@2
    assert q2.predict_topm(v[None], 3)[0].tolist() == [1, 3, 4]
    # brute force against a lexicographic (value, index) ordering on random small ties
    rng = np.random.default_rng(5)
    for _ in range(200):
        v = rng.integers(0, 4, size=9).astype(np.float64)
        k = int(rng.integers(1, 9))
        keys = sorted(range(9), key=lambda i: (v[i], i))
        assert q2.topk_ascending(v, k).tolist() == keys[-k:]
        top = keys[-k:]
        assert q2.predict_topm(v[None], k)[0].tolist() == sorted(top, key=lambda i: (-v[i], i))


def test_round_to_fp16_is_single_rounding_and_bf16_rne():
    x = np.array([1.0, 1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 65504.0, 1e-8])
    # exact ties go to even
    assert q2.round_to(x, "f16").tolist()[:3] == [1.0, 1.0, 1.0 + 2 ** -9]
    # just above a tie: one rounding goes up; rounding through float32 would land on the tie
    # and go to even (the double-rounding trap)
    y = np.array([1.0 + 2 ** -11 + 2 ** -40])
    assert q2.round_to(y, "f16")[0] == 1.0 + 2 ** -10
    assert y.astype(np.float32).astype(np.float16)[0] == 1.0
    # bf16 ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1
    assert q2.round_to(np.array([1.0 + 2 ** -8]), "bf16")[0] == 1.0
    assert q2.round_to(np.array([1.0 + 3 * 2 ** -8]), "bf16")[0] == 1.0 + 2 ** -6


def test_prefill_plan_reference_shapes():
    """Chunk/slot bookkeeping on the reference test's shapes (test_prefill_qproj.py:80-81):
    slots are ranks within each chunk, every chunk slot < capacity, the rebuilt LRU is a
    bijection with the last chunk's slots newest, and hit/miss accounting sums to M."""
    rng = np.random.default_rng(0)
    shapes = [(63, 19), (190, 55), (404, 102), (128, 33), (99, 26), (22, 9), (73, 25), (372, 102),
              (61, 17), (80, 25), (587, 102), (246, 39), (64, 16), (2000, 90), (5, 2), (1500, 102)]
    for rows, ne in shapes:
        ids = rng.permutation(np.concatenate([np.arange(ne), rng.integers(0, ne, rows - ne)]))
        prior = rng.choice(512, size=30, replace=False)
        plan = q2.prefill_plan(ids + 100, list(prior), list(range(30)), 102)
        assert plan["add_req"] == rows
        new_e, new_s = plan["new_lru"]
        assert len(set(new_s)) == len(new_s) and len(set(new_e)) == len(new_e)
        assert all(0 <= s < 102 for s in new_s)
        last = plan["chunks"][-1]
        n_last = last[1] - last[0]
        assert sorted(new_s[-n_last:]) == list(range(n_last))
        assert new_e[-n_last:] == [int(e) for e in plan["uniq"][last[0]:last[1]]]
        misses = len(set(int(e) for e in ids + 100) - set(int(p) for p in prior))
        assert plan["add_misses"] == misses and plan["add_hits"] == rows - misses
        assert q2.k_hdr(rows, 102) == max(1, min(102, max(rows, 16) // 4))


def test_prefill_plan_slot_contents_brute_force():
    """Replays the plan against a physical model of the pool (slot -> expert held) starting from
    the prior LRU: before each chunk's GEMM every chunk expert sits in the slot of its rank, a
    slot is loaded exactly when it held another expert, and the rebuilt LRU names what the
    slots hold.  A plan that reused stale slots or loaded into the wrong slot fails here."""
    rng = np.random.default_rng(1)
    for trial in range(200):
        cap = int(rng.choice([16, 24, 102]))
        n_prior = int(rng.integers(0, cap + 1))
        prior_e = [int(e) for e in rng.choice(512, size=n_prior, replace=False)]
        prior_s = [int(s) for s in rng.choice(cap, size=n_prior, replace=False)]
        m = int(rng.integers(0, 400))
        hot = rng.choice(512, size=int(rng.integers(1, 300)), replace=False)
        ids = rng.choice(hot, size=m)
        plan = q2.prefill_plan(ids, prior_e, prior_s, cap)
        held = dict(zip(prior_s, prior_e))
        for u0, u1, le, ls in plan["chunks"]:
            chunk = [int(e) for e in plan["uniq"][u0:u1]]
            want_loads = [(s, e) for s, e in enumerate(chunk) if held.get(s) != e]
            assert list(zip(ls, le)) == want_loads, trial
            for e, s in zip(le, ls):
                held[s] = e
            assert all(held[s] == e for s, e in enumerate(chunk)), trial
        new_e, new_s = plan["new_lru"]
        # stale entries (slots whose expert moved to another slot) are dropped, the rest kept
        assert all(held[s] == e for e, s in zip(new_e, new_s)), trial
        assert len(set(new_e)) == len(new_e)
        uniq = set(int(e) for e in ids)
        assert plan["add_misses"] == len(uniq - set(prior_e)) and plan["add_req"] == m


def test_round_bf16_once_against_exact_rationals():
    """q2.round_bf16_once rounds float64 to bf16 once (nearest, ties to even), checked against
    exact rational arithmetic: random values over many binades and constructed ties / near-ties,
    where a float32 step first (q2.round_to(.., 'bf16'), MLX's double rounding) differs."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    vals = list(rng.standard_normal(4000) * np.exp2(rng.integers(-20, 20, 4000)))
    for _ in range(600):                              # exact ties and one-ulp-of-f64 neighbours
        m = int(rng.integers(128, 256))               # 8 significand bits
        e = int(rng.integers(-30, 30))
        tie = (m + 0.5) * 2.0 ** e                    # halfway between two bf16 values
        vals += [tie, np.nextafter(tie, np.inf), np.nextafter(tie, -np.inf), -tie]
    # the double-rounding trap: just above a bf16 tie by less than half a float32 ulp
    for m in (129, 130, 200, 255):
        t = (m + 0.5) * 2.0 ** -3
        vals.append(t + 2.0 ** -3 * 2.0 ** -20)
    x = np.array(vals, np.float64)
    got = q2.bf16_bits_to_f32(q2.round_bf16_once(x)).astype(np.float64)

    def exact(v):
        f = Fraction(v)
        if f == 0:
            return 0.0
        sgn = -1 if f < 0 else 1
        a = abs(f)
        e = a.numerator.bit_length() - a.denominator.bit_length()
        while Fraction(2) ** e > a:
            e -= 1
        while Fraction(2) ** (e + 1) <= a:
            e += 1
        ulp = Fraction(2) ** (e - 7)                  # 8 significand bits
        lo = (a // ulp) * ulp
        d = a - lo
        if d > ulp / 2 or (d == ulp / 2 and (lo / ulp) % 2 == 1):
            lo += ulp
        return sgn * float(lo)
    want = np.array([exact(float(v)) for v in x])
    assert np.array_equal(got, want)
    dbl = q2.round_to(x, "bf16")
    assert not np.array_equal(dbl, want)              # the float32 step rounds some of them twice


def _rebuild_by_prior_recency(plan, lru_eids, capacity):
    """A plausible mistake in the LRU rebuild after prefill: untouched residents kept in their prior
    recency order (then the last chunk), instead of slot-index order as loader.py:671-680 does."""
    new_e, new_s = plan["new_lru"]
    last_len = plan["chunks"][-1][1] - plan["chunks"][-1][0]
    pos = {e: i for i, e in enumerate(lru_eids)}
    tail = [(e, s) for e, s in zip(new_e, new_s) if s < last_len]
    rest = [(e, s) for e, s in zip(new_e, new_s) if s >= last_len]
    rest.sort(key=lambda t: pos.get(t[0], -1))
    both = rest + tail
    return [e for e, _ in both], [s for _, s in both]


def test_prefill_plan_known_answers():
    """q2.prefill_plan on two cases worked by hand from loader.py:566-699 (chunk placement: chunk
    expert of rank r goes to slot r, loaded when the slot held another expert; LRU rebuilt from the
    final slot bijection with slots [last chunk length, capacity) oldest in slot order, then the
    last chunk's slots in slot order; the prefill counters).  The planted prior-recency rebuild
    fails case B."""
    # A: capacity 4, prior LRU->MRU (eid, slot) = (7, 2), (3, 0), (9, 3); slot 1 free.  Tokens
    # (5, 3), (8, 5), (1, 2): unique experts 1 2 3 5 8 -> chunks [1 2 3 5], [8].
    # chunk 0: slot0 held 3 -> load 1; slot1 free -> load 2; slot2 held 7 -> load 3 (3 left slot 0);
    #          slot3 held 9 -> load 5.   chunk 1: slot0 held 1 -> load 8.
    # final slots {0: 8, 1: 2, 2: 3, 3: 5}, last chunk length 1: LRU = slots 1 2 3, then 0.
    # counters: 6 requests; 3 was cached (1 hit); 5 missed once then hit; 1 2 8 missed: 4 misses, 2 hits.
    p = q2.prefill_plan(np.array([5, 3, 8, 5, 1, 2]), [7, 3, 9], [2, 0, 3], 4)
    assert [(u0, u1, le, ls) for u0, u1, le, ls in p["chunks"]] == [(0, 4, [1, 2, 3, 5], [0, 1, 2, 3]),
                                                                     (4, 5, [8], [0])]
    assert p["new_lru"] == ([2, 3, 5, 8], [1, 2, 3, 0])
    assert (p["add_req"], p["add_hits"], p["add_misses"]) == (6, 2, 4)
    # B: capacity 6, prior LRU->MRU (40, 5), (41, 2), (42, 4), (43, 3); slots 0 1 free.  Tokens
    # (11, 10), (10, 11): one chunk [10 11] into slots 0 1 (both loaded).  Slots 2..5 keep their
    # experts untouched and go first in slot order: 41 43 42 40, then 10 11.  4 requests, 2 misses.
    lru_e, lru_s = [40, 41, 42, 43], [5, 2, 4, 3]
    p = q2.prefill_plan(np.array([11, 10, 10, 11]), lru_e, lru_s, 6)
    assert [(u0, u1, le, ls) for u0, u1, le, ls in p["chunks"]] == [(0, 2, [10, 11], [0, 1])]
    known = ([41, 43, 42, 40, 10, 11], [2, 3, 4, 5, 0, 1])
    assert p["new_lru"] == known
    assert (p["add_req"], p["add_hits"], p["add_misses"]) == (4, 2, 2)
    assert _rebuild_by_prior_recency(p, lru_e, 6) != known          # the planted mistake is caught
    # C: a chunk expert already in its rank slot is not loaded again: capacity 4, prior (20, 0),
    # (21, 1); tokens (20, 22): chunk [20 22] -> slot 0 keeps 20, slot 1 (held 21) loads 22.
    p = q2.prefill_plan(np.array([20, 22]), [20, 21], [0, 1], 4)
    assert p["chunks"] == [(0, 2, [22], [1])]
    assert p["new_lru"] == ([20, 22], [0, 1])
    assert (p["add_req"], p["add_hits"], p["add_misses"]) == (2, 1, 1)
