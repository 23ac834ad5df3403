"""The real checkpoint's 8-bit router and predictor (moe_router_q8) against the oracle and the
reference's own fixture.

* fixture router (16 experts, hidden 256, top-4): all 21 rows (1 decode + 20 prefill) give the
  oracle's ids, order and bf16 scores exactly; 20 of 21 are the reference's too (the 21st is the
  one where MLX's fp32-accumulating kernel rounds a logit one ulp low, as the oracle test shows);
* fixture predictor (64 experts, hidden 2560, top-12): both rows equal the reference's top-12;
* the real shape (512 experts, hidden 2560): logits bit-exact to the oracle's bf16-rounded fp64
  dot, ids / scores / predictions exact on 24 tokens; equal logits ordered by id in both modes.
"""
import numpy as np
import pytest

from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a).view(dt)).cuda()


class Q8:
    def __init__(self, codes, scales, biases):
        self.n, self.hidden = codes.shape[0], codes.shape[1] * 4
        self.c = _dev(codes.astype(np.uint32), np.int32)
        self.s = _dev(scales.astype(np.uint16), np.int16)
        self.b = _dev(biases.astype(np.uint16), np.int16)
        self.W = q2.dequantize(codes, scales, biases, 8, 64, "bf16")
        from moe_offload import _lib
        self.L = _lib.lib()
        self.ws = torch.zeros(int(self.L.moe_router_q8_workspace_bytes(self.n)), dtype=torch.uint8, device="cuda")

    def run(self, xbits, k=0, m=0):
        from moe_offload import _lib
        x = _dev(xbits.astype(np.uint16), np.int16)
        ids = torch.zeros(max(k, 1), dtype=torch.int32, device="cuda")
        sc = torch.zeros(max(k, 1), dtype=torch.int16, device="cuda")
        pred = torch.zeros(max(m, 1), dtype=torch.int32, device="cuda")
        lg = torch.zeros(self.n, dtype=torch.int16, device="cuda")
        rc = self.L.moe_router_q8(x.data_ptr(), self.c.data_ptr(), self.s.data_ptr(), self.b.data_ptr(), self.hidden,
                                  self.n, 64, k, m, self.ws.data_ptr(), ids.data_ptr(), sc.data_ptr(), pred.data_ptr(),
                                  lg.data_ptr(), torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "moe_router_q8")
        torch.cuda.synchronize()
        return (ids.cpu().numpy()[:k].astype(np.uint32), sc.cpu().numpy()[:k].view(np.uint16),
                pred.cpu().numpy()[:m], lg.cpu().numpy().view(np.uint16))

    def oracle(self, xbits, k=0, m=0):
        x = q2.to_f64(xbits, "bf16")
        logits = q2.round_to(x @ self.W.T, "bf16")
        out = {"logits": logits}
        if k:
            out["ids"], out["scores"], _ = q2.route(logits[None], k, "bf16")
        if m:
            out["pred"] = q2.predict_topm(logits[None], m)[0]
        return out


def _bf16_bits(v):
    return q2.f32_to_bf16_bits(np.asarray(v, np.float32))


def test_fixture_router(golden_moe):
    d = golden_moe
    r = Q8(d["moe.gate.weight"], d["moe.gate.scales"], d["moe.gate.biases"])
    rows = [(d["moe.x_dec"].reshape(-1, 256), d["moe.inds_dec"].reshape(-1, 4), d["moe.scores_dec"].reshape(-1, 4)),
            (d["moe.x_pre"].reshape(-1, 256), d["moe.inds_pre"].reshape(-1, 4), d["moe.scores_pre"].reshape(-1, 4))]
    agree = 0
    for X, I, S in rows:
        for t in range(X.shape[0]):
            ids, sc, _, lg = r.run(X[t], k=4)
            o = r.oracle(X[t], k=4)
            assert np.array_equal(q2.to_f64(lg, "bf16"), o["logits"]), t
            assert ids.tolist() == o["ids"][0].tolist(), t
            assert np.array_equal(q2.to_f64(sc, "bf16"), o["scores"][0]), t
            assert ids.tolist() == I[t].tolist(), t                  # ids and order: all 21 rows
            agree += int(np.array_equal(sc, S[t].astype(np.uint16)))
    assert agree == 20


@pytest.mark.parametrize("which", ["nowrite", "write"])
def test_fixture_predictor(golden_moe, which):
    d = golden_moe
    r = Q8(d["pred_next.gate.weight"], d["pred_next.gate.scales"], d["pred_next.gate.biases"])
    _, _, pred, _ = r.run(d[f"hc.r1.m_{which}"].reshape(-1), m=12)
    assert pred.tolist() == d[f"pred_next.top12_{which}"].reshape(-1).astype(np.int32).tolist()


def test_real_shape_against_oracle():
    rng = np.random.default_rng(11)
    E, H = 512, 2560
    codes = rng.integers(0, 2**32, size=(E, H // 4), dtype=np.uint32)
    scales = _bf16_bits(rng.standard_normal((E, H // 64)) * 2e-4)
    biases = _bf16_bits(-128 * q2.to_f64(scales, "bf16") + rng.standard_normal((E, H // 64)) * 1e-4)
    r = Q8(codes, scales, biases)
    for t in range(24):
        x = _bf16_bits(rng.standard_normal(H))
        ids, sc, _, lg = r.run(x, k=10)
        o = r.oracle(x, k=10, m=12)
        assert np.array_equal(q2.to_f64(lg, "bf16"), o["logits"]), t
        assert ids.tolist() == o["ids"][0].tolist(), t
        assert np.array_equal(q2.to_f64(sc, "bf16"), o["scores"][0]), t
        _, _, pred, _ = r.run(x, m=12)
        assert pred.tolist() == o["pred"].tolist(), t


def test_ties_order_by_id():
    rng = np.random.default_rng(12)
    E, H = 64, 256
    row = rng.integers(0, 2**32, size=(1, H // 4), dtype=np.uint32)
    codes = np.repeat(row, E, axis=0)
    scales = np.repeat(_bf16_bits(rng.standard_normal((1, H // 64)) * 1e-3), E, axis=0)
    biases = np.repeat(_bf16_bits(rng.standard_normal((1, H // 64)) * 1e-3), E, axis=0)
    codes[[5, 17, 40]] = codes[0] ^ 0x01010101        # three rows slightly apart, the rest all equal
    r = Q8(codes, scales, biases)
    x = _bf16_bits(rng.standard_normal(H))
    o = r.oracle(x, k=8, m=12)
    ids, sc, _, _ = r.run(x, k=8)
    assert ids.tolist() == o["ids"][0].tolist()
    assert np.array_equal(q2.to_f64(sc, "bf16"), o["scores"][0])
    _, _, pred, _ = r.run(x, m=12)
    assert pred.tolist() == o["pred"].tolist()


def test_rejects_bad_arguments():
    from moe_offload import _lib
    L = _lib.lib()
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda")
    p = buf.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    assert L.moe_router_q8(p, p, p, p, 256, 16, 32, 4, 0, p, p, p, p, p, s) == -1        # group 32
    assert L.moe_router_q8(p, p, p, p, 100, 16, 64, 4, 0, p, p, p, p, p, s) == -1        # hidden % 64
    assert L.moe_router_q8(p, p, p, p, 256, 16, 64, 4, 4, p, p, p, p, p, s) == -1        # both modes
    assert L.moe_router_q8(p, p, p, p, 256, 16, 64, 20, 0, p, p, p, p, p, s) == -1       # k > n_rows
    L.c_clear_error()


@pytest.mark.parametrize("with_w", [False, True])
def test_norm_fused_router_equals_norm_then_router(with_w):
    """moe_router_q8_norm (the bf16 RMSNorm inside the router launch) against moe_rmsnorm_bf16
    followed by moe_router_q8, at the real shape: x as bf16 and fp16, logits, ids, scores and
    predictions bit for bit, in all three modes, over h of varied magnitude."""
    from moe_offload import _lib
    rng = np.random.default_rng(13)
    E, H, eps = 512, 2560, 1e-6
    codes = rng.integers(0, 2**32, size=(E, H // 4), dtype=np.uint32)
    scales = _bf16_bits(rng.standard_normal((E, H // 64)) * 2e-4)
    biases = _bf16_bits(-128 * q2.to_f64(scales, "bf16") + rng.standard_normal((E, H // 64)) * 1e-4)
    r = Q8(codes, scales, biases)
    L, s = r.L, torch.cuda.current_stream().cuda_stream
    nw = _dev(_bf16_bits(1.0 + 0.1 * rng.standard_normal(H)), np.int16) if with_w else None
    nwp = nw.data_ptr() if with_w else None
    for t in range(6):
        h = torch.from_numpy((rng.standard_normal(H) * 10.0 ** (t - 2)).astype(np.float32)).cuda()
        xb = torch.zeros(H, dtype=torch.int16, device="cuda")
        xh = torch.zeros(H, dtype=torch.float16, device="cuda")
        _lib.check(L.moe_rmsnorm_bf16(h.data_ptr(), nwp, eps, H, xb.data_ptr(), xh.data_ptr(), s), "rmsnorm_bf16")
        torch.cuda.synchronize()
        xbits = xb.cpu().numpy().view(np.uint16)
        for k, m in ((10, 0), (0, 12), (0, 0)):
            ref = r.run(xbits, k=k, m=m)
            ids = torch.zeros(max(k, 1), dtype=torch.int32, device="cuda")
            sc = torch.zeros(max(k, 1), dtype=torch.int16, device="cuda")
            pred = torch.zeros(max(m, 1), dtype=torch.int32, device="cuda")
            lg = torch.zeros(E, dtype=torch.int16, device="cuda")
            xb2 = torch.full((H,), -1, dtype=torch.int16, device="cuda")
            xh2 = torch.full((H,), -1.0, dtype=torch.float16, device="cuda")
            rc = L.moe_router_q8_norm(h.data_ptr(), nwp, eps, xb2.data_ptr(), xh2.data_ptr(), r.c.data_ptr(),
                                      r.s.data_ptr(), r.b.data_ptr(), H, E, 64, k, m, r.ws.data_ptr(), ids.data_ptr(),
                                      sc.data_ptr(), pred.data_ptr(), lg.data_ptr(), s)
            _lib.check(rc, "moe_router_q8_norm")
            torch.cuda.synchronize()
            where = (t, k, m)
            assert torch.equal(xb2, xb) and torch.equal(xh2.view(torch.int16), xh.view(torch.int16)), where
            assert np.array_equal(lg.cpu().numpy().view(np.uint16), ref[3]), where
            assert np.array_equal(ids.cpu().numpy()[:k].astype(np.uint32), ref[0]), where
            assert np.array_equal(sc.cpu().numpy()[:k].view(np.uint16), ref[1]), where
            assert np.array_equal(pred.cpu().numpy()[:m], ref[2]), where
