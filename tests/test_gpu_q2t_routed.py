"""GPU: the routed tensor-form gate/up (moe_q2t_gate_up_routed: the selection of the checkpoint's
8-bit router inside the gate/up blocks, loader.py:903-908 in bf16) selects exactly what
moe_router_q8 selects in route mode (ids, order, bf16 scores) and computes exactly
moe_q2t_gate_up's h for those ids; the ids and scores are the oracle's; equal logits order by id."""
import numpy as np
import pytest

from helpers import experts_bf16
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _dev(a, dt):
    return torch.from_numpy(np.ascontiguousarray(a).view(dt)).cuda()


def _bf16(v):
    return q2.f32_to_bf16_bits(np.asarray(v, np.float32))


def _pools(mlx):
    import ctypes
    ts = []
    for w, s, b in mlx:
        ts += [_dev(w, np.int32), _dev(s, np.int16), _dev(b, np.int16)]
    u64_9 = ctypes.c_uint64 * 9
    return ts, u64_9(*[t.data_ptr() for t in ts]), u64_9(*[t[0].numel() * t.element_size() for t in ts])


def _router(rng, E, H, equal_rows=False):
    rows = 1 if equal_rows else E
    codes = rng.integers(0, 2**32, size=(rows, H // 4), dtype=np.uint32)
    scales = _bf16(rng.standard_normal((rows, H // 64)) * 2e-4)
    biases = _bf16(-128 * q2.to_f64(scales, "bf16") + rng.standard_normal((rows, H // 64)) * 1e-4)
    if equal_rows:
        codes, scales, biases = (np.repeat(a, E, axis=0) for a in (codes, scales, biases))
    return codes, scales, biases


def _both(L, xb, x16, router, pools, E, H, I, k):
    """(ids, score bits, h) of moe_router_q8 route mode + moe_q2t_gate_up, and of moe_router_q8
    logits mode + moe_q2t_gate_up_routed; plus the logits."""
    from moe_offload import _lib
    s = torch.cuda.current_stream().cuda_stream
    codes, scales, biases = router
    ws = torch.zeros(int(L.moe_router_q8_workspace_bytes(E)), dtype=torch.uint8, device="cuda")
    ts, ptrs, nbytes = pools
    ids_a = torch.zeros(k, dtype=torch.int32, device="cuda")
    sc_a = torch.zeros(k, dtype=torch.int16, device="cuda")
    _lib.check(L.moe_router_q8(xb.data_ptr(), codes.data_ptr(), scales.data_ptr(), biases.data_ptr(), H, E, 64, k, 0,
                               ws.data_ptr(), ids_a.data_ptr(), sc_a.data_ptr(), None, None, s), "router_q8 route")
    h_a = torch.zeros(k * I, dtype=torch.float16, device="cuda")
    _lib.check(L.moe_q2t_gate_up(x16.data_ptr(), ptrs, nbytes, 1, E, ids_a.data_ptr(), k, H, I, 64, h_a.data_ptr(), s),
               "q2t_gate_up")
    lg = torch.zeros(E, dtype=torch.int16, device="cuda")
    _lib.check(L.moe_router_q8(xb.data_ptr(), codes.data_ptr(), scales.data_ptr(), biases.data_ptr(), H, E, 64, 0, 0,
                               ws.data_ptr(), None, None, None, lg.data_ptr(), s), "router_q8 logits")
    ids_b = torch.full((k,), -1, dtype=torch.int32, device="cuda")
    sc_b = torch.zeros(k, dtype=torch.int16, device="cuda")
    h_b = torch.full((k * I,), float("nan"), dtype=torch.float16, device="cuda")
    _lib.check(L.moe_q2t_gate_up_routed(x16.data_ptr(), lg.data_ptr(), E, k, ptrs, nbytes, 1, H, I, 64,
                                        ids_b.data_ptr(), sc_b.data_ptr(), h_b.data_ptr(), s), "q2t_gate_up_routed")
    torch.cuda.synchronize()
    return (ids_a, sc_a, h_a), (ids_b, sc_b, h_b), lg.cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("E,H,I,k,equal", [(64, 2560, 640, 10, False), (128, 2048, 512, 10, False),
                                           (24, 1024, 320, 16, False), (40, 2560, 640, 10, True)])
def test_routed_tensor_form_matches_router_and_gate_up(E, H, I, k, equal):
    from moe_offload import _lib
    L = _lib.lib()
    rng = np.random.default_rng(E + H + k)
    mlx = experts_bf16(E, H, I, seed=E + I)
    pools = _pools(mlx)
    router_np = _router(rng, E, H, equal_rows=equal)
    router = (_dev(router_np[0], np.int32), _dev(router_np[1], np.int16), _dev(router_np[2], np.int16))
    W = q2.dequantize(*router_np, 8, 64, "bf16")
    for t in range(4):
        xbits = _bf16(rng.standard_normal(H))
        x = q2.to_f64(xbits, "bf16")
        xb = _dev(xbits, np.int16)
        x16 = torch.from_numpy(x.astype(np.float16)).cuda()
        a, b, lg = _both(L, xb, x16, router, pools, E, H, I, k)
        assert torch.equal(a[0], b[0]), f"token {t}: ids {a[0].tolist()} vs {b[0].tolist()}"
        assert torch.equal(a[1], b[1]), f"token {t}: scores"
        assert torch.equal(a[2], b[2]), f"token {t}: h"
        logits = q2.round_to(x @ W.T, "bf16")
        assert np.array_equal(q2.to_f64(lg, "bf16"), logits)
        want_i, want_s, _ = q2.route(logits[None], k, "bf16")
        assert b[0].cpu().numpy().astype(np.int64).tolist() == want_i[0].astype(np.int64).tolist(), t
        assert np.array_equal(q2.to_f64(b[1].cpu().numpy().view(np.uint16), "bf16"), want_s[0]), t
        if equal:                                    # every gate equal: the k highest ids, ascending
            assert b[0].cpu().numpy().tolist() == list(range(E - k, E))


def test_routed_tensor_form_rejects_bad_arguments():
    from moe_offload import _lib
    L = _lib.lib()
    E, H, I = 8, 256, 64
    mlx = experts_bf16(E, H, I, seed=1)
    ts, ptrs, nbytes = _pools(mlx)
    x = torch.zeros(H, dtype=torch.float16, device="cuda")
    lg = torch.zeros(E, dtype=torch.int16, device="cuda")
    ids = torch.zeros(16, dtype=torch.int32, device="cuda")
    sc = torch.zeros(16, dtype=torch.int16, device="cuda")
    h = torch.zeros(16 * I, dtype=torch.float16, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    call = lambda n_exp, k, hidden=H, lgp=lg.data_ptr(): L.moe_q2t_gate_up_routed(
        x.data_ptr(), lgp, n_exp, k, ptrs, nbytes, 1, hidden, I, 64, ids.data_ptr(), sc.data_ptr(), h.data_ptr(), s)
    def rejects(what, *a, **kw):                      # the library keeps the first failure until cleared
        L.c_clear_error()
        assert call(*a, **kw) == -1 and what in _lib.last_error(), _lib.last_error()
    rejects("n_exp", E, 9)                            # k > n_exp
    rejects("n_exp", 2000, 4)                         # more experts than the selection holds
    rejects("null", E, 4, lgp=None)
    rejects("hidden", E, 4, hidden=100)               # not a multiple of 64
    L.c_clear_error()
    assert call(E, 4) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_routed_tensor_form_gate_ties_from_distinct_logits(seed):
    """bf16 logits packed into a band of adjacent values, so that distinct logits round to equal
    bf16 gates around the k boundary: the blocks' logit ranking gives way to the rule's own
    selection where the two can differ.  Ids, order and bf16 scores are the oracle's, h is
    moe_q2t_gate_up's for those ids."""
    from moe_offload import _lib
    L = _lib.lib()
    E, H, I, k = 512, 2560, 640, 10
    rng = np.random.default_rng(100 + seed)
    mlx = experts_bf16(E, H, I, seed=21)
    ts, ptrs, nbytes = _pools(mlx)
    base = 0x3E80 + 16 * seed                                   # bf16 0.25 and above
    lg = np.full(E, _bf16(-6.0), dtype=np.uint16)
    band = rng.choice(E, size=40, replace=False)
    lg[band] = (base + rng.integers(0, 10, size=40)).astype(np.uint16)
    logits = _dev(lg, np.int16)
    x16 = torch.from_numpy(q2.to_f64(_bf16(rng.standard_normal(H)), "bf16").astype(np.float16)).cuda()
    s = torch.cuda.current_stream().cuda_stream
    ids = torch.full((k,), -1, dtype=torch.int32, device="cuda")
    sc = torch.zeros(k, dtype=torch.int16, device="cuda")
    h = torch.zeros(k * I, dtype=torch.float16, device="cuda")
    _lib.check(L.moe_q2t_gate_up_routed(x16.data_ptr(), logits.data_ptr(), E, k, ptrs, nbytes, 1, H, I, 64,
                                        ids.data_ptr(), sc.data_ptr(), h.data_ptr(), s), "q2t_gate_up_routed")
    torch.cuda.synchronize()
    want_i, want_s, _ = q2.route(q2.to_f64(lg, "bf16")[None], k, "bf16")
    assert ids.cpu().numpy().astype(np.int64).tolist() == want_i[0].astype(np.int64).tolist()
    assert np.array_equal(q2.to_f64(sc.cpu().numpy().view(np.uint16), "bf16"), want_s[0])
    ids_o = torch.from_numpy(want_i[0].astype(np.int32)).cuda()
    h_ref = torch.zeros(k * I, dtype=torch.float16, device="cuda")
    _lib.check(L.moe_q2t_gate_up(x16.data_ptr(), ptrs, nbytes, 1, E, ids_o.data_ptr(), k, H, I, 64, h_ref.data_ptr(), s),
               "q2t_gate_up")
    torch.cuda.synchronize()
    assert torch.equal(h_ref, h)
