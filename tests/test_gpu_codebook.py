"""GPU parity of the 2-bit codebook experts (moe_cb_up / moe_cb_down / moe_cb_moe).

At the Nemotron-style shape (hidden 3072, intermediate 1536, top-9) and at small and maximum
shapes, the kernels' outputs match the fp64 oracle (oracle/codebook.py): within 1e-3 x RMS of the
oracle that rounds h to bf16 as the kernels store it, and within 1e-2 x RMS of the oracle without
that rounding.  Per-expert rows, the score-weighted combine with a residual, and an out-of-range
slot (contributes zero) are checked.  The reference runs this path only inside llama.cpp (not
vendored): parity against the reference itself is unpinned.
"""
import numpy as np
import pytest

from helpers import assert_close_rms
from oracle import codebook as cbo

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def random_pool(n_exp, hidden, inter, seed, d_scale=0.01):
    """Random blobs: any byte is a valid code byte; the two scale planes get |N(0, d_scale)|."""
    from moe_offload import cbformat
    o = cbformat.blob_offsets(hidden, inter)
    rng = np.random.default_rng(seed)
    blobs = rng.integers(0, 256, size=(n_exp, o["bytes"]), dtype=np.uint8)
    nd = (o["bytes"] - o["up_d"]) // 2
    d = np.abs(rng.standard_normal((n_exp, nd)) * d_scale).astype(np.float16)
    blobs[:, o["up_d"]:] = d.view(np.uint8).reshape(n_exp, -1)
    return blobs


@pytest.fixture(scope="module")
def grid_dev():
    from moe_offload import cbformat
    return torch.from_numpy(cbformat.grid()).cuda()


def run_case(grid_dev, n_exp, hidden, inter, k, seed, slots=None, residual=True):
    from moe_offload import cbformat, ops
    blobs = random_pool(n_exp, hidden, inter, seed)
    pool = torch.from_numpy(blobs).cuda()
    rng = np.random.default_rng(seed + 1)
    ids = rng.choice(n_exp, size=k, replace=False) if slots is None else np.asarray(slots)
    scores = rng.random(k).astype(np.float16)
    x = rng.standard_normal(hidden).astype(np.float16)
    res = rng.standard_normal(hidden).astype(np.float16) if residual else None
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    y = ops.cb_moe(t(x), pool, t(ids.astype(np.int32)), grid_dev, hidden, inter, scores=t(scores),
                   residual=t(res) if residual else None)
    yp = ops.cb_moe(t(x), pool, t(ids.astype(np.int32)), grid_dev, hidden, inter, per_expert=True)
    torch.cuda.synchronize()
    grid = cbformat.grid()
    experts = lambda e: cbformat.from_blob(blobs[e], hidden, inter)
    valid = [j for j in range(k) if ids[j] < n_exp]
    return (x, ids, scores, res, y.cpu().numpy().astype(np.float64), yp.cpu().numpy().astype(np.float64),
            experts, grid, valid)


def test_codebook_moe_at_the_nemotron_shape(grid_dev):
    x, ids, scores, res, y, yp, experts, grid, _ = run_case(grid_dev, 24, 3072, 1536, 9, seed=3)
    for j in (0, 4, 8):
        up, down = experts(int(ids[j]))
        assert_close_rms(yp[j], cbo.expert(x, up, down, grid, h_bf16=True), 1e-3, f"expert {j} (bf16 h)")
        assert_close_rms(yp[j], cbo.expert(x, up, down, grid), 1e-2, f"expert {j} (fp64)")
    want_b = cbo.moe_combine(x, ids, scores, experts, grid, residual=res, h_bf16=True)
    want = cbo.moe_combine(x, ids, scores, experts, grid, residual=res)
    assert_close_rms(y, want_b, 1e-3, "combine (bf16 h)")
    assert_close_rms(y, want, 1e-2, "combine (fp64)")


# k covers every remainder of k mod 4: the down kernel gives its 4 waves whole experts in rounds of
# four and deals the remaining experts' row halves round robin (k = 1..3 are remainders only)
@pytest.mark.parametrize("hidden,inter,k", [(256, 256, 1), (512, 256, 16), (1024, 768, 5), (4096, 2048, 12),
                                            (256, 256, 2), (256, 256, 3), (512, 512, 6), (512, 512, 7),
                                            (768, 512, 10), (768, 512, 11), (1024, 256, 14), (1024, 256, 15)])
def test_codebook_moe_shapes(grid_dev, hidden, inter, k):
    x, ids, scores, res, y, yp, experts, grid, _ = run_case(grid_dev, k + 2, hidden, inter, k, seed=hidden + k)
    want = cbo.moe_combine(x, ids, scores, experts, grid, residual=res, h_bf16=True)
    assert_close_rms(y, want, 1e-3, f"{hidden}x{inter} k={k}")
    for j in (0, k - 1):                                 # per-expert rows: first and last expert
        up, down = experts(int(ids[j]))
        assert_close_rms(yp[j], cbo.expert(x, up, down, grid, h_bf16=True), 1e-3, f"expert {j}")


def test_codebook_out_of_range_slot_contributes_zero(grid_dev):
    slots = [3, 999, 5]
    x, ids, scores, res, y, yp, experts, grid, valid = run_case(grid_dev, 8, 512, 256, 3, seed=9, slots=slots,
                                                                residual=False)
    assert (yp[1] == 0).all()
    want = cbo.moe_combine(x, [3, 5], [scores[0], scores[2]], experts, grid, h_bf16=True)
    assert_close_rms(y, want, 1e-3, "combine without the invalid slot")


def test_codebook_rejects_bad_shapes(grid_dev):
    from moe_offload import _lib
    L = _lib.lib()
    pool = torch.zeros((2, 1 << 20), dtype=torch.uint8, device="cuda")
    s = torch.zeros(2, dtype=torch.int32, device="cuda")
    x = torch.zeros(3072, dtype=torch.float16, device="cuda")
    h = torch.zeros((2, 1536), dtype=torch.bfloat16, device="cuda")
    assert L.moe_cb_up(x.data_ptr(), pool.data_ptr(), pool.shape[1], 2, s.data_ptr(), 2, 3072, 1536,
                       grid_dev.data_ptr(), h.data_ptr(), 0) == -1          # stride < blob bytes
    assert "stride" in _lib.last_error()
    L.c_clear_error()
    assert L.moe_cb_up(x.data_ptr(), pool.data_ptr(), pool.shape[1], 2, s.data_ptr(), 2, 3000, 1536,
                       grid_dev.data_ptr(), h.data_ptr(), 0) == -1          # not a multiple of 256
    L.c_clear_error()


@pytest.mark.parametrize("hidden,inter,k,with_w", [(3072, 1536, 9, True), (1024, 512, 4, False), (4096, 2048, 16, True)])
def test_norm_fused_layer_equals_rmsnorm_then_moe(grid_dev, hidden, inter, k, with_w):
    """moe_cb_moe_norm (RMSNorm inside the up-projection) gives bit for bit the x of moe_rmsnorm
    (and the oracle's fp64 norm rounded once) and the y of moe_cb_moe on that x."""
    import ctypes

    from moe_offload import _lib
    from oracle import q2
    L = _lib.lib()
    n_exp = 24
    pool = torch.from_numpy(random_pool(n_exp, hidden, inter, seed=hidden + k)).cuda()
    rng = np.random.default_rng(k)
    ids = torch.from_numpy(rng.choice(n_exp, size=k, replace=False).astype(np.int32)).cuda()
    scores = torch.from_numpy(rng.random(k).astype(np.float16)).cuda()
    h = torch.from_numpy((rng.standard_normal(hidden) * 3).astype(np.float32)).cuda()
    w = torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)).cuda() if with_w else None
    wp = w.data_ptr() if with_w else None
    stride = pool.shape[1]
    s = torch.cuda.current_stream().cuda_stream
    eps = 1e-6
    x_ref = torch.zeros(hidden, dtype=torch.float16, device="cuda")
    y_ref = torch.zeros(hidden, dtype=torch.float32, device="cuda")
    ws = torch.zeros(k * inter, dtype=torch.bfloat16, device="cuda")
    _lib.check(L.moe_rmsnorm(h.data_ptr(), wp, eps, hidden, x_ref.data_ptr(), s), "rmsnorm")
    _lib.check(L.moe_cb_moe(x_ref.data_ptr(), pool.data_ptr(), stride, n_exp, ids.data_ptr(), scores.data_ptr(), k,
                            hidden, inter, grid_dev.data_ptr(), x_ref.data_ptr(), ws.data_ptr(), y_ref.data_ptr(), 0,
                            s), "cb_moe")
    for rep in range(2):                                  # the second call overwrites the first's outputs
        x = torch.full((hidden,), float("nan"), dtype=torch.float16, device="cuda")
        y = torch.full((hidden,), float("nan"), dtype=torch.float32, device="cuda")
        ws2 = torch.zeros(k * inter, dtype=torch.bfloat16, device="cuda")
        _lib.check(L.moe_cb_moe_norm(h.data_ptr(), wp, ctypes.c_float(eps), x.data_ptr(), pool.data_ptr(), stride,
                                     n_exp, ids.data_ptr(), scores.data_ptr(), k, hidden, inter, grid_dev.data_ptr(),
                                     ws2.data_ptr(), y.data_ptr(), s), "cb_moe_norm")
        torch.cuda.synchronize()
        assert torch.equal(x.view(torch.int16), x_ref.view(torch.int16)), rep
        assert torch.equal(ws2.view(torch.int16), ws.view(torch.int16)), rep
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)), rep
    w64 = w.cpu().numpy() if with_w else np.ones(hidden, np.float16)
    want_x = q2.round_to(q2.rmsnorm(h.cpu().numpy().astype(np.float64), w64, eps), "f16")
    assert np.array_equal(x.cpu().numpy().astype(np.float64), want_x)


def test_norm_fused_layer_rejects_bad_arguments(grid_dev):
    import ctypes

    from moe_offload import _lib
    L = _lib.lib()
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda")
    p = buf.data_ptr()
    s = torch.cuda.current_stream().cuda_stream
    f = ctypes.c_float(1e-6)
    assert L.moe_cb_moe_norm(p, None, f, None, p, 4096, 4, p, p, 4, 1024, 512, grid_dev.data_ptr(), p, p, s) == -1
    assert L.moe_cb_moe_norm(None, None, f, p, p, 4096, 4, p, p, 4, 1024, 512, grid_dev.data_ptr(), p, p, s) == -1
    assert L.moe_cb_moe_norm(p, None, f, p, p, 4096, 4, p, p, 4, 1000, 512, grid_dev.data_ptr(), p, p, s) == -1
    L.c_clear_error()
