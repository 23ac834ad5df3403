"""moe_router_noalloc (the router with its scratch in a static device array) against moe_router
(the same kernels with a caller workspace), through the C-ABI.

Two calls in a row, the second smaller (fewer experts, a shorter hidden vector, a smaller k and
prediction), each bit-identical to moe_router on the same inputs: ids (order included), scores,
predictions and the RMSNorm output.  A size beyond the static array is rejected with an error.
"""
import ctypes

import numpy as np
import pytest

from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def _call(lib, fn, args, ws):
    from moe_offload import _lib
    (h, nw, x, x_out, w, wn, hidden, n_exp, k, m, ids, sc, pred) = args
    s = torch.cuda.current_stream().cuda_stream
    p = lambda t: None if t is None else t.data_ptr()
    if fn == "workspace":
        rc = lib.moe_router(p(h), p(nw), 1e-6, p(x), p(x_out), p(w), p(wn), hidden, n_exp, k, m, p(ws), p(ids), p(sc),
                            p(pred), s)
    else:
        rc = lib.moe_router_noalloc(p(h), p(nw), 1e-6, p(x), p(x_out), p(w), p(wn), hidden, n_exp, k, m, p(ids),
                                    p(sc), p(pred), s)
    _lib.check(rc, fn)


def _case(dev, n_exp, hidden, k, m, seed, norm):
    rng = np.random.default_rng(seed)
    w = torch.from_numpy((rng.standard_normal((n_exp, hidden)) * 0.02).astype(np.float16)).to(dev)
    wn = torch.from_numpy((rng.standard_normal((n_exp, hidden)) * 0.02).astype(np.float16)).to(dev)
    if norm:
        h = torch.from_numpy(rng.standard_normal(hidden).astype(np.float32) * 3).to(dev)
        nw = torch.from_numpy((1 + 0.1 * rng.standard_normal(hidden)).astype(np.float16)).to(dev)
        x = None
    else:
        h = nw = None
        x = torch.from_numpy(rng.standard_normal(hidden).astype(np.float16)).to(dev)
    return h, nw, x, w, wn


def _outputs(dev, hidden, k, m):
    return (torch.full((hidden,), -1, dtype=torch.int16, device=dev).view(torch.float16),
            torch.full((k,), -1, dtype=torch.int32, device=dev),
            torch.full((k,), -1, dtype=torch.int16, device=dev).view(torch.float16),
            torch.full((m,), -1, dtype=torch.int32, device=dev))


def test_router_noalloc_matches_router_two_calls():
    from moe_offload import _lib
    assert torch.cuda.is_available()
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    # (n_exp, hidden, k, m, norm): the workload's router, then a smaller one
    for n_exp, hidden, k, m, norm in [(512, 2048, 10, 12, True), (96, 1024, 6, 8, False)]:
        print(f"[case] n_exp={n_exp} hidden={hidden} k={k} m={m} norm={norm}", flush=True)
        h, nw, x, w, wn = _case(dev, n_exp, hidden, k, m, seed=n_exp, norm=norm)
        ws = torch.zeros(int(lib.moe_router_workspace_bytes(n_exp)), dtype=torch.uint8, device=dev)
        got, want = _outputs(dev, hidden, k, m), _outputs(dev, hidden, k, m)
        _call(lib, "noalloc", (h, nw, x, got[0] if norm else None, w, wn, hidden, n_exp, k, m, *got[1:]), None)
        _call(lib, "workspace", (h, nw, x, want[0] if norm else None, w, wn, hidden, n_exp, k, m, *want[1:]), ws)
        torch.cuda.synchronize()
        for a, b, what in zip(got, want, ("x_out", "ids", "scores", "pred")):
            if what == "x_out" and not norm:
                continue
            assert torch.equal(a.view(torch.int16) if a.dtype == torch.float16 else a,
                               b.view(torch.int16) if b.dtype == torch.float16 else b), (n_exp, what)
        # and both are the oracle's selection
        xin = got[0].cpu().numpy() if norm else x.cpu().numpy()
        want_i, want_s, _ = q2.route(q2.router_logits(xin, w.cpu().numpy(), "f16")[None], k, "f16")
        assert got[1].cpu().numpy().tolist() == want_i[0].astype(np.int64).tolist()
        assert np.array_equal(got[2].cpu().numpy().astype(np.float64), want_s[0])


def test_router_noalloc_rejects_sizes_beyond_static_scratch():
    from moe_offload import _lib
    dev = torch.device("cuda:0")
    lib = _lib.lib()
    lib.c_clear_error()
    x = torch.zeros(256, dtype=torch.float16, device=dev)
    w = torch.zeros((1, 256), dtype=torch.float16, device=dev)
    ids = torch.zeros(4, dtype=torch.int32, device=dev)
    sc = torch.zeros(4, dtype=torch.float16, device=dev)
    rc = lib.moe_router_noalloc(None, None, 1e-6, x.data_ptr(), None, w.data_ptr(), None, 256, 2048, 4, 0,
                                ids.data_ptr(), sc.data_ptr(), None, torch.cuda.current_stream().cuda_stream)
    assert rc == -1
    msg = _lib.last_error()
    lib.c_clear_error()
    assert "static scratch" in msg, msg
