"""GPU parity of the tensor-form Q2 SwitchGLU (the reference's 9 slot-pool tensors, loader.py:332-406,
read in place; bf16 or fp16 scales; any multiple-of-64 shape).

* the real model's layer shape (hidden 2560, inter 640) with bf16 scales and biases in 9 separate
  pools: combined output and every expert's output within 1e-2 x RMS of the fp64 oracle;
* the reference's own 16-expert bf16 fixture in its native format: the routed part of moe.y_dec /
  moe.y_pre within the reference's tolerance (test_prefill_qproj.py:106);
* blob pools at 2560 / 640 (the blob kernels' fallback to the tensor form) against the oracle;
* at the workload shape (2048 / 512) the tensor form and the blob kernels agree within 5e-4 x RMS
  (their fp32 gate/up sums run in different orders, so an h near an fp16 rounding boundary can
  land one ulp apart; observed 6e-5);
* a layer initialised with its 9 tensors in file-offset order, as loader.py passes them, then
  c_layer_set_format9: decode steps with staging from the host store (host and device tables) give
  the oracle's outputs and fill every slot with its expert's bytes in all 9 pools.
"""
import ctypes

import numpy as np
import pytest

from helpers import assert_close_rms, experts_bf16
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

u64_9 = ctypes.c_uint64 * 9


def _pools(mlx, dev):
    """9 device tensors in role order and their bytes per expert."""
    ts = []
    for w, s, b in mlx:
        ts += [torch.from_numpy(np.ascontiguousarray(w).view(np.int32)).to(dev),
               torch.from_numpy(np.ascontiguousarray(s).view(np.int16)).to(dev),
               torch.from_numpy(np.ascontiguousarray(b).view(np.int16)).to(dev)]
    ptrs = u64_9(*[t.data_ptr() for t in ts])
    nbytes = u64_9(*[t[0].numel() * t.element_size() for t in ts])
    return ts, ptrs, nbytes


def _fn(mlx, sdtype):
    return lambda e: tuple((p[0][e], p[1][e], p[2][e]) for p in mlx)


def _run(L, x, ptrs, nbytes, bf16, n_slots, slots, scores, k, H, I, residual=None, per_expert=0):
    from moe_offload import _lib
    dev = x.device
    h_ws = torch.empty(k * I, dtype=torch.float16, device=dev)
    y = torch.empty((k, H) if per_expert == 1 else (H,), dtype=torch.float32, device=dev)
    rc = L.moe_q2t_switch_glu(x.data_ptr(), ptrs, nbytes, bf16, n_slots, slots.data_ptr(),
                              scores.data_ptr() if scores is not None else None, k, H, I, 64,
                              residual.data_ptr() if residual is not None else None, h_ws.data_ptr(), y.data_ptr(),
                              per_expert, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_q2t_switch_glu")
    return y.cpu().numpy()


def test_real_model_shape_bf16_nine_pools():
    from moe_offload import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E, K = 2560, 640, 24, 10
    mlx = experts_bf16(E, H, I, seed=3)
    ts, ptrs, nbytes = _pools(mlx, dev)
    assert list(nbytes) == [409_600, 51_200, 51_200] * 3        # the reference's 1,536,000-byte expert
    rng = np.random.default_rng(4)
    f = _fn(mlx, "bf16")
    for t in range(4):
        x = (rng.standard_normal(H)).astype(np.float16)
        ids = rng.choice(E, size=K, replace=False).astype(np.int32)
        sc = rng.dirichlet(np.ones(K)).astype(np.float16)
        xt = torch.from_numpy(x).to(dev)
        y = _run(L, xt, ptrs, nbytes, 1, E, torch.from_numpy(ids).to(dev), torch.from_numpy(sc).to(dev), K, H, I,
                 residual=xt)
        want = q2.moe_combine(x.astype(np.float64), ids, sc.astype(np.float64), f, bits=2, group=64, sdtype="bf16")
        assert_close_rms(y, want + x.astype(np.float64), 1e-2, f"token {t}")
    # per-expert rows
    ids = np.arange(K, dtype=np.int32) * 2
    yk = _run(L, xt, ptrs, nbytes, 1, E, torch.from_numpy(ids).to(dev), None, K, H, I, per_expert=1)
    for j, e in enumerate(ids):
        want = q2.switch_glu_expert(x.astype(np.float64), *f(int(e)), bits=2, group=64, sdtype="bf16")
        assert_close_rms(yk[j], want, 1e-2, f"expert {e}")


def test_reference_fixture_in_native_bf16(golden_moe):
    from moe_offload import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    d = golden_moe
    mlx = tuple((d[f"moe.switch_{p}.weight"], d[f"moe.switch_{p}.scales"], d[f"moe.switch_{p}.biases"])
                for p in ("gate", "up", "down"))
    ts, ptrs, nbytes = _pools(mlx, dev)
    bf = lambda n: q2.to_f64(d[n], "bf16")
    for suffix in ("dec", "pre"):
        X = bf(f"moe.x_{suffix}").reshape(-1, 256).astype(np.float16)
        IDS = d[f"moe.inds_{suffix}"].reshape(-1, 4).astype(np.int32)
        S = bf(f"moe.scores_{suffix}").reshape(-1, 4).astype(np.float16)
        full = bf(f"moe.y_{suffix}").reshape(-1, 256)
        Y = full - bf(f"moe.sh_{suffix}").reshape(-1, 256)
        for t in range(X.shape[0]):
            y = _run(L, torch.from_numpy(X[t]).to(dev), ptrs, nbytes, 1, 16, torch.from_numpy(IDS[t]).to(dev),
                     torch.from_numpy(S[t]).to(dev), 4, 256, 128)
            assert np.abs(y - Y[t]).max() <= 0.02 * np.abs(full[t]).max() + 1e-4, (suffix, t)


def test_blob_pools_at_real_shape_use_tensor_kernels():
    from moe_offload import ops, q2format, synth
    from helpers import oracle_moe
    dev = torch.device("cuda")
    H, I, E, K = 2560, 640, 16, 10
    gate, up, down = synth.q2_experts(E, H, I, seed=5)
    pool = torch.from_numpy(q2format.to_blobs(gate, up, down, H, I)).to(dev)
    rng = np.random.default_rng(6)
    for t in range(3):
        x = rng.standard_normal(H).astype(np.float16)
        ids = rng.choice(E, size=K, replace=False).astype(np.int32)
        sc = rng.dirichlet(np.ones(K)).astype(np.float16)
        y = ops.q2_switch_glu(torch.from_numpy(x).to(dev), pool, torch.from_numpy(ids).to(dev), H, I,
                              scores=torch.from_numpy(sc).to(dev))
        assert_close_rms(y.cpu().numpy(), oracle_moe(x, ids, sc, (gate, up, down)), 1e-2, f"token {t}")


def test_tensor_form_agrees_with_blob_kernels_at_workload_shape():
    from moe_offload import _lib, ops, q2format, synth
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E, K = 2048, 512, 32, 10
    gate, up, down = synth.q2_experts(E, H, I, seed=7)
    pool = torch.from_numpy(q2format.to_blobs(gate, up, down, H, I)).to(dev)
    ts, ptrs, nbytes = _pools((gate, up, down), dev)
    rng = np.random.default_rng(8)
    for t in range(4):
        x = rng.standard_normal(H).astype(np.float16)
        ids = torch.from_numpy(rng.choice(E, size=K, replace=False).astype(np.int32)).to(dev)
        sc = torch.from_numpy(rng.dirichlet(np.ones(K)).astype(np.float16)).to(dev)
        xt = torch.from_numpy(x).to(dev)
        a = ops.q2_switch_glu(xt, pool, ids, H, I, scores=sc).cpu().numpy()
        b = _run(L, xt, ptrs, nbytes, 0, E, ids, sc, K, H, I)
        assert_close_rms(b, a, 5e-4, f"token {t}")


@pytest.mark.parametrize("mode", ["host", "device"])
def test_nine_tensor_layer_in_file_offset_order(mode):
    """c_layer_init with the 9 tensors in a shuffled (file-offset) order, c_layer_set_format9 with
    their roles; decode steps staged from pinned host stores."""
    from moe_offload import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E, K, cap = 2560, 640, 48, 10, 16
    layer = 44 if mode == "host" else 45
    mlx = experts_bf16(E, H, I, seed=9)
    role_arrays = []
    for w, s, b in mlx:
        role_arrays += [np.ascontiguousarray(w).view(np.uint8).reshape(E, -1),
                        np.ascontiguousarray(s).view(np.uint8).reshape(E, -1),
                        np.ascontiguousarray(b).view(np.uint8).reshape(E, -1)]
    order = [6, 0, 3, 7, 8, 1, 2, 4, 5]          # tensor t holds role order[t] (like sorted file offsets)
    host, pools = [], []
    try:
        for t, r in enumerate(order):
            a = role_arrays[r]
            p = L.c_host_alloc(a.nbytes)
            assert p
            np.ctypeslib.as_array(ctypes.cast(p, ctypes.POINTER(ctypes.c_uint8)), shape=a.shape)[:] = a
            host.append(p)
            pools.append(torch.zeros((cap, a.shape[1]), dtype=torch.uint8, device=dev))
        slots = torch.zeros(16, dtype=torch.int32, device=dev)
        L.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        L.c_layer_init(layer, -1, cap, u64_9(*host), u64_9(*[role_arrays[r].shape[1] for r in order]),
                       u64_9(*[p.data_ptr() for p in pools]), slots.data_ptr())
        _lib.check_error("c_layer_init")
        roles = (ctypes.c_int32 * 9)(*order)
        _lib.check(L.c_layer_set_format9(layer, H, I, 64, roles, 1), "set_format9")
        if mode == "device":
            _lib.check(L.c_layer_set_device_mode(layer, 1), "device_mode")
        ref = olru.PyLru(0, cap)
        rng = np.random.default_rng(10)
        stream = torch.cuda.current_stream().cuda_stream
        f = _fn(mlx, "bf16")
        h_ws = torch.empty(K * I, dtype=torch.float16, device=dev)
        y = torch.empty(H, dtype=torch.float32, device=dev)
        for step in range(12):
            ids = rng.choice(E, size=K, replace=False).astype(np.uint32)
            if mode == "host":
                n = L.c_layer_step_decode_ex(layer, (ctypes.c_uint32 * K)(*[int(v) for v in ids]), K, 1)
                _lib.check(n, "step")
            else:
                it = torch.from_numpy(ids.astype(np.int32)).to(dev)
                _lib.check(L.c_layer_step_decode_dev(layer, it.data_ptr(), K, 0, stream), "step_dev")
            x = rng.standard_normal(H).astype(np.float16)
            sc = rng.dirichlet(np.ones(K)).astype(np.float16)
            xt, sct = torch.from_numpy(x).to(dev), torch.from_numpy(sc).to(dev)
            _lib.check(L.c_layer_switch_glu(layer, xt.data_ptr(), sct.data_ptr(), None, h_ws.data_ptr(), y.data_ptr(),
                                            0, K, stream), "switch_glu")
            want_slots, _ = ref.step([int(v) for v in ids])
            assert slots[:K].cpu().tolist() == want_slots, step
            want = q2.moe_combine(x.astype(np.float64), ids, sc.astype(np.float64), f, bits=2, group=64,
                                  sdtype="bf16")
            assert_close_rms(y.cpu().numpy(), want, 1e-2, f"step {step}")
            for t, r in enumerate(order):
                got = pools[t][torch.tensor(want_slots, device=dev)].cpu().numpy()
                assert np.array_equal(got, role_arrays[r][ids.astype(np.int64)]), (step, t)
    finally:
        torch.cuda.synchronize()
        L.c_sync_copies()
        L.c_layer_init(layer, -1, 16, None, None, None, 0)
        for p in host:
            L.c_host_free(p)


def _grouped_t(L, x, row_tok, row_out, seg_start, seg_slot, ptrs, nbytes, bf16, n_slots, H, I, n_out):
    from moe_offload import _lib
    dev = x.device
    M, n_seg = row_tok.numel(), seg_start.numel() - 1
    h_ws = torch.empty((M, I), dtype=torch.float16, device=dev)
    y = torch.empty((n_out, H), dtype=torch.float16, device=dev)
    rc = L.moe_q2t_grouped_switch_glu(x.data_ptr(), x.shape[0], row_tok.data_ptr(), row_out.data_ptr(), M, n_out,
                                      seg_start.data_ptr(), seg_slot.data_ptr(), n_seg, ptrs, nbytes, bf16, n_slots, H,
                                      I, 64, h_ws.data_ptr(), y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_q2t_grouped_switch_glu")
    torch.cuda.synchronize()
    return y.cpu().numpy()


def test_grouped_tensor_form_equals_blob_kernels():
    """fp16 scales: the 9-tensor grouped path loads the same (scale, bias) values as the blob path
    and gives bit-identical outputs (512 tokens x top-10 of 64 experts, hidden 2048 / inter 512)."""
    from moe_offload import _lib, ops, prefill, q2format, synth
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E, K = 2048, 512, 64, 10
    gate, up, down = synth.q2_experts(E, H, I, seed=21)
    pool = torch.from_numpy(q2format.to_blobs(gate, up, down, H, I)).to(dev)
    ts, ptrs, nbytes = _pools((gate, up, down), dev)
    ids, _ = synth.prefill_routing(256, K, E)
    xs = synth.hidden_states(256, H, seed=22)
    row_tok, row_out, seg_start, seg_slot = prefill.resident_plan(ids, K)
    t = lambda a: torch.from_numpy(a).to(dev)
    want = ops.q2_grouped_switch_glu(t(xs), t(row_tok), t(seg_start), pool, H, I, row_out=t(row_out),
                                     n_out_rows=ids.size, seg_slot=t(seg_slot)).cpu().numpy()
    got = _grouped_t(L, t(xs), t(row_tok), t(row_out), t(seg_start), t(seg_slot), ptrs, nbytes, 0, E, H, I, ids.size)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


def test_grouped_tensor_form_bf16_real_shape():
    """bf16 scales at hidden 2560 / inter 640 (the real model's layer): every row of a subset of
    experts against the fp64 oracle within 1e-2 x RMS."""
    from moe_offload import _lib, prefill, synth
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E, K = 2560, 640, 48, 10
    mlx = experts_bf16(E, H, I, seed=23)
    ts, ptrs, nbytes = _pools(mlx, dev)
    ids, _ = synth.prefill_routing(128, K, E)
    xs = synth.hidden_states(128, H, seed=24)
    row_tok, row_out, seg_start, seg_slot = prefill.resident_plan(ids, K)
    t = lambda a: torch.from_numpy(a).to(dev)
    y = _grouped_t(L, t(xs), t(row_tok), t(row_out), t(seg_start), t(seg_slot), ptrs, nbytes, 1, E, H, I,
                   ids.size).astype(np.float64)
    flat = ids.reshape(-1)
    f = _fn(mlx, "bf16")
    counts = np.diff(seg_start)
    chosen = [int(seg_slot[np.argmax(counts)])] + [int(e) for e in np.random.default_rng(25).choice(seg_slot, 8, replace=False)]
    for e in chosen:
        pairs = np.nonzero(flat == e)[0]
        want = q2.switch_glu_expert(xs[pairs // K].astype(np.float64), *f(e), bits=2, group=64, sdtype="bf16")
        assert_close_rms(y[pairs], want, 1e-2, f"expert {e}")


@pytest.mark.parametrize("k", [1, 9, 16])
def test_tensor_form_every_expert_count(k):
    """The tensor-form down block deals expert j to wave j mod 8: one expert (seven idle waves),
    nine (one wave with two), sixteen (every wave with two), at hidden 1024 / inter 320 (5 groups
    per down row) with bf16 scales: the weighted sum with residual and every expert's row against
    the fp64 oracle."""
    from moe_offload import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    H, I, E = 1024, 320, 24
    mlx = experts_bf16(E, H, I, seed=50 + k)
    ts, ptrs, nbytes = _pools(mlx, dev)
    f = _fn(mlx, "bf16")
    rng = np.random.default_rng(51 + k)
    x = rng.standard_normal(H).astype(np.float16)
    ids = rng.choice(E, size=k, replace=False).astype(np.int32)
    sc = rng.dirichlet(np.ones(k)).astype(np.float16)
    xt = torch.from_numpy(x).to(dev)
    y = _run(L, xt, ptrs, nbytes, 1, E, torch.from_numpy(ids).to(dev), torch.from_numpy(sc).to(dev), k, H, I,
             residual=xt)
    want = q2.moe_combine(x.astype(np.float64), ids, sc.astype(np.float64), f, bits=2, group=64, sdtype="bf16")
    assert_close_rms(y, want + x.astype(np.float64), 1e-2, f"k={k} weighted")
    yk = _run(L, xt, ptrs, nbytes, 1, E, torch.from_numpy(ids).to(dev), None, k, H, I, per_expert=1)
    for j, e in enumerate(ids):
        want = q2.switch_glu_expert(x.astype(np.float64), *f(int(e)), bits=2, group=64, sdtype="bf16")
        assert_close_rms(yk[j], want, 1e-2, f"k={k} expert {e}")


@pytest.mark.parametrize("H,I", [(2560, 640), (256, 64), (512, 1024), (1024, 192), (320, 448)])
def test_down_modes_agree_across_shapes(H, I):
    """The down product's three modes at shapes that leave the row layout's last block partial
    and its lanes partly idle (inter / 64 = 1..16 groups per row): the sum (mode 0, against the
    fp64 oracle), the score-weighted sum of the per-expert rows (mode 1) equal to it within fp32
    rounding, and mode 2 adding exactly that sum to y's previous value."""
    from moe_offload import _lib
    L = _lib.lib()
    dev = torch.device("cuda")
    E, K = 12, 10
    mlx = experts_bf16(E, H, I, seed=H + I)
    ts, ptrs, nbytes = _pools(mlx, dev)
    f = _fn(mlx, "bf16")
    rng = np.random.default_rng(H * 7 + I)
    x = rng.standard_normal(H).astype(np.float16)
    ids = rng.choice(E, size=K, replace=False).astype(np.int32)
    sc = rng.dirichlet(np.ones(K)).astype(np.float16)
    xt, it, st = torch.from_numpy(x).to(dev), torch.from_numpy(ids).to(dev), torch.from_numpy(sc).to(dev)
    y0 = _run(L, xt, ptrs, nbytes, 1, E, it, st, K, H, I)
    want = q2.moe_combine(x.astype(np.float64), ids, sc.astype(np.float64), f, bits=2, group=64, sdtype="bf16")
    assert_close_rms(y0, want, 1e-2, "mode 0")
    yk = _run(L, xt, ptrs, nbytes, 1, E, it, None, K, H, I, per_expert=1)
    comb = (sc.astype(np.float64)[:, None] * yk.astype(np.float64)).sum(axis=0)
    assert np.abs(comb - y0).max() <= 1e-5 * np.abs(y0).max() + 1e-7
    base = torch.from_numpy(rng.standard_normal(H).astype(np.float32)).to(dev)
    y2 = base.clone()
    h_ws = torch.empty(K * I, dtype=torch.float16, device=dev)
    rc = L.moe_q2t_switch_glu(xt.data_ptr(), ptrs, nbytes, 1, E, it.data_ptr(), st.data_ptr(), K, H, I, 64, None,
                              h_ws.data_ptr(), y2.data_ptr(), 2, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "moe_q2t_switch_glu mode 2")
    assert np.array_equal(y2.cpu().numpy(), (base.cpu().numpy() + y0).astype(np.float32))
