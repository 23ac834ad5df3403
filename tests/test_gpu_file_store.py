"""On-disk tier on the GPU: a cached layer whose misses are read from an expert blob file with
pread into a pinned bounce buffer and copied to the HBM slot pool (the reference reads its shard
the same way, `mlx-qwen38/expert_io.c:113-185`).

40 decode steps (capacity 16 over 64 experts) then an 8-token prefill: slot decisions and
counters match the oracle LRU, every slot holds the expert the table names, outputs match the
fp64 oracle within 1e-2 x RMS.
"""
import ctypes

import numpy as np
import pytest

from helpers import H, I, K, assert_close_rms, expert_fn, experts_np, oracle_moe
from oracle import lru as olru
from oracle import q2

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

N_EXP, CAP, LAYER = 64, 16, 34


def _state(L, layer):
    e, s, c = (ctypes.c_int32 * 512)(), (ctypes.c_int32 * 512)(), ctypes.c_int(0)
    L.c_layer_get_lru_state(layer, e, s, ctypes.byref(c))
    return list(e[:c.value]), list(s[:c.value])


def test_file_backed_layer(tmp_path):
    from moe_offload import _lib, q2format, synth
    from moe_offload.loader import CachedSwitchGLU, FileExpertStore
    dev = torch.device("cuda:0")
    mlx, blobs = experts_np(N_EXP, H, I, seed=17)
    path = tmp_path / "layer34.q2blob"
    q2format.write_blob_file(path, blobs, H, I)
    store = FileExpertStore({LAYER: str(path)})
    mod = CachedSwitchGLU(store, LAYER, CAP, H, I)
    ora = olru.CLru(LAYER, CAP, expert_bytes=blobs.shape[1])
    ora.reset_stats()
    L = _lib.lib()
    try:
        ids_seq = synth.expert_id_stream(40, K, N_EXP, seed=21)
        xs = synth.hidden_states(40, H, seed=22)
        rng = np.random.default_rng(23)
        for t, ids in enumerate(ids_seq):
            ids = [int(v) for v in ids]
            sc = rng.random(K).astype(np.float16)
            out = mod.forward_combined(torch.from_numpy(xs[t]).to(dev), ids, torch.from_numpy(sc).to(dev))
            slots, _ = ora.step(ids)
            assert mod._slot_inds_buf[:K].cpu().tolist() == slots, t
            if t in (0, 17, 39):
                want = oracle_moe(xs[t], np.array(ids), sc, mlx)
                assert_close_rms(out.cpu().numpy(), want, 1e-2, f"step {t}")
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()

        # prefill through the file-backed layer (loads go through c_layer_load_sync)
        n_tok = 8
        pids = np.stack([rng.choice(N_EXP, K, replace=False) for _ in range(n_tok)]).astype(np.int32)
        px = synth.hidden_states(n_tok, H, seed=24)
        e0, s0 = ora.get_state()
        plan = q2.prefill_plan(pids.reshape(-1), e0, s0, CAP)
        y = mod(torch.from_numpy(px).to(dev)[None], torch.from_numpy(pids).to(dev)[None])
        torch.cuda.synchronize()
        yh = y[0].reshape(n_tok * K, H).cpu().numpy().astype(np.float64)
        flat = pids.reshape(-1)
        for e in sorted(set(flat.tolist()))[:6]:
            pairs = np.nonzero(flat == e)[0]
            want = q2.switch_glu_expert(px[pairs // K].astype(np.float64), *expert_fn(mlx)(e), bits=2, group=64)
            assert_close_rms(yh[pairs], want, 1e-2, f"prefill expert {e}")
        for _, _, le, ls in plan["chunks"]:
            if le:
                ora.load_sync(le, ls, 1)
        ora.set_state(*plan["new_lru"], plan["add_req"], plan["add_hits"], plan["add_misses"])
        assert _state(L, LAYER) == ora.get_state()
        mod.sync_stats_from_c()
        assert [int(v) for v in mod._c_stats_buf] == ora.stats()
        pool = mod.pool.cpu().numpy()
        for e, s in zip(*ora.get_state()):
            assert np.array_equal(pool[s], blobs[e]), (e, s)
        assert _lib.last_error() == ""
    finally:
        mod.close()
        store.close()
