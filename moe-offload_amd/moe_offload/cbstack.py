"""Stacked decode of the 2-bit codebook experts (the Nemotron-style workload) on one MI355X.

Each layer l has 240 non-gated experts (up 3072 -> 1536, squared ReLU, down 1536 -> 3072) in
the codebook format of `cbformat`, top-9 routing drawn from a seeded Zipf(s) over the experts
(a per-layer random permutation maps popularity rank to expert id; scores are seeded and
normalised), and an fp16 RMSNorm after it (builder glue, as in `stack.py`):

    h_l     = x_l + sum_j scores_j * down_j(relu(up_j x_l)^2)      (fp32)
    x_{l+1} = RMSNorm(h_l)                                          (fp16, eps 1e-6)

A layer is two launches: the up-projection of layer l > 0 normalises h_{l-1} itself
(`moe_cb_moe_norm`), so only the last layer's output needs a standalone RMSNorm.

Every layer keeps `capacity` slots in HBM (the expert-cache budget split evenly over the
layers), fed from a pinned host store; the slot tables are device-driven (same decisions as the
reference's expert_io.c LRU) and misses are staged by the staging kernel.  No prefetch: the
workload has no router to predict with.  `resident=True` keeps every expert in HBM instead
(slot = expert id) for the kernels' own roofline.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib, cbformat
from .loader import HostExpertStore


@dataclass
class CbStackConfig:
    n_layers: int = 40
    hidden: int = 3072
    inter: int = 1536
    n_exp: int = 240
    top_k: int = 9
    cache_gib: float = 4.0
    zipf_s: float = 1.0
    eps: float = 1e-6
    seed: int = 0
    layer_base: int = 0
    stage_ctas: int = 8          # staging blocks per 2.4 MB expert (118.1 tok/s at the 4 GiB cache against
                                 # 115.0 with 2, 117.5 with 4, 117.4 with 16)
    resident: bool = False
    d_scale: float = 0.01


def zipf_routing(n_tok: int, n_layers: int, n_exp: int, k: int, s: float, seed: int):
    """ids int32 [n_tok, n_layers, k] (distinct per token-layer) and fp16 scores summing to 1."""
    rng = np.random.default_rng(seed)
    p = 1.0 / np.arange(1, n_exp + 1) ** s
    p /= p.sum()
    perm = np.stack([rng.permutation(n_exp) for _ in range(n_layers)])
    ids = np.empty((n_tok, n_layers, k), np.int32)
    for t in range(n_tok):
        for l in range(n_layers):
            ids[t, l] = perm[l][rng.choice(n_exp, size=k, replace=False, p=p)]
    sc = rng.random((n_tok, n_layers, k)) + 0.05
    sc = (sc / sc.sum(-1, keepdims=True)).astype(np.float16)
    return ids, sc


def gpu_random_blobs(n_exp: int, hidden: int, inter: int, gen: torch.Generator, device, d_scale: float):
    """Random codebook experts generated on the GPU: any byte is a valid code byte; the two scale
    planes get |N(0, d_scale)| fp16."""
    o = cbformat.blob_offsets(hidden, inter)
    blobs = torch.randint(0, 256, (n_exp, o["bytes"]), dtype=torch.uint8, device=device, generator=gen)
    nd = (o["bytes"] - o["up_d"]) // 2
    d = (torch.randn((n_exp, nd), device=device, generator=gen) * d_scale).abs().half()
    blobs[:, o["up_d"]:] = d.view(torch.uint8).view(n_exp, nd * 2)
    return blobs


class CodebookStack:
    def __init__(self, cfg: CbStackConfig = CbStackConfig(), device="cuda"):
        c = self.cfg = cfg
        self.device = dev = torch.device(device)
        self.L = L = _lib.lib()
        self.blob_bytes = cbformat.expert_bytes(c.hidden, c.inter)
        self.grid = torch.from_numpy(cbformat.grid()).to(dev)
        gen = torch.Generator(device=dev)
        gen.manual_seed(c.seed)
        self.norm_w = (1.0 + 0.1 * torch.randn((c.n_layers, c.hidden), device=dev, generator=gen)).half()
        self.capacity = max(c.top_k, min(c.n_exp, int(c.cache_gib * (1 << 30) // (c.n_layers * self.blob_bytes))))
        self.pools, self.slot_inds, self.store = [], [], None
        if c.resident:
            self.pools = [gpu_random_blobs(c.n_exp, c.hidden, c.inter, gen, dev, c.d_scale) for _ in range(c.n_layers)]
        else:
            self.store = HostExpertStore(c.n_layers, c.n_exp, self.blob_bytes)
            L.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
            u64 = ctypes.c_uint64 * 9
            for l in range(c.n_layers):
                blobs = gpu_random_blobs(c.n_exp, c.hidden, c.inter, gen, dev, c.d_scale)
                self.store.tensor(l).copy_(blobs)
                del blobs
                pool = torch.zeros((self.capacity, self.blob_bytes), dtype=torch.uint8, device=dev)
                si = torch.zeros(16, dtype=torch.int32, device=dev)
                self.pools.append(pool)
                self.slot_inds.append(si)
                li = c.layer_base + l
                L.c_layer_init(li, -1, self.capacity, u64(self.store.layer_ptr(l), *[0] * 8),
                               u64(self.blob_bytes, *[0] * 8), u64(pool.data_ptr(), *[0] * 8), si.data_ptr())
                _lib.check(L.c_layer_set_device_mode(li, 1), "set_device_mode")
            _lib.check_error("c_layer_init")
        torch.cuda.synchronize()
        self.ids = torch.zeros((c.n_layers, c.top_k), dtype=torch.int32, device=dev)
        self.scores = torch.zeros((c.n_layers, c.top_k), dtype=torch.float16, device=dev)
        self.xs = torch.zeros((c.n_layers + 1, c.hidden), dtype=torch.float16, device=dev)
        self.hs = torch.zeros((c.n_layers, c.hidden), dtype=torch.float32, device=dev)
        self.h_ws = torch.zeros(c.top_k * c.inter, dtype=torch.bfloat16, device=dev)
        self.graph = None

    def cidx(self, l: int) -> int:
        return self.cfg.layer_base + l

    def decode_token_device(self):
        """One token from xs[0] and the routing in ids/scores; writes xs[n_layers]."""
        c, L = self.cfg, self.L
        stream = torch.cuda.current_stream().cuda_stream
        for l in range(c.n_layers):
            if c.resident:
                pool, n_slots, slots = self.pools[l], c.n_exp, self.ids[l]
            else:
                _lib.check(L.c_layer_step_decode_dev(self.cidx(l), self.ids[l].data_ptr(), c.top_k, c.stage_ctas,
                                                     stream), "step_dev")
                pool, n_slots, slots = self.pools[l], self.capacity, self.slot_inds[l]
            if l == 0:
                _lib.check(L.moe_cb_moe(self.xs[0].data_ptr(), pool.data_ptr(), self.blob_bytes, n_slots,
                                        slots.data_ptr(), self.scores[0].data_ptr(), c.top_k, c.hidden, c.inter,
                                        self.grid.data_ptr(), self.xs[0].data_ptr(), self.h_ws.data_ptr(),
                                        self.hs[0].data_ptr(), 0, stream), "cb_moe")
            else:
                # x_l = RMSNorm(h_{l-1}) inside the up-projection (also written to xs[l])
                _lib.check(L.moe_cb_moe_norm(self.hs[l - 1].data_ptr(), self.norm_w[l - 1].data_ptr(), c.eps,
                                             self.xs[l].data_ptr(), pool.data_ptr(), self.blob_bytes, n_slots,
                                             slots.data_ptr(), self.scores[l].data_ptr(), c.top_k, c.hidden, c.inter,
                                             self.grid.data_ptr(), self.h_ws.data_ptr(), self.hs[l].data_ptr(),
                                             stream), "cb_moe_norm")
        n = c.n_layers
        _lib.check(L.moe_rmsnorm(self.hs[n - 1].data_ptr(), self.norm_w[n - 1].data_ptr(), c.eps, c.hidden,
                                 self.xs[n].data_ptr(), stream), "rmsnorm")

    def capture_graph(self):
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream(device=self.device)
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(g, stream=s):
                self.decode_token_device()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        self.graph = g

    def decode_token(self, x0: torch.Tensor, ids: torch.Tensor, scores: torch.Tensor) -> torch.Tensor:
        """ids int32 [n_layers, k], scores fp16 [n_layers, k] (device) for this token."""
        self.xs[0].copy_(x0)
        self.ids.copy_(ids)
        self.scores.copy_(scores)
        if self.graph is not None:
            self.graph.replay()
        else:
            self.decode_token_device()
        return self.xs[self.cfg.n_layers]

    def layer_stats(self, l: int) -> list[int]:
        o = (ctypes.c_uint64 * 18)()
        self.L.c_layer_get_stats(self.cidx(l), o)
        return list(o)

    def totals(self) -> list[int]:
        """(lru hits, prefetch hits, misses, requests, demand bytes, prefetch bytes) over all layers."""
        t = [0] * 6
        if self.cfg.resident:
            return t
        for l in range(self.cfg.n_layers):
            st = self.layer_stats(l)
            for i, w in enumerate((1, 2, 3, 0, 4, 5)):
                t[i] += st[w]
        return t

    def routed_bytes_per_token(self) -> int:
        return self.cfg.n_layers * self.cfg.top_k * self.blob_bytes

    def close(self):
        torch.cuda.synchronize()
        self.graph = None
        if self.store is not None:
            self.L.c_sync_copies()
            for l in range(self.cfg.n_layers):
                self.L.c_layer_init(self.cidx(l), -1, 16, None, None, None, 0)
            self.store.close()
            self.store = None
        self.pools = []
