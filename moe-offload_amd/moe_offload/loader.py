"""Drop-in host API of the reference loader (`mlx-qwen38/loader.py`) on MI355X.

Names, arguments and return values follow the reference:
  compute_layer_capacities  loader.py:245-303
  CachedSwitchGLU           loader.py:306-749   (per-layer slot cache + SwitchGLU)
  OffloadEngine             loader.py:1004-1343 (capacities, stats, greedy decode loop)
Storage differs by design: the slot pool is HBM and the "SSD" tier is a pinned host expert
store (HostExpertStore), a blob file per layer (FileExpertStore) or the reference's own
experts-XX.safetensors shards read in place (ShardExpertStore: the 9 tensors of each layer, 9
HBM slot pools); file-backed layers are read by the library's reader threads.  The cache decisions, counters and
slot ids come from libmoe_offload.so (the expert_io.c ABI); the compute is its HIP kernels.
"""
from __future__ import annotations

import ctypes
import json
import time
from pathlib import Path
from typing import Any

import numpy as np
import torch

from . import _lib, ops, q2format

NUM_LAYERS = 48
NUM_EXPERTS = 512
TOP_K = 10
PREFETCH_TOP_M = 12
PREFETCH_MAX_CAP = 3
MAX_K = 16


def compute_layer_capacities(budget_gb: float | None = None, budget_pct: float | None = None,
                             alloc_mode: str = "even", num_layers: int = NUM_LAYERS,
                             num_experts: int = NUM_EXPERTS, expert_bytes: int = 983_040,
                             analysis_summary: str | Path | None = None) -> dict[int, int]:
    """Slots per cached layer 1..num_layers-1 (layer 0 is pinned), as loader.py:245-303:
    budget_pct -> max(16, min(E, round(pct/100 * E))) per layer; budget_gb -> total slots
    round(budget / expert_bytes) clamped to [16, E] per layer, split evenly (the first
    remainder layers get one more) or in proportion to per-layer active-expert counts."""
    n = num_layers - 1
    if budget_pct is not None:
        frac = budget_pct / 100.0 if budget_pct > 1.0 else budget_pct
        per = max(16, min(num_experts, round(frac * num_experts)))
        total = n * per
    else:
        if budget_gb is None:
            budget_gb = 7.5
        total = int(round((budget_gb * 1e9) / expert_bytes))
        total = max(n * 16, min(n * num_experts, total))
    if alloc_mode == "proportional" and analysis_summary is not None and Path(analysis_summary).exists():
        summary = json.loads(Path(analysis_summary).read_text(encoding="utf-8"))
        info = summary["expert_concentration"]["per_layer"]
        w = np.array([float(info[il]["active_experts_decode"]) for il in range(1, num_layers)], np.float64)
        raw = w / w.sum() * total
        caps = np.clip(np.floor(raw).astype(int), 16, num_experts)
        rem = total - int(caps.sum())
        fr = raw - np.floor(raw)
        if rem > 0:
            for idx in np.argsort(-fr):
                if rem == 0:
                    break
                if caps[idx] < num_experts:
                    caps[idx] += 1
                    rem -= 1
        elif rem < 0:
            for idx in np.argsort(fr):
                if rem == 0:
                    break
                if caps[idx] > 16:
                    caps[idx] -= 1
                    rem += 1
        return {il: int(caps[il - 1]) for il in range(1, num_layers)}
    base, rem = divmod(total, n)
    return {il: min(num_experts, max(16, base + (1 if (il - 1) < rem else 0))) for il in range(1, num_layers)}


class HostExpertStore:
    """Pinned, device-mapped host memory with every expert blob of layers [first_layer, n_layers)."""

    def __init__(self, n_layers: int, n_exp: int, blob_bytes: int, first_layer: int = 0):
        self.n_layers, self.n_exp, self.blob_bytes, self.first = n_layers, n_exp, blob_bytes, first_layer
        self._ptr: dict[int, int] = {}
        L = _lib.lib()
        for l in range(first_layer, n_layers):
            p = L.c_host_alloc(n_exp * blob_bytes)
            if not p:
                self.close()
                raise _lib.NativeError(f"host store alloc failed: {_lib.last_error()}")
            self._ptr[l] = p
        _lib.lib().c_clear_error()

    def layer_ptr(self, l: int) -> int:
        return self._ptr[l]

    def view(self, l: int) -> np.ndarray:
        """uint8 [n_exp, blob_bytes] numpy view of layer l's store (shares memory)."""
        return np.ctypeslib.as_array(ctypes.cast(self._ptr[l], ctypes.POINTER(ctypes.c_uint8)),
                                     shape=(self.n_exp, self.blob_bytes))

    def tensor(self, l: int) -> torch.Tensor:
        return torch.from_numpy(self.view(l))

    def close(self):
        L = _lib.lib()
        for p in self._ptr.values():
            L.c_host_free(p)
        self._ptr.clear()


class FileExpertStore:
    """The on-disk tier: one expert blob file per layer (q2format.write_blob_file).  Misses are
    read with pread into a pinned bounce buffer and copied to HBM (expert_io.c:113-185 reads the
    reference's safetensors shard the same way, one row per tensor)."""

    def __init__(self, paths: dict[int, str]):
        import os
        self.paths = dict(paths)
        self.fds: dict[int, int] = {}
        self.headers: dict[int, dict] = {}
        for l, p in self.paths.items():
            self.headers[l] = q2format.read_blob_header(p)
            self.fds[l] = os.open(p, os.O_RDONLY)
        bb = {h["blob_bytes"] for h in self.headers.values()}
        if len(bb) != 1:
            raise ValueError("layers of one store must share the blob size")
        self.blob_bytes = bb.pop()

    def close(self):
        import os
        for fd in self.fds.values():
            os.close(fd)
        self.fds.clear()


def read_safetensors_header(fd: int) -> tuple[dict, int]:
    """(header, data_start) of a safetensors file: an 8-byte little-endian header length, the JSON
    header, then the data (loader.py:318-320 reads it the same way)."""
    import os
    import struct
    n = struct.unpack("<Q", os.pread(fd, 8, 0))[0]
    if n > (1 << 28):
        raise ValueError(f"safetensors header of {n} bytes")
    raw = os.pread(fd, n, 8)
    if len(raw) != n:
        raise ValueError("truncated safetensors header")
    return json.loads(raw), 8 + n


SHARD_ROLES = [(proj, suffix) for proj in ("gate_proj", "up_proj", "down_proj")
               for suffix in ("weight", "scales", "biases")]


class ShardExpertStore:
    """The reference's on-disk tier read in place: layer l's experts live in
    `experts-{l:02d}.safetensors` as 9 tensors `language_model.model.layers.{l}.mlp.switch_mlp.
    {gate,up,down}_proj.{weight,scales,biases}` (U32 codes [E, out, in/16]; BF16 or F16 scales and
    biases [E, out, in/group]).  Per layer the 9 (file offset, bytes per expert) pairs are listed in
    ascending file offset, as loader.py:336-395 hands them to c_layer_init, with each tensor's role
    (MOE_Q2T_* order: gate w/s/b, up w/s/b, down w/s/b) for c_layer_set_format9."""

    def __init__(self, shards: "dict[int, str] | str | Path", layers=None):
        import os
        if not isinstance(shards, dict):
            root = Path(shards)
            shards = {l: str(root / f"experts-{l:02d}.safetensors") for l in (layers or range(1, NUM_LAYERS))}
        self.paths = dict(shards)
        self.fds: dict[int, int] = {}
        self.layout: dict[int, dict] = {}
        try:
            for l, path in self.paths.items():
                fd = os.open(path, os.O_RDONLY)
                self.fds[l] = fd
                self.layout[l] = self._layer_layout(fd, l, os.fstat(fd).st_size)
        except Exception:
            self.close()
            raise
        dims = {(v["n_exp"], v["hidden"], v["inter"], v["group"]) for v in self.layout.values()}
        if len(dims) != 1:
            raise ValueError(f"shards disagree on (experts, hidden, inter, group): {sorted(dims)}")
        self.n_exp, self.hidden, self.inter, self.group = dims.pop()
        self.blob_bytes = sum(next(iter(self.layout.values()))["row_bytes"])

    @staticmethod
    def _layer_layout(fd: int, layer: int, file_size: int) -> dict:
        hdr, data_start = read_safetensors_header(fd)
        pre = f"language_model.model.layers.{layer}.mlp.switch_mlp"
        specs, sdt = [], set()
        for role, (proj, suffix) in enumerate(SHARD_ROLES):
            name = f"{pre}.{proj}.{suffix}"
            if name not in hdr:
                raise KeyError(f"{name} missing from the layer {layer} shard")
            info = hdr[name]
            shape, (a, b) = info["shape"], info["data_offsets"]
            want = "U32" if suffix == "weight" else ("BF16", "F16")
            if info["dtype"] not in (want if isinstance(want, tuple) else (want,)) or len(shape) != 3:
                raise ValueError(f"{name}: dtype {info['dtype']} shape {shape}")
            if suffix != "weight":
                sdt.add(info["dtype"])
            if (b - a) % shape[0] or data_start + b > file_size:
                raise ValueError(f"{name}: data range {a}..{b} does not fit the file")
            specs.append((data_start + a, (b - a) // shape[0], role, tuple(shape)))
        if len(sdt) != 1:
            raise ValueError(f"layer {layer}: mixed scale dtypes {sorted(sdt)}")
        gw = specs[0][3]
        n_exp, inter, hidden = gw[0], gw[1], gw[2] * 16
        group = hidden // specs[1][3][2]
        specs.sort(key=lambda t: t[0])                 # ascending file offset (loader.py:395)
        return {"offsets": [t[0] for t in specs], "row_bytes": [t[1] for t in specs],
                "roles": [t[2] for t in specs], "scale_bf16": sdt.pop() == "BF16",
                "n_exp": n_exp, "hidden": hidden, "inter": inter, "group": group}

    def close(self):
        import os
        for fd in self.fds.values():
            os.close(fd)
        self.fds.clear()


class HostShardStore:
    """The reference's shards in pinned, device-mapped host memory: per layer, the 9 tensors of
    `experts-{l:02d}.safetensors` (as ShardExpertStore lists them: ascending file offset, with
    their roles) each read whole -- one read per tensor, by the library's reader threads
    (c_io_read_ranges) -- into its own pinned buffer [n_exp, bytes per expert].  Layers bound to
    it stage misses from host memory (DMA, or the staging kernel when device-driven)."""

    def __init__(self, shards: "dict[int, str] | str | Path", layers=None, threads: int = 8):
        files = ShardExpertStore(shards, layers)
        L = _lib.lib()
        self.layout, self.ptrs = files.layout, {}
        self.n_exp, self.hidden, self.inter, self.group = files.n_exp, files.hidden, files.inter, files.group
        self.blob_bytes = files.blob_bytes
        L.c_io_init(threads)
        try:
            for l, lay in self.layout.items():
                ptrs = []
                for rb in lay["row_bytes"]:
                    ptr = L.c_host_alloc(self.n_exp * rb)
                    if not ptr:
                        raise _lib.NativeError(f"pinned shard store: {_lib.last_error()}")
                    ptrs.append(ptr)
                self.ptrs[l] = ptrs
                n = len(ptrs)
                u64 = ctypes.c_uint64 * n
                rc = L.c_io_read_ranges(files.fds[l], u64(*lay["offsets"]),
                                        u64(*[self.n_exp * rb for rb in lay["row_bytes"]]), u64(*ptrs), n)
                _lib.check(rc, f"reading the layer {l} shard")
        except Exception:
            self.close()
            raise
        finally:
            files.close()

    def tensor(self, l: int, t: int) -> np.ndarray:
        """uint8 [n_exp, bytes per expert] view of layer l's tensor t (file-offset order)."""
        rb = self.layout[l]["row_bytes"][t]
        return np.ctypeslib.as_array(ctypes.cast(self.ptrs[l][t], ctypes.POINTER(ctypes.c_uint8)),
                                     shape=(self.n_exp, rb))

    def close(self):
        L = _lib.lib()
        for ptrs in self.ptrs.values():
            for ptr in ptrs:
                L.c_host_free(ptr)
        self.ptrs.clear()


class CachedSwitchGLU:
    """Per-layer slot cache over an HBM pool + Q2 SwitchGLU (loader.py:306-749).

    `store` is the path of the layer's `experts-XX.safetensors` shard, as the reference passes it
    (loader.py:311, 1045-1046: read in place by the reader threads, a ShardExpertStore the module
    owns and closes), or a HostExpertStore (pinned host memory, fd == -1), a FileExpertStore (a blob file,
    fd >= 0; the pool holds `capacity` blobs), a ShardExpertStore (the reference's shard read in
    place, fd >= 0; `pools` are the 9 tensors' slot pools, each [capacity, bytes per expert], as
    loader.py:336-366 allocates them, and hidden/inter/group come from the shard) or a
    HostShardStore (the same 9 tensors from pinned host memory, fd == -1).
    decode: __call__(x [1,1,H] fp16, indices [1,1,k]) -> per-expert outputs [1,1,k,H], exactly
    like SwitchGLU; forward_combined() returns the score-weighted sum directly.
    """

    def __init__(self, store: "str | Path | HostExpertStore | FileExpertStore | ShardExpertStore | HostShardStore",
                 layer_idx: int, capacity: int,
                 hidden: int = 2048, inter: int = 512, group: int = 64, device: str | torch.device = "cuda"):
        self._own_store = isinstance(store, (str, Path))
        if self._own_store:                           # the reference's call: a shard path
            store = ShardExpertStore({layer_idx: str(store)})
        shard = isinstance(store, (ShardExpertStore, HostShardStore))
        if shard:
            hidden, inter, group = store.hidden, store.inter, store.group
        self.layer_idx, self.capacity = layer_idx, capacity
        self.hidden, self.inter, self.group = hidden, inter, group
        self.store = store
        dev = torch.device(device)
        u64 = ctypes.c_uint64 * 9
        L = _lib.lib()
        L.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        self._slot_inds_buf = torch.zeros(MAX_K, dtype=torch.int32, device=dev)
        self._h_ws = torch.zeros(MAX_K * inter, dtype=torch.float16, device=dev)
        if shard:
            lay = store.layout[layer_idx]
            self.blob_bytes = sum(lay["row_bytes"])
            self.pool = None
            self.pools = [torch.zeros((capacity, rb), dtype=torch.uint8, device=dev) for rb in lay["row_bytes"]]
            if isinstance(store, HostShardStore):         # host addresses in place of file offsets
                fd, src = -1, store.ptrs[layer_idx]
            else:
                fd, src = store.fds[layer_idx], lay["offsets"]
            L.c_layer_init(layer_idx, fd, capacity, u64(*src), u64(*lay["row_bytes"]),
                           u64(*[p.data_ptr() for p in self.pools]), self._slot_inds_buf.data_ptr())
            _lib.check_error("c_layer_init")
            _lib.check(L.c_layer_set_format9(layer_idx, hidden, inter, group, (ctypes.c_int32 * 9)(*lay["roles"]),
                                             int(lay["scale_bf16"])), "c_layer_set_format9")
        else:
            self.blob_bytes = q2format.expert_bytes(hidden, inter, group)
            assert store.blob_bytes == self.blob_bytes
            self.pool = torch.zeros((capacity, self.blob_bytes), dtype=torch.uint8, device=dev)
            self.pools = [self.pool]
            if isinstance(store, FileExpertStore):
                fd, base = store.fds[layer_idx], store.headers[layer_idx]["data_offset"]
            else:
                fd, base = -1, store.layer_ptr(layer_idx)
            L.c_layer_init(layer_idx, fd, capacity, u64(base, *[0] * 8),
                           u64(self.blob_bytes, *[0] * 8), u64(self.pool.data_ptr(), *[0] * 8),
                           self._slot_inds_buf.data_ptr())
            _lib.check_error("c_layer_init")
            _lib.check(L.c_layer_set_format(layer_idx, hidden, inter, group), "c_layer_set_format")
        self._c_stats_buf = (ctypes.c_uint64 * 18)()
        self.reset_stats()

    # -- cache management (loader.py:421-555) --
    def reset_cache(self) -> None:
        self.wait_prefetch()
        _lib.lib().c_layer_reset_cache(self.layer_idx)

    def reset_stats(self) -> None:
        _lib.lib().c_layer_reset_stats(self.layer_idx)

    def sync_stats_from_c(self) -> None:
        st = self._c_stats_buf
        _lib.lib().c_layer_get_stats(self.layer_idx, st)
        (self.decode_requests, self.decode_lru_hits, self.decode_prefetch_hits, self.decode_demand_misses,
         self.decode_demand_bytes, self.decode_prefetch_bytes, self.prefill_requests, self.prefill_lru_hits,
         self.prefill_demand_misses, self.prefill_demand_bytes, self.pred_top16_hits, self.pred_top16_total_actual,
         self.pred_top16_total_pred, self.miss_pref_hits, self.miss_pref_total_actual_misses,
         self.miss_pref_total_fetched, self.uncoalesced_tensor_reads, self.coalesced_preadv_calls) = [int(v) for v in st]

    def start_prefetch(self, pred_eids: list[int], max_fetch: int = PREFETCH_MAX_CAP) -> None:
        L = _lib.lib()
        n = len(pred_eids)
        if n == 10:
            L.c_layer_start_prefetch10(self.layer_idx, max_fetch, *pred_eids)
        elif n == 12:
            L.c_layer_start_prefetch12(self.layer_idx, max_fetch, *pred_eids)
        else:
            L.c_layer_start_prefetch(self.layer_idx, (ctypes.c_int32 * max(n, 1))(*pred_eids), n, max_fetch)
        _lib.check_error("start_prefetch")

    def wait_prefetch(self) -> None:
        _lib.lib().c_layer_wait_prefetch(self.layer_idx)

    def step(self, eids: list[int]) -> int:
        n = _lib.lib().c_layer_step_decode_ex(self.layer_idx, (ctypes.c_uint32 * len(eids))(*eids), len(eids), 1)
        return _lib.check(n, "step_decode")

    # -- compute --
    def forward_combined(self, x: torch.Tensor, indices, scores: torch.Tensor, residual: torch.Tensor | None = None,
                         out: torch.Tensor | None = None) -> torch.Tensor:
        """sum_j scores[j] * SwitchGLU_{indices[j]}(x) (+ residual), fp32 [H]; one token."""
        eids = [int(e) for e in (indices.reshape(-1).tolist() if torch.is_tensor(indices) else indices)]
        k = len(eids)
        self.step(eids)
        out = out if out is not None else torch.empty(self.hidden, dtype=torch.float32, device=x.device)
        rc = _lib.lib().c_layer_switch_glu(self.layer_idx, x.data_ptr(), scores.data_ptr(),
                                           residual.data_ptr() if residual is not None else None,
                                           self._h_ws.data_ptr(), out.data_ptr(), 0, k,
                                           torch.cuda.current_stream().cuda_stream)
        _lib.check(rc, "c_layer_switch_glu")
        return out

    def __call__(self, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        B, Lq, K = indices.shape
        if Lq == 1 and B == 1:
            eids = [int(e) for e in indices.reshape(-1).tolist()]
            self.step(eids)
            out = torch.empty((K, self.hidden), dtype=torch.float32, device=x.device)
            xr = x.reshape(-1).to(torch.float16).contiguous()
            rc = _lib.lib().c_layer_switch_glu(self.layer_idx, xr.data_ptr(), None, None, self._h_ws.data_ptr(),
                                               out.data_ptr(), 1, K, torch.cuda.current_stream().cuda_stream)
            _lib.check(rc, "c_layer_switch_glu")
            return out.to(x.dtype).reshape(1, 1, K, self.hidden)
        from .prefill import cached_prefill
        return cached_prefill(self, x, indices)

    def get_layer_stats(self) -> dict[str, Any]:
        """Same keys as loader.py:701-739 (bytes are real blob bytes)."""
        self.sync_stats_from_c()
        dec_req = max(1, self.decode_requests)
        pre_req = max(1, self.prefill_requests)
        return {
            "layer": self.layer_idx,
            "capacity_experts": self.capacity,
            "capacity_mb": round(self.capacity * self.blob_bytes / 1e6, 3),
            "decode_requests": self.decode_requests,
            "decode_lru_hits": self.decode_lru_hits,
            "decode_prefetch_hits": self.decode_prefetch_hits,
            "decode_demand_misses": self.decode_demand_misses,
            "decode_pure_hit_rate": round(self.decode_lru_hits / dec_req, 5),
            "decode_effective_hit_rate": round((self.decode_lru_hits + self.decode_prefetch_hits) / dec_req, 5),
            "decode_demand_bytes": self.decode_demand_bytes,
            "decode_prefetch_bytes": self.decode_prefetch_bytes,
            "decode_total_bytes": self.decode_demand_bytes + self.decode_prefetch_bytes,
            "prefill_requests": self.prefill_requests,
            "prefill_lru_hits": self.prefill_lru_hits,
            "prefill_demand_misses": self.prefill_demand_misses,
            "prefill_hit_rate": round(self.prefill_lru_hits / pre_req, 5),
            "prefill_demand_bytes": self.prefill_demand_bytes,
            "top16_router_recall": round(self.pred_top16_hits / max(1, self.pred_top16_total_actual), 5),
            "top16_router_precision": round(self.pred_top16_hits / max(1, self.pred_top16_total_pred), 5),
            "miss_prefetch_recall": round(self.miss_pref_hits / max(1, self.miss_pref_total_actual_misses), 5),
            "miss_prefetch_precision": round(self.miss_pref_hits / max(1, self.miss_pref_total_fetched), 5),
            "uncoalesced_tensor_reads": self.uncoalesced_tensor_reads,
            "coalesced_preadv_calls": self.coalesced_preadv_calls,
        }

    def close(self) -> None:
        self.wait_prefetch()
        torch.cuda.synchronize()
        _lib.lib().c_sync_copies()
        _lib.lib().c_layer_init(self.layer_idx, -1, 16, None, None, None, 0)
        if self._own_store:
            self.store.close()


class OffloadEngine:
    """Routed-expert offload engine (loader.py:1004-1343).

    model_path: a model directory in the reference's layout (experts-XX.safetensors shards, the
    8-bit routers in base-*.safetensors): the routed-expert stack over it (ckpt.CheckpointStack:
    layer 0 pinned, layers 1.. cached).  A path that is not such a directory raises.  Without a
    model_path, the synthetic 48-layer stack of the benchmark workload (stack.DecodeStack).
    There is no tokenizer or attention here (out of scope): a "token" is a hidden state fed to the
    routed-expert stack; `generate_greedy` runs it and reports the reference's timing and hit-rate
    keys.
    """

    def __init__(self, model_path=None, budget_gb: float | None = None, budget_pct: float | None = 20.0,
                 alloc_mode: str = "even", prefetch: bool = True, prefetch_top_m: int = PREFETCH_TOP_M,
                 prefetch_cap: int = PREFETCH_MAX_CAP, mode: str = "device", n_layers: int = NUM_LAYERS,
                 hidden: int = 2048, inter: int = 512, seed: int = 0, store_file: str | None = None,
                 io_threads: int = 8, io_direct: bool = False, shard_store: str = "host"):
        """Synthetic stack (no model_path) -- store_file: the cached layers read their misses from
        this blob file (the on-disk tier) with `io_threads` reader threads, through the page cache or
        with O_DIRECT; device mode then publishes each layer's misses to the library's feeder
        thread.  Without it they come from a pinned host store.  n_layers / hidden / inter / seed
        shape the synthetic model.
        Model directory -- shard_store: "host" reads the cached layers' shards once into pinned host
        memory (misses are then PCIe copies), "file" reads each miss from the shard in place with
        the reader threads (mode="host"); the shapes come from the files."""
        t0 = time.perf_counter()
        self.model_path, self.alloc_mode = model_path, alloc_mode
        self.prefetch, self.prefetch_top_m, self.prefetch_cap = prefetch, prefetch_top_m, prefetch_cap
        if model_path is not None:
            from .ckpt import CheckpointStack, CkptConfig
            if store_file is not None:
                raise ValueError("store_file names a synthetic stack's blob file; a model directory has its shards")
            ccfg = CkptConfig(budget_pct=budget_pct, budget_gb=budget_gb, prefetch=prefetch, top_m=prefetch_top_m,
                              prefetch_cap=prefetch_cap, store=shard_store, io_threads=io_threads)
            self.model = CheckpointStack(model_path, ccfg, mode=mode)
        else:
            from .stack import DecodeStack, StackConfig
            cfg = StackConfig(n_layers=n_layers, hidden=hidden, inter=inter, budget_pct=budget_pct,
                              budget_gb=budget_gb, prefetch=prefetch, top_m=prefetch_top_m, prefetch_cap=prefetch_cap,
                              seed=seed, store_file=store_file, io_threads=io_threads, io_direct=io_direct)
            self.model = DecodeStack(cfg, mode=mode)
        n_layers = self.model.cfg.n_layers
        self.capacities = self.model.capacities
        self.total_cached_slots = sum(self.capacities.values())
        self.cache_budget_bytes = self.total_cached_slots * self.model.blob_bytes
        self.layer0_pinned_bytes = self.model.cfg.n_exp * self.model.blob_bytes
        self.cached_modules = {l: l for l in range(1, n_layers)}
        self.tokenizer = None
        self.load_seconds = time.perf_counter() - t0

    def set_prefetch(self, enabled: bool, top_m: int | None = None, cap: int | None = None) -> None:
        self.prefetch = self.model.cfg.prefetch = enabled
        if top_m is not None:
            self.prefetch_top_m = self.model.cfg.top_m = top_m
        if cap is not None:
            self.prefetch_cap = self.model.cfg.prefetch_cap = cap
        self.model.graph = None

    def reset_caches(self) -> None:
        self.model.reset_caches()

    def reset_stats(self) -> None:
        self.model.reset_stats()

    def _snapshot_decode_totals(self) -> tuple[int, int, int, int, int, int]:
        return tuple(self.model.decode_totals())

    def generate_greedy(self, user_content=None, max_new_tokens: int = 128, reset_cache_before: bool = False,
                        reset_stats_before: bool = False, seed: int = 1234) -> dict[str, Any]:
        """Decode `max_new_tokens` synthetic tokens (hidden states ~ N(0,1) seeded from
        user_content) and report the reference's keys (loader.py:1223-1244)."""
        if reset_cache_before:
            self.reset_caches()
        if reset_stats_before:
            self.reset_stats()
        c = self.model.cfg
        if isinstance(user_content, str):
            seed = sum(user_content.encode()) + seed
        gen = torch.Generator(device=self.model.device)
        gen.manual_seed(seed)
        xs = torch.randn((max_new_tokens, c.hidden), device=self.model.device, generator=gen).half()
        s_start = self._snapshot_decode_totals()
        s_mid = s_start
        mid = min(32, max_new_tokens // 2) if max_new_tokens >= 16 else max_new_tokens // 2
        lat = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for d in range(max_new_tokens):
            ts = time.perf_counter()
            self.model.decode_token(xs[d])
            torch.cuda.synchronize()
            self.model.check_io()                    # this token's staging, not only earlier ones
            lat.append(round((time.perf_counter() - ts) * 1000.0, 3))
            if d + 1 == mid:
                s_mid = self._snapshot_decode_totals()
        dec = time.perf_counter() - t0
        s_end = self._snapshot_decode_totals()
        tot_req = max(1, s_end[3] - s_start[3])
        w1_req, w2_req = max(1, s_mid[3] - s_start[3]), max(1, s_end[3] - s_mid[3])
        w1 = sum(lat[:mid]) / 1000.0
        w2 = sum(lat[mid:]) / 1000.0
        return {
            "prompt_tokens": 0,
            "decode_tokens": max_new_tokens,
            "decode_seconds": round(dec, 4),
            "decode_tok_per_s": round(max_new_tokens / dec, 3),
            "prompt_pure_lru_hit_rate": round((s_end[0] - s_start[0]) / tot_req, 5),
            "prompt_effective_hit_rate": round((s_end[0] - s_start[0] + s_end[1] - s_start[1]) / tot_req, 5),
            "prompt_mb_per_token": round((s_end[4] - s_start[4] + s_end[5] - s_start[5]) / max(1, max_new_tokens) / 1e6, 3),
            "first_window_tokens": mid,
            "first_window_pure_hit_rate": round((s_mid[0] - s_start[0]) / w1_req, 5),
            "first_window_effective_hit_rate": round((s_mid[0] - s_start[0] + s_mid[1] - s_start[1]) / w1_req, 5),
            "first_window_tok_per_s": round(mid / max(1e-6, w1), 3),
            "steady_window_tokens": max_new_tokens - mid,
            "steady_window_pure_hit_rate": round((s_end[0] - s_mid[0]) / w2_req, 5),
            "steady_window_effective_hit_rate": round((s_end[0] - s_mid[0] + s_end[1] - s_mid[1]) / w2_req, 5),
            "steady_window_tok_per_s": round((max_new_tokens - mid) / max(1e-6, w2), 3),
            "step_latencies_ms": lat,
        }

    def collect_stats(self, total_decode_tokens: int, total_prefill_tokens: int = 0) -> dict[str, Any]:
        n = self.model.cfg.n_layers
        per = []
        for l in range(1, n):
            st = self.model.layer_stats(l)
            per.append({"layer": l, "capacity_experts": self.capacities[l], "decode_requests": st[0],
                        "decode_lru_hits": st[1], "decode_prefetch_hits": st[2], "decode_demand_misses": st[3],
                        "decode_demand_bytes": st[4], "decode_prefetch_bytes": st[5], "prefill_requests": st[6],
                        "prefill_lru_hits": st[7], "prefill_demand_misses": st[8], "prefill_demand_bytes": st[9],
                        "pred_hits": st[10], "pred_actual": st[11], "pred_total": st[12], "miss_pref_hits": st[13],
                        "miss_actual": st[14], "miss_fetched": st[15]})
        req = sum(p["decode_requests"] for p in per)
        lru = sum(p["decode_lru_hits"] for p in per)
        pref = sum(p["decode_prefetch_hits"] for p in per)
        dem_b = sum(p["decode_demand_bytes"] for p in per)
        pref_b = sum(p["decode_prefetch_bytes"] for p in per)
        dec_tok = max(1, total_decode_tokens)
        return {
            "budget_summary": {
                "alloc_mode": self.alloc_mode, "prefetch_enabled": self.prefetch,
                "prefetch_top_m": self.prefetch_top_m if self.prefetch else 0,
                "prefetch_cap": self.prefetch_cap if self.prefetch else 0,
                "layer0_pinned_experts": self.model.cfg.n_exp, "layer0_pinned_bytes": self.layer0_pinned_bytes,
                "cached_layers_count": n - 1, "total_cached_slots": self.total_cached_slots,
                "cache_budget_bytes": self.cache_budget_bytes,
            },
            "decode_aggregate": {
                "total_decode_tokens": total_decode_tokens, "total_requests": req, "lru_hits": lru,
                "prefetch_hits": pref, "demand_misses": sum(p["decode_demand_misses"] for p in per),
                "pure_lru_hit_rate": round(lru / max(1, req), 5),
                "effective_hit_rate": round((lru + pref) / max(1, req), 5),
                "top_m_router_recall": round(sum(p["pred_hits"] for p in per) / max(1, sum(p["pred_actual"] for p in per)), 5),
                "miss_prefetch_recall": round(sum(p["miss_pref_hits"] for p in per) / max(1, sum(p["miss_actual"] for p in per)), 5),
                "demand_bytes_read": dem_b, "prefetch_bytes_read": pref_b,
                "total_mb_per_token": round((dem_b + pref_b) / dec_tok / 1e6, 3),
            },
            "per_layer": per,
        }

    def close(self) -> None:
        self.model.close()
