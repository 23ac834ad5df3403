"""Routed-expert decode over the reference's own model directory (the real checkpoint's format).

A model directory holds, as the reference's engine reads it (`mlx-qwen38/loader.py:1004-1095`,
`cpp/src/loader.cpp:281-292,398-460`):

* `experts-{l:02d}.safetensors` for layers l = 0..L-1: the routed experts of layer l as 9 tensors
  `language_model.model.layers.{l}.mlp.switch_mlp.{gate,up,down}_proj.{weight,scales,biases}`
  (2-bit codes U32 [E, out, in/16], BF16 scales and biases [E, out, in/64]); layer 0 is pinned in
  HBM (loader.py:1059-1060), layers 1.. are cached (loader.py:1045-1046);
* `base-*.safetensors`: among the trunk, each layer's router `language_model.model.layers.{l}.
  mlp.gate.{weight,scales,biases}`, an 8-bit affine group-64 linear layer (U32 [E, H/4], BF16
  [E, H/64]; loader.cpp:450, kernels.cpp:997-1019).

Per layer l of a token (loader.py:903-977, decode):

    ids_l, scores_l = router_q8(x_l; gate_l)                 bf16 rule (softmax, top-k, renormalise)
    pred_{l+1}      = top-m(gate_{l+1} . x_l)                  (loader.py:237-242, 950-958)
    h_l             = x_l + sum_j scores_j SwitchGLU_{ids_j}(x_l)          (fp32)
    x_{l+1}         = bf16(RMSNorm(h_l))                         builder-defined glue (the model mixes
                                                                 hyper-connections and attention here)

The router reads x_l in bf16; the expert kernels read its fp16 copy (exact in fp16's normal range).
The slot decisions are the library's (the expert_io.c ABI), device-driven (tables on the GPU,
staging kernel, HIP-graph replay) or host-driven (one device->host read per layer, the reference's
shape).  Layer 0 predicts layer 1 from x_0 as every other layer predicts from its own input; the
reference predicts layer 1 from layer 0's post-MoE state (loader.py:923-932).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from . import _lib
from .loader import HostShardStore, ShardExpertStore, compute_layer_capacities, read_safetensors_header

ROUTER = "language_model.model.layers.{l}.mlp.gate.{s}"


@dataclass
class CkptConfig:
    budget_pct: float | None = 20.0
    budget_gb: float | None = None
    top_k: int = 10
    prefetch: bool = True
    top_m: int = 12
    prefetch_cap: int = 3
    eps: float = 1e-6
    store: str = "host"          # "host": shards read once into pinned host memory (HostShardStore);
                                 # "file": read in place by the reader threads at each miss (host mode)
    io_threads: int = 8
    layer_base: int = 0          # first C-ABI layer index used
    stage_ctas: int = 8          # staging blocks per copied expert (its 9 tensors in one launch; at 48 layers,
                                 # 20% cache: 2 -> 41, 4 -> 69, 8 -> 81, 16 -> 77 tok/s on one box)
    fused_norm: bool = True      # device path: the RMSNorm runs inside the router launch (moe_router_q8_norm)
                                 # instead of a launch of its own; the host path keeps the two launches
    # set from the directory
    n_layers: int = 0
    hidden: int = 0
    inter: int = 0
    n_exp: int = 0
    group: int = 64


def expert_layers(model_dir: Path) -> int:
    """Number of consecutive experts-XX.safetensors shards from experts-00."""
    n = 0
    while (model_dir / f"experts-{n:02d}.safetensors").exists():
        n += 1
    return n


def _read(fd: int, off: int, nbytes: int) -> np.ndarray:
    buf = bytearray(nbytes)
    view, done = memoryview(buf), 0
    while done < nbytes:
        got = os.preadv(fd, [view[done:]], off + done)
        if got <= 0:
            raise ValueError(f"short read at offset {off + done}")
        done += got
    return np.frombuffer(buf, np.uint8)


def load_routers(model_dir: Path, n_layers: int, n_exp: int, hidden: int, group: int = 64) -> list[tuple]:
    """Each layer's 8-bit router (codes int32 [E, H/4], scales / biases bf16 bits int16 [E, H/group])
    from the directory's base-*.safetensors, checked against the expert shards' shape."""
    found: dict[str, tuple[Path, int, dict]] = {}
    bases = sorted(model_dir.glob("base-*.safetensors"))
    if not bases:
        raise FileNotFoundError(f"{model_dir}: no base-*.safetensors (the routers live there)")
    for p in bases:
        fd = os.open(p, os.O_RDONLY)
        try:
            hdr, start = read_safetensors_header(fd)
        finally:
            os.close(fd)
        for name, info in hdr.items():
            if name.endswith((".mlp.gate.weight", ".mlp.gate.scales", ".mlp.gate.biases")):
                found[name] = (p, start, info)
    out = []
    for l in range(n_layers):
        arrs = []
        for s, dt, cols in (("weight", "U32", hidden // 4), ("scales", "BF16", hidden // group),
                            ("biases", "BF16", hidden // group)):
            name = ROUTER.format(l=l, s=s)
            if name not in found:
                raise KeyError(f"{model_dir}: {name} missing from base-*.safetensors")
            p, start, info = found[name]
            if info["dtype"] != dt or info["shape"] != [n_exp, cols]:
                raise ValueError(f"{name}: {info['dtype']} {info['shape']}, want {dt} {[n_exp, cols]} "
                                 "(an 8-bit group-64 router over the experts' hidden size)")
            a, b = info["data_offsets"]
            fd = os.open(p, os.O_RDONLY)
            try:
                raw = _read(fd, start + a, b - a)
            finally:
                os.close(fd)
            arrs.append(raw.view(np.int32 if dt == "U32" else np.int16).reshape(n_exp, cols))
        out.append(tuple(arrs))
    return out


class SyntheticCheckpoint:
    """The real checkpoint's shapes with seeded random content, made on the GPU (no files): per layer
    the 9 expert tensors in role order (2-bit codes uniform over all patterns, bf16 scales
    N(0, scale_std), biases -1.5 x scale, as the synthetic blob stacks draw them) and an 8-bit
    group-64 router (scales ~2e-4, biases ~ -128 x scale: logits of order one).  For measuring the
    production shape at 48 layers, whose files would be 37.7 GB."""

    def __init__(self, n_layers: int = 48, n_exp: int = 512, hidden: int = 2560, inter: int = 640, seed: int = 0,
                 scale_std: float = 0.02, device="cuda"):
        self.n_layers, self.n_exp, self.hidden, self.inter, self.group = n_layers, n_exp, hidden, inter, 64
        self.scale_std = scale_std
        self.device = torch.device(device)
        self.gen = torch.Generator(device=self.device)
        self.gen.manual_seed(seed)
        self.row_bytes = []
        for out_f, in_f in ((inter, hidden), (inter, hidden), (hidden, inter)):
            self.row_bytes += [out_f * in_f // 4, out_f * (in_f // 64) * 2, out_f * (in_f // 64) * 2]

    def layer(self, l: int) -> list[torch.Tensor]:
        """Layer l's 9 tensors, uint8 [n_exp, bytes per expert] on the GPU, role order."""
        g, dev, E = self.gen, self.device, self.n_exp
        out = []
        for out_f, in_f in ((self.inter, self.hidden), (self.inter, self.hidden), (self.hidden, self.inter)):
            w = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, out_f, in_f // 16), dtype=torch.int32, device=dev, generator=g)
            sc = (torch.randn((E, out_f, in_f // 64), device=dev, generator=g) * self.scale_std).to(torch.bfloat16)
            bi = (-1.5 * sc.float()).to(torch.bfloat16)
            out += [t.contiguous().view(torch.uint8).reshape(E, -1) for t in (w, sc, bi)]
        return out

    def routers(self) -> list[tuple]:
        g, dev, E, H = self.gen, self.device, self.n_exp, self.hidden
        res = []
        for _ in range(self.n_layers):
            codes = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, H // 4), dtype=torch.int32, device=dev, generator=g)
            sc = (torch.randn((E, H // 64), device=dev, generator=g) * 2e-4).to(torch.bfloat16)
            bi = (-128 * sc.float() + torch.randn((E, H // 64), device=dev, generator=g) * 1e-4).to(torch.bfloat16)
            res.append((codes, sc.view(torch.int16), bi.view(torch.int16)))
        return res


class _PinnedLayers:
    """Layers 1.. of a SyntheticCheckpoint copied into pinned, device-mapped host memory, with the
    attributes the stack reads from a HostShardStore (layout, ptrs, close)."""

    def __init__(self, src: SyntheticCheckpoint, layers):
        L = _lib.lib()
        self.layout, self.ptrs = {}, {}
        try:
            for l in layers:
                ts = src.layer(l)
                ptrs = []
                for t in ts:
                    ptr = L.c_host_alloc(t.numel())
                    if not ptr:
                        raise _lib.NativeError(f"pinned synthetic store: {_lib.last_error()}")
                    ptrs.append(ptr)
                    host = torch.from_numpy(np.ctypeslib.as_array(ctypes.cast(ptr, ctypes.POINTER(ctypes.c_uint8)),
                                                                  shape=tuple(t.shape)))
                    host.copy_(t)
                self.ptrs[l] = ptrs
                self.layout[l] = {"offsets": [0] * 9, "row_bytes": list(src.row_bytes), "roles": list(range(9)),
                                  "scale_bf16": True, "n_exp": src.n_exp, "hidden": src.hidden, "inter": src.inter,
                                  "group": src.group}
                del ts
        except Exception:
            self.close()
            raise

    def close(self):
        L = _lib.lib()
        for ptrs in self.ptrs.values():
            for p in ptrs:
                L.c_host_free(p)
        self.ptrs.clear()


class CheckpointStack:
    """The 48-layer routed-expert decode over a model directory (module docstring).

    synthetic: a SyntheticCheckpoint in place of a directory (the production shape at any depth).
    resident=True: every layer's experts in HBM (no cache, no tables): per layer the 8-bit router's
    logits, then moe_q2t_gate_up_routed (its blocks select the experts), then the down product."""

    def __init__(self, model_path=None, cfg: CkptConfig | None = None, mode: str = "device", device="cuda",
                 synthetic: SyntheticCheckpoint | None = None, resident: bool = False):
        if mode not in ("device", "host"):
            raise ValueError(f"mode {mode!r}: 'device' or 'host'")
        self.cfg = c = cfg or CkptConfig()
        self.mode = mode
        self.resident = resident
        self.device = dev = torch.device(device)
        if c.store not in ("host", "file"):
            raise ValueError(f"store {c.store!r}: 'host' or 'file'")
        if c.store == "file" and mode == "device":
            raise ValueError("store='file' runs host-driven tables (mode='host')")
        if resident and mode != "device":
            raise ValueError("resident=True is device-driven")
        if synthetic is None:
            root = Path(model_path)
            if not root.is_dir():
                raise FileNotFoundError(f"{root}: not a model directory")
            n_layers = expert_layers(root)
            if n_layers < 2:
                raise FileNotFoundError(f"{root}: needs experts-00.safetensors and experts-01.safetensors at least")
        else:
            n_layers = synthetic.n_layers
        self.L = L = _lib.lib()
        if synthetic is None:
            shards = {l: str(root / f"experts-{l:02d}.safetensors") for l in range(n_layers)}
            lay0 = ShardExpertStore({0: shards[0]})
            c.n_layers, c.n_exp, c.hidden, c.inter, c.group = n_layers, lay0.n_exp, lay0.hidden, lay0.inter, lay0.group
            if c.group != 64:
                lay0.close()
                raise ValueError(f"{root}: experts of group {c.group} (the kernels take 64)")
            self.scale_bf16 = int(lay0.layout[0]["scale_bf16"])
            self.blob_bytes = lay0.blob_bytes                      # bytes per expert over its 9 tensors
            # layer 0: all 9 tensors in HBM, in role order (MOE_Q2T_*: gate w/s/b, up w/s/b, down w/s/b)
            try:
                self.pool0, self.ptrs0, self.nbytes0 = self._pack(self._read_resident(lay0, 0))
            finally:
                lay0.close()
            r = load_routers(root, n_layers, c.n_exp, c.hidden, c.group)
            self.routers = [tuple(torch.from_numpy(a).to(dev) for a in t) for t in r]
        else:
            c.n_layers, c.n_exp, c.hidden, c.inter, c.group = (n_layers, synthetic.n_exp, synthetic.hidden,
                                                               synthetic.inter, synthetic.group)
            self.scale_bf16 = 1
            self.blob_bytes = sum(synthetic.row_bytes)
            self.routers = synthetic.routers()
            self.pool0, self.ptrs0, self.nbytes0 = self._pack(synthetic.layer(0))
        self.capacities = compute_layer_capacities(budget_gb=c.budget_gb, budget_pct=c.budget_pct,
                                                   num_layers=n_layers, num_experts=c.n_exp,
                                                   expert_bytes=self.blob_bytes)
        self.pools, self.slot_inds = {}, {}
        self.full = None
        if resident:                                      # every layer in HBM, slot = expert id
            self.store = None
            self.full = [(self.pool0, self.ptrs0, self.nbytes0)]
            for l in range(1, n_layers):
                self.full.append(self._pack(synthetic.layer(l) if synthetic is not None else
                                            self._read_file_layer(shards[l], l)))
            self._init_buffers()
            return
        # layers 1..: cached pools fed from pinned host memory or the files
        L.c_set_compute_stream(ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream))
        if synthetic is not None:
            self.store = _PinnedLayers(synthetic, range(1, n_layers))
        elif c.store == "host":
            self.store = HostShardStore({l: shards[l] for l in range(1, n_layers)}, threads=c.io_threads)
        else:
            L.c_io_init(c.io_threads)
            self.store = ShardExpertStore({l: shards[l] for l in range(1, n_layers)})
        u64 = ctypes.c_uint64 * 9
        for l in range(1, n_layers):
            lay = self.store.layout[l]
            if (lay["n_exp"], lay["hidden"], lay["inter"], lay["group"]) != (c.n_exp, c.hidden, c.inter, c.group):
                raise ValueError(f"experts-{l:02d}: shape differs from experts-00")
            li = self.cidx(l)
            self.pools[l] = [torch.zeros((self.capacities[l], rb), dtype=torch.uint8, device=dev)
                             for rb in lay["row_bytes"]]
            self.slot_inds[l] = torch.zeros(16, dtype=torch.int32, device=dev)
            src = self.store.ptrs[l] if c.store == "host" else lay["offsets"]
            fd = -1 if c.store == "host" else self.store.fds[l]
            L.c_layer_init(li, fd, self.capacities[l], u64(*src), u64(*lay["row_bytes"]),
                           u64(*[p.data_ptr() for p in self.pools[l]]), self.slot_inds[l].data_ptr())
            _lib.check_error(f"c_layer_init {li}")
            # bit 1: the layer's scores are the 8-bit router's bf16 scores
            _lib.check(L.c_layer_set_format9(li, c.hidden, c.inter, c.group, (ctypes.c_int32 * 9)(*lay["roles"]),
                                             int(lay["scale_bf16"]) | 2), "c_layer_set_format9")
            if mode == "device":
                _lib.check(L.c_layer_set_device_mode(li, 1), "set_device_mode")
        self._init_buffers()

    def _init_buffers(self):
        c, L, dev, n_layers = self.cfg, self.L, self.device, self.cfg.n_layers
        k, m = c.top_k, max(c.top_m, 1)
        self.xb = torch.zeros((n_layers + 1, c.hidden), dtype=torch.int16, device=dev)   # bf16 bits
        self.xf = torch.zeros((n_layers + 1, c.hidden), dtype=torch.float16, device=dev)
        self.hs = torch.zeros((n_layers, c.hidden), dtype=torch.float32, device=dev)
        self.ids = torch.zeros((n_layers, k), dtype=torch.int32, device=dev)
        self.scores = torch.zeros((n_layers, k), dtype=torch.int16, device=dev)          # bf16 bits
        self.pred = torch.zeros((n_layers, m), dtype=torch.int32, device=dev)
        self.logits = torch.zeros((n_layers, c.n_exp), dtype=torch.int16, device=dev)    # bf16 bits
        wsb = int(L.moe_router_q8_workspace_bytes(c.n_exp))
        self.ws_route = [torch.zeros(wsb, dtype=torch.uint8, device=dev) for _ in range(n_layers)]
        self.ws_pred = [torch.zeros(wsb, dtype=torch.uint8, device=dev) for _ in range(n_layers)]
        self.h_ws = torch.zeros(16 * c.inter, dtype=torch.float16, device=dev)
        self.side = torch.cuda.Stream(device=dev)
        self.ev_pred = [torch.cuda.Event() for _ in range(n_layers)]
        self.ev_pref = [torch.cuda.Event() for _ in range(n_layers)]
        self.ev_copy = [torch.cuda.Event() for _ in range(n_layers)]
        self.ev_demand = [torch.cuda.Event() for _ in range(n_layers)]
        self.graph = None
        self.file_device = False
        torch.cuda.synchronize()

    def _read_resident(self, files: ShardExpertStore, l: int) -> list[torch.Tensor]:
        """Layer l's 9 tensors from its shard into HBM, role order."""
        lay = files.layout[l]
        by_role = [None] * 9
        for off, rb, role in zip(lay["offsets"], lay["row_bytes"], lay["roles"]):
            raw = _read(files.fds[l], off, lay["n_exp"] * rb)
            by_role[role] = torch.from_numpy(raw.reshape(lay["n_exp"], rb)).to(self.device)
        return by_role

    def _read_file_layer(self, path: str, l: int) -> list[torch.Tensor]:
        files = ShardExpertStore({l: path})
        try:
            lay = files.layout[l]
            if (lay["n_exp"], lay["hidden"], lay["inter"]) != (self.cfg.n_exp, self.cfg.hidden, self.cfg.inter):
                raise ValueError(f"{path}: shape differs from experts-00")
            return self._read_resident(files, l)
        finally:
            files.close()

    @staticmethod
    def _pack(by_role: list[torch.Tensor]):
        u64 = ctypes.c_uint64 * 9
        return by_role, u64(*[t.data_ptr() for t in by_role]), u64(*[t.shape[1] for t in by_role])

    def cidx(self, l: int) -> int:
        return self.cfg.layer_base + l

    # ---- one token ---------------------------------------------------------------------------
    def _router_call(self, l: int, s: int, norm: bool, k: int, ids, scores, logits):
        """Layer l's router (route mode k > 0, or logits only); norm: with the RMSNorm of the
        previous layer's output fused in (writes xb[l] and xf[l] as the separate norm does)."""
        c, L = self.cfg, self.L
        codes, scales, biases = self.routers[l]
        if norm:
            rc = L.moe_router_q8_norm(self.hs[l - 1].data_ptr(), None, c.eps, self.xb[l].data_ptr(),
                                      self.xf[l].data_ptr(), codes.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                      c.hidden, c.n_exp, c.group, k, 0, self.ws_route[l].data_ptr(), ids, scores, None,
                                      logits, s)
        else:
            rc = L.moe_router_q8(self.xb[l].data_ptr(), codes.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                 c.hidden, c.n_exp, c.group, k, 0, self.ws_route[l].data_ptr(), ids, scores, None,
                                 logits, s)
        _lib.check(rc, "router_q8_norm" if norm else "router_q8")

    def _router(self, l: int, s: int, norm: bool = False):
        c, L = self.cfg, self.L
        self._router_call(l, s, norm, c.top_k, self.ids[l].data_ptr(), self.scores[l].data_ptr(), None)
        if c.prefetch and l + 1 < c.n_layers:
            codes, scales, biases = self.routers[l + 1]
            _lib.check(L.moe_router_q8(self.xb[l].data_ptr(), codes.data_ptr(), scales.data_ptr(), biases.data_ptr(),
                                       c.hidden, c.n_exp, c.group, 0, c.top_m, self.ws_pred[l].data_ptr(), None, None,
                                       self.pred[l].data_ptr(), None, s), "router_q8 predict")

    def _glu(self, l: int, s: int):
        c, L = self.cfg, self.L
        if l == 0:
            rc = L.moe_q2t_switch_glu(self.xf[0].data_ptr(), self.ptrs0, self.nbytes0, self.scale_bf16 | 2, c.n_exp,
                                      self.ids[0].data_ptr(), self.scores[0].data_ptr(), c.top_k, c.hidden, c.inter,
                                      c.group, self.xf[0].data_ptr(), self.h_ws.data_ptr(), self.hs[0].data_ptr(), 0, s)
        else:
            rc = L.c_layer_switch_glu(self.cidx(l), self.xf[l].data_ptr(), self.scores[l].data_ptr(),
                                      self.xf[l].data_ptr(), self.h_ws.data_ptr(), self.hs[l].data_ptr(), 0, c.top_k, s)
        _lib.check(rc, "switch_glu")

    def _norm(self, l: int, s: int):
        _lib.check(self.L.moe_rmsnorm_bf16(self.hs[l - 1].data_ptr(), None, self.cfg.eps, self.cfg.hidden,
                                           self.xb[l].data_ptr(), self.xf[l].data_ptr(), s), "rmsnorm_bf16")

    def _layer_resident(self, l: int, s: int, norm: bool = False):
        """Resident layer: the router's bf16 logits, then gate/up whose blocks select the top k
        themselves (the router's rule, bit for bit), then the down product with the bf16 scores."""
        c, L = self.cfg, self.L
        self._router_call(l, s, norm, 0, None, None, self.logits[l].data_ptr())
        _, ptrs, nbytes = self.full[l]
        _lib.check(L.moe_q2t_gate_up_routed(self.xf[l].data_ptr(), self.logits[l].data_ptr(), c.n_exp, c.top_k, ptrs,
                                            nbytes, self.scale_bf16, c.hidden, c.inter, c.group, self.ids[l].data_ptr(),
                                            self.scores[l].data_ptr(), self.h_ws.data_ptr(), s), "q2t_gate_up_routed")
        _lib.check(L.moe_q2t_down(self.h_ws.data_ptr(), ptrs, nbytes, self.scale_bf16 | 2, c.n_exp,
                                  self.ids[l].data_ptr(), self.scores[l].data_ptr(), c.top_k, c.hidden, c.inter,
                                  c.group, self.xf[l].data_ptr(), self.hs[l].data_ptr(), 0, s), "q2t_down")

    def decode_token_device(self):
        """Device-driven token (DecodeStack's device path with the checkpoint's kernels): main stream
        (norm in) router (+ predictor) -> [join prefetch table(l)] -> step(l) -> [join prefetch
        copies(l)] -> demand copies(l) -> SwitchGLU; side stream: prefetch table(l+1), then its copies
        once layer l's demand copies are queued."""
        c, L = self.cfg, self.L
        main = torch.cuda.current_stream()
        ms = main.cuda_stream
        fuse = c.fused_norm
        for l in range(c.n_layers):
            if l > 0 and not fuse:
                self._norm(l, ms)
            if self.resident:
                self._layer_resident(l, ms, norm=fuse and l > 0)
                continue
            self._router(l, ms, norm=fuse and l > 0)
            if l >= 1:
                if c.prefetch:
                    main.wait_event(self.ev_pref[l])
                _lib.check(L.c_layer_step_decode_dev(self.cidx(l), self.ids[l].data_ptr(), c.top_k, -1, ms), "step_dev")
            pf = c.prefetch and l + 1 < c.n_layers
            if pf:
                self.ev_pred[l].record(main)
                self.side.wait_event(self.ev_pred[l])
                _lib.check(L.c_layer_start_prefetch_dev(self.cidx(l + 1), self.pred[l].data_ptr(), c.top_m,
                                                        c.prefetch_cap, -1, self.side.cuda_stream), "prefetch_dev")
                self.ev_pref[l + 1].record(self.side)
            if l >= 1:
                if c.prefetch:
                    main.wait_event(self.ev_copy[l])
                _lib.check(L.c_layer_stage_dev(self.cidx(l), 0, c.stage_ctas, ms), "stage_demand")
            if pf:
                self.ev_demand[l].record(main)
                self.side.wait_event(self.ev_demand[l])
                _lib.check(L.c_layer_stage_dev(self.cidx(l + 1), 1, c.stage_ctas, self.side.cuda_stream),
                           "stage_prefetch")
                self.ev_copy[l + 1].record(self.side)
            self._glu(l, ms)
        self._norm(c.n_layers, ms)

    def decode_token_host(self):
        """The reference's token (loader.py:920-977): per cached layer one device->host read of the
        ids and the prediction, the host table's step, the SwitchGLU (ordered after the step's
        copies), then the next layer's prefetch."""
        c, L = self.cfg, self.L
        main = torch.cuda.current_stream()
        ms = main.cuda_stream
        L.c_set_compute_stream(ctypes.c_void_p(ms))
        m = c.top_m
        for l in range(c.n_layers):
            if l > 0:
                self._norm(l, ms)
            self._router(l, ms)
            if l == 0:
                self._glu(0, ms)
                if c.prefetch:
                    p = self.pred[0, :m].tolist()
                    L.c_layer_start_prefetch(self.cidx(1), (ctypes.c_int32 * m)(*p), m, c.prefetch_cap)
                continue
            sel = torch.cat([self.ids[l], self.pred[l, :m]]).tolist()          # the one sync per layer
            ids, pred = sel[:c.top_k], sel[c.top_k:]
            _lib.check(L.c_layer_step_decode_ex(self.cidx(l), (ctypes.c_uint32 * c.top_k)(*ids), c.top_k, 1), "step")
            self._glu(l, ms)
            if c.prefetch and l + 1 < c.n_layers:
                L.c_layer_start_prefetch(self.cidx(l + 1), (ctypes.c_int32 * m)(*pred), m, c.prefetch_cap)
        _lib.check_error("decode_token_host")
        self._norm(c.n_layers, ms)

    def decode_token(self, x0: torch.Tensor | None = None) -> torch.Tensor:
        """One token from x0 (any float dtype; used as bf16); returns x_L (bf16 bits, int16)."""
        if x0 is not None:
            xb = x0.to(self.device, torch.bfloat16)
            self.xb[0].copy_(xb.view(torch.int16))
            self.xf[0].copy_(xb.to(torch.float16))
        if self.mode == "device":
            if self.graph is not None:
                self.graph.replay()
            else:
                self.decode_token_device()
        else:
            self.decode_token_host()
        return self.xb[self.cfg.n_layers]

    def capture_graph(self):
        assert self.mode == "device"
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

    # ---- cache state and counters (the DecodeStack interface OffloadEngine drives) -------------
    def check_io(self):
        return None

    def table_status(self) -> dict[int, int]:
        if self.mode != "device" or self.resident:
            return {}
        st = {l: self.L.c_layer_table_status(self.cidx(l)) for l in range(1, self.cfg.n_layers)}
        return {l: v for l, v in st.items() if v}

    def reset_caches(self):
        if self.resident:
            return
        for l in range(1, self.cfg.n_layers):
            self.L.c_layer_reset_cache(self.cidx(l))
        _lib.check_error("reset_cache")

    def reset_stats(self):
        if self.resident:
            return
        for l in range(1, self.cfg.n_layers):
            self.L.c_layer_reset_stats(self.cidx(l))

    def layer_stats(self, l: int) -> list[int]:
        o = (ctypes.c_uint64 * 18)()
        self.L.c_layer_get_stats(self.cidx(l), o)
        return list(o)

    def decode_totals(self) -> list[int]:
        if self.resident:
            return [0] * 6
        o = (ctypes.c_uint64 * 6)()
        self.L.c_get_decode_totals(self.cidx(self.cfg.n_layers), o)
        return list(o)

    def routed_bytes_per_token(self) -> int:
        return self.cfg.n_layers * self.cfg.top_k * self.blob_bytes

    def close(self):
        torch.cuda.synchronize()
        self.graph = None
        if self.resident:
            self.full = None
            return
        self.L.c_sync_copies()
        for l in range(1, self.cfg.n_layers):
            self.L.c_layer_init(self.cidx(l), -1, 16, None, None, None, 0)
        self.store.close()
