"""Chunked prefill through a cached layer (loader.py:566-699) on the grouped-GEMM kernels.

The host side keeps the reference's bookkeeping step for step: read the LRU state from the
library, sort the (token, k) rows by expert, split the distinct experts into chunks of at most
`capacity`, give the expert of rank s in a chunk slot s (loading it there when the slot holds
another expert), run the grouped SwitchGLU over the chunk, and finally rebuild the LRU from the
slot bijection (last chunk at the MRU end) and push it back with the prefill counters.  The
arithmetic runs in libmoe_offload (MFMA grouped GEMM); there is no other compute path.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib

NUM_EXPERTS = 512


def sort_rows(ids: np.ndarray, k: int):
    """Stable sort of the flattened (token, k) expert ids (loader.py:583-591).

    Returns (order, idx_sorted, uniq, first_pos, counts); row r of the sorted order is pair
    order[r] = token * k + j.
    """
    flat = np.asarray(ids).reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    idx_s = flat[order]
    uniq, first_pos, counts = np.unique(idx_s, return_index=True, return_counts=True)
    return order, idx_s, uniq, first_pos, counts


def prefill_counts(uniq, counts, prior_cached) -> tuple[int, int]:
    """(hits, misses) added to the layer's prefill counters (loader.py:596-607)."""
    hits = misses = 0
    for e, c in zip(uniq.tolist(), counts.tolist()):
        if e in prior_cached:
            hits += c
        else:
            misses += 1
            hits += c - 1
    return hits, misses


def plan_chunk(chunk_eids: list[int], slot_to_eid: dict, eid_to_slot: dict):
    """Slot assignment of one chunk: slot s gets the chunk's s-th expert (loader.py:636-649).

    Updates both maps in place; returns the (eids, slots) to load.
    """
    load_e, load_s = [], []
    for s_idx, eid in enumerate(chunk_eids):
        if slot_to_eid.get(s_idx) != eid:
            old = slot_to_eid.get(s_idx)
            if old is not None and eid_to_slot.get(old) == s_idx:
                del eid_to_slot[old]
            prev = eid_to_slot.get(eid)
            if prev is not None and prev != s_idx:
                slot_to_eid.pop(prev, None)
            slot_to_eid[s_idx] = eid
            eid_to_slot[eid] = s_idx
            load_e.append(eid)
            load_s.append(s_idx)
    return load_e, load_s


def final_lru(slot_to_eid: dict, last_chunk_len: int, capacity: int):
    """LRU -> MRU (eids, slots) after prefill: slots past the last chunk first, then the last
    chunk in slot order (loader.py:677-683)."""
    eids, slots = [], []
    for s_idx in list(range(last_chunk_len, capacity)) + list(range(last_chunk_len)):
        if s_idx in slot_to_eid:
            eids.append(slot_to_eid[s_idx])
            slots.append(s_idx)
    return eids, slots


def cached_prefill(module, x: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
    """Per-(token, k) SwitchGLU outputs of a cached layer for L > 1 tokens.

    x: [..., hidden] (any float dtype; computed from its fp16 rounding), indices: [..., k] expert
    ids.  Returns fp16 [..., k, hidden] like the reference's `_scatter_unsort` output.
    """
    L = _lib.lib()
    layer, cap, H = module.layer_idx, module.capacity, module.hidden
    k = int(indices.shape[-1])
    ids = indices.reshape(-1).to(torch.int64).cpu().numpy()
    if ids.size and (ids.min() < 0 or ids.max() >= NUM_EXPERTS):
        raise ValueError("expert id out of range")
    n_tok = ids.size // k
    xs = x.reshape(n_tok, H).to(torch.float16).contiguous()
    dev = xs.device

    out_e = (ctypes.c_int32 * NUM_EXPERTS)()
    out_s = (ctypes.c_int32 * NUM_EXPERTS)()
    out_n = ctypes.c_int(0)
    L.c_layer_get_lru_state(layer, out_e, out_s, ctypes.byref(out_n))
    _lib.check_error("c_layer_get_lru_state")
    lru = [(int(out_e[i]), int(out_s[i])) for i in range(out_n.value)]

    order, _, uniq, first_pos, counts = sort_rows(ids, k)
    M = ids.size
    hits, misses = prefill_counts(uniq, counts, {e for e, _ in lru})
    slot_to_eid = {s: e for e, s in lru}
    eid_to_slot = {e: s for e, s in lru}

    n_uniq = len(uniq)
    chunks = []
    seg_host = []
    for u0 in range(0, n_uniq, cap):
        u1 = min(n_uniq, u0 + cap)
        p0 = int(first_pos[u0])
        p1 = int(first_pos[u1 - 1] + counts[u1 - 1])
        seg = np.append(first_pos[u0:u1] - p0, p1 - p0).astype(np.int32)
        chunks.append((u0, u1, p0, p1, len(seg_host)))
        seg_host.extend(seg.tolist())

    y = torch.empty((M, H), dtype=torch.float16, device=dev)
    if M:
        row_tok = torch.from_numpy((order // k).astype(np.int32)).to(dev)
        row_out = torch.from_numpy(order.astype(np.int32)).to(dev)
        seg_dev = torch.tensor(seg_host, dtype=torch.int32, device=dev)
        max_rows = max(p1 - p0 for _, _, p0, p1, _ in chunks)
        h_ws = torch.empty((max_rows, module.inter), dtype=torch.float16, device=dev)
        stream = torch.cuda.current_stream(dev).cuda_stream
        for u0, u1, p0, p1, so in chunks:
            le, ls = plan_chunk([int(e) for e in uniq[u0:u1]], slot_to_eid, eid_to_slot)
            if le:
                n = len(le)
                L.c_layer_load_sync(layer, (ctypes.c_int32 * n)(*le), (ctypes.c_int32 * n)(*ls), n, 1)
                _lib.check_error("c_layer_load_sync")
            rc = L.c_layer_grouped_switch_glu(layer, xs.data_ptr(), n_tok, row_tok.data_ptr() + 4 * p0,
                                              row_out.data_ptr() + 4 * p0, p1 - p0, M, seg_dev.data_ptr() + 4 * so,
                                              u1 - u0, h_ws.data_ptr(), y.data_ptr(), stream)
            _lib.check(rc, "c_layer_grouped_switch_glu")

    last_len = (chunks[-1][1] - chunks[-1][0]) if chunks else 0
    ne, ns = final_lru(slot_to_eid, last_len, cap)
    n = len(ne)
    L.c_layer_set_lru_state(layer, (ctypes.c_int32 * max(n, 1))(*ne), (ctypes.c_int32 * max(n, 1))(*ns), n, M,
                            hits, misses)
    _lib.check_error("c_layer_set_lru_state")
    return y.reshape(*indices.shape, H)


def tile_segments(seg_start: np.ndarray, seg_slot: np.ndarray, rows: int = 16):
    """The same sorted rows cut into segments of at most `rows` rows, each keeping its expert's slot.

    For the blob pool's gate/up at hidden 2048 (the whole-K form): that kernel gives every
    (segment, 128-row slice) one block that takes the segment's 16-row M tiles one after the
    other; an expert of several tiles given as several one-tile segments runs as neighbouring
    blocks on one XCD instead, which read its weights together (from L2 after the first) rather
    than one block re-reading them per tile.  Outputs are bit-identical (each tile is multiplied
    the same way).  The chunked kernels (down, other shapes) multiply two tiles per weight pass
    and are faster over the expert segments.  Empty segments are dropped.
    Returns int32 (seg_start', seg_slot').
    """
    seg_start = np.asarray(seg_start, dtype=np.int64)
    seg_slot = np.asarray(seg_slot, dtype=np.int64)
    counts = np.diff(seg_start)
    if counts.size != seg_slot.size:
        raise ValueError("seg_start must have one more entry than seg_slot")
    if np.any(counts < 0) or rows <= 0:
        raise ValueError("segments must be ascending and rows positive")
    pieces = (counts + rows - 1) // rows
    n = int(pieces.sum())
    first_piece = np.cumsum(pieces) - pieces
    within = np.arange(n) - np.repeat(first_piece, pieces)
    starts = np.repeat(seg_start[:-1], pieces) + rows * within
    return (np.append(starts, seg_start[-1]).astype(np.int32), np.repeat(seg_slot, pieces).astype(np.int32))


def resident_plan(ids: np.ndarray, k: int):
    """Row plan for a pool holding every expert at slot = expert id (the pinned layer 0).

    Returns int32 arrays (row_token, row_out, seg_start, seg_slot) for the grouped kernels.
    """
    order, _, uniq, first_pos, _ = sort_rows(ids, k)
    m = order.size
    return ((order // k).astype(np.int32), order.astype(np.int32),
            np.append(first_pos, m).astype(np.int32), uniq.astype(np.int32))
