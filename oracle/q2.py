"""numpy restatement of the routed-expert math -- test infrastructure only (see __init__).

Format (MLX affine quantisation, as the reference stores it):
  weight  [out, in*bits/32] uint32, codes packed LSB-first, 32/bits codes per word
          (`mlx-qwen38/cpp/tools/convert_v4_2bit.py:43-56`, `cpp/src/loader.cpp:1413-1427`)
  scales  [out, in/group]   fp16 or bf16
  biases  [out, in/group]   fp16 or bf16
  W[o, i] = scales[o, i // group] * q[o, i] + biases[o, i // group]

Router rule (`mlx-qwen38/loader.py:903-908`, `cpp/src/layers.cpp:311-325`):
  logits = round(x . W^T); gates = round(softmax(logits)); the top-k are the last k of a
  stable ascending argsort of the gates (ids come out in ascending-gate order, equal gates in
  ascending id, so at the k boundary the higher id wins); scores = round(g / round(sum g)).
Predictor (`loader.py:237-242`, `layers.cpp:327-341`): top-m of the raw logits, selected by
  the same stable ascending rule, emitted in descending value order (equal values keep
  ascending id order).

Arithmetic convention shared with the HIP kernels: dot products, the softmax and RMSNorm are
evaluated in float64 and rounded once, directly, to fp16, so that two correct implementations
agree bit for bit on every rounded value.

Pinning:
  dequant / SwitchGLU  -> golden `moe.y_dec`, `moe.y_pre` (fixtures.safetensors) within
                          tolerance, plus closed forms (codes 0..3 round trip, W = s*q + b on
                          hand-built words) in tests/test_oracle_q2.py
  router ids/scores    -> golden `moe.inds_dec/scores_dec`, `moe.inds_pre/scores_pre`, exact
  predictor            -> golden `pred_next.top12_nowrite/_write`, exact; tie rule by brute force
  prefill bookkeeping  -> reference test shapes of `test_prefill_qproj.py:79-81` and invariants
"""
from __future__ import annotations

import numpy as np

# ----------------------------------------------------------------------------------------
# dtype helpers
# ----------------------------------------------------------------------------------------


def bf16_bits_to_f32(u16: np.ndarray) -> np.ndarray:
    return (np.asarray(u16, dtype=np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit pattern."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u >> 16) & 1) + 0x7FFF
    return ((u + r) >> 16).astype(np.uint16)


def round_to(x: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64 values to `dtype`; returns float64.

    'f16' rounds once, directly from float64 (round-to-nearest-even), as the HIP kernels do;
    'bf16' goes through float32 like MLX's fp32 compute followed by a cast."""
    x64 = np.asarray(x, dtype=np.float64)
    if dtype == "f16":
        return x64.astype(np.float16).astype(np.float64)
    x32 = x64.astype(np.float32)
    if dtype == "f32":
        return x32.astype(np.float64)
    if dtype == "bf16":
        return bf16_bits_to_f32(f32_to_bf16_bits(x32)).astype(np.float64)
    raise ValueError(dtype)


def round_bf16_once(x: np.ndarray) -> np.ndarray:
    """float64 -> bf16 bit patterns with ONE round-to-nearest-even from float64 (no float32 step):
    the 53-bit significand is cut to bf16's 8 bits on the integer bit pattern (ties to even), then
    the exactly representable result is read off its float32 form.  Normal-range values (the
    RMSNorm glue's outputs); the checkpoint glue's kernel rounds this way."""
    b = np.ascontiguousarray(np.asarray(x, np.float64)).view(np.uint64).copy()
    cut = np.uint64(45)                               # 52 - 7 fraction bits dropped
    rem = b & np.uint64((1 << 45) - 1)
    half = np.uint64(1 << 44)
    keep = b >> cut
    up = (rem > half) | ((rem == half) & ((keep & np.uint64(1)) == np.uint64(1)))
    r = ((keep + up.astype(np.uint64)) << cut).view(np.float64)
    return f32_to_bf16_bits(r.astype(np.float32))


def to_f64(a: np.ndarray, dtype: str | None = None) -> np.ndarray:
    """Interpret an array (float16/float32, or uint16 bf16 bits when dtype='bf16') as float64."""
    if dtype == "bf16" or (dtype is None and np.asarray(a).dtype == np.uint16):
        return bf16_bits_to_f32(a).astype(np.float64)
    return np.asarray(a).astype(np.float64)


# ----------------------------------------------------------------------------------------
# affine group quantisation (MLX layout)
# ----------------------------------------------------------------------------------------


def unpack_codes(w: np.ndarray, bits: int) -> np.ndarray:
    """[.., n_words] uint32 -> [.., n_words*32/bits] uint8 codes, LSB-first within each word."""
    w = np.asarray(w, dtype=np.uint32)
    per = 32 // bits
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    codes = (w[..., None] >> shifts) & np.uint32((1 << bits) - 1)
    return codes.reshape(*w.shape[:-1], w.shape[-1] * per).astype(np.uint8)


def pack_codes(q: np.ndarray, bits: int) -> np.ndarray:
    """Inverse of unpack_codes."""
    q = np.asarray(q, dtype=np.uint32)
    per = 32 // bits
    q = q.reshape(*q.shape[:-1], q.shape[-1] // per, per)
    shifts = (np.arange(per, dtype=np.uint32) * bits)
    return np.bitwise_or.reduce(q << shifts, axis=-1).astype(np.uint32)


def dequantize(w, scales, biases, bits: int, group: int, sdtype: str | None = None) -> np.ndarray:
    """W = s*q + b in float64 (exact for fp16/bf16 s, b and small integer q)."""
    q = unpack_codes(w, bits).astype(np.float64)
    s = np.repeat(to_f64(scales, sdtype), group, axis=-1)
    b = np.repeat(to_f64(biases, sdtype), group, axis=-1)
    return s * q + b


def qmatvec(x, w, scales, biases, bits: int, group: int, sdtype: str | None = None) -> np.ndarray:
    """y[..., o] = sum_i x[..., i] * W[o, i] in float64 (gather_qmm / quantized_matmul, transpose=True)."""
    W = dequantize(w, scales, biases, bits, group, sdtype)
    return np.asarray(x, dtype=np.float64) @ W.T


# ----------------------------------------------------------------------------------------
# router, predictor
# ----------------------------------------------------------------------------------------


def softmax64(logits: np.ndarray) -> np.ndarray:
    l = np.asarray(logits, dtype=np.float64)
    e = np.exp(l - l.max(axis=-1, keepdims=True))
    return e / e.sum(axis=-1, keepdims=True)


def topk_ascending(vals: np.ndarray, k: int) -> np.ndarray:
    """Last k of a stable ascending argsort along the last axis (MLX argpartition order)."""
    order = np.argsort(vals, axis=-1, kind="stable")
    return order[..., -k:]


def seq_sum(vals: np.ndarray, dtype: str) -> np.ndarray:
    """Left-to-right sum along the last axis with every partial rounded to `dtype`.

    This is how the renormalising `scores.sum(axis=-1)` of `loader.py:908` comes out of MLX
    for a short row: it reproduces 21/21 golden rows where one exact, rounded-once sum
    reproduces 16/21 (tests/test_oracle_q2.py)."""
    acc = np.zeros(vals.shape[:-1] + (1,), np.float64)
    for j in range(vals.shape[-1]):
        acc = round_to(acc + vals[..., j:j + 1], dtype)
    return acc


def route(logits_rounded: np.ndarray, k: int, dtype: str):
    """Router rule on already-rounded logits. Returns (inds uint32 [..,k], scores float64 [..,k], gates)."""
    gates = round_to(softmax64(logits_rounded), dtype)
    inds = topk_ascending(gates, k)
    g = np.take_along_axis(gates, inds, axis=-1)
    denom = seq_sum(g, dtype)
    scores = round_to(g / denom, dtype)
    return inds.astype(np.uint32), scores, gates


def router_logits(x, w_router, dtype: str) -> np.ndarray:
    """fp16/bf16 dense router: round(x . W^T) with float64 accumulation."""
    return round_to(np.asarray(x, np.float64) @ np.asarray(w_router, np.float64).T, dtype)


def predict_topm(logits_rounded: np.ndarray, m: int) -> np.ndarray:
    """topk_sorted_indices: stable-ascending selection, then stable sort by descending value."""
    part = topk_ascending(logits_rounded, m)
    vals = np.take_along_axis(logits_rounded, part, axis=-1)
    order = np.argsort(-vals, axis=-1, kind="stable")
    return np.take_along_axis(part, order, axis=-1).astype(np.int32)


# ----------------------------------------------------------------------------------------
# SwitchGLU
# ----------------------------------------------------------------------------------------


def silu(x):
    return x / (1.0 + np.exp(-x))


def switch_glu_expert(x, gate, up, down, bits=2, group=64, sdtype=None, act_dtype: str | None = None):
    """One expert: down(silu(gate.x) * up.x).  gate/up/down are (w, s, b) triples for one expert.

    act_dtype=None keeps everything in float64 (the build's fp32-accumulation contract);
    act_dtype='bf16'/'f16' rounds the projection outputs and the activation like MLX's
    gather_qmm -> compiled SwiGLU -> gather_qmm chain does (`cpp/src/kernels.cpp:1090-1094`).
    """
    g = qmatvec(x, *gate, bits, group, sdtype)
    u = qmatvec(x, *up, bits, group, sdtype)
    if act_dtype is not None:
        g, u = round_to(g, act_dtype), round_to(u, act_dtype)
        a = round_to(round_to(silu(g), act_dtype) * u, act_dtype)
    else:
        a = silu(g) * u
    y = qmatvec(a, *down, bits, group, sdtype)
    return round_to(y, act_dtype) if act_dtype is not None else y


def moe_combine(x, inds, scores, experts, **kw):
    """sum_j scores[j] * SwitchGLU_{inds[j]}(x) for one token; experts(e) -> (gate, up, down)."""
    y = 0.0
    for e, s in zip(np.asarray(inds).ravel(), np.asarray(scores).ravel()):
        y = y + float(s) * switch_glu_expert(x, *experts(int(e)), **kw)
    return y


# ----------------------------------------------------------------------------------------
# decode stack layer (builder-defined glue: residual + RMSNorm between MoE layers)
# ----------------------------------------------------------------------------------------


def rmsnorm(h, weight, eps=1e-6):
    h = np.asarray(h, np.float64)
    return h / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps) * np.asarray(weight, np.float64)


# ----------------------------------------------------------------------------------------
# prefill bookkeeping (loader.py:566-699 / cpp/src/layers.cpp:403-600)
# ----------------------------------------------------------------------------------------


def prefill_plan(indices: np.ndarray, lru_eids, lru_slots, capacity: int):
    """Chunk/slot plan of the offloaded prefill path.

    indices: [M] flattened (token, k) expert ids in token-major order.
    lru_eids/lru_slots: LRU->MRU resident state before the call.
    Returns dict with: order (stable argsort of ids), uniq, first_pos, counts, chunks = list of
    (u0, u1, load_eids, load_slots), new_lru (eids, slots) LRU->MRU, add_req/add_hits/add_misses.
    """
    idx = np.asarray(indices).ravel().astype(np.int64)
    M = idx.size
    order = np.argsort(idx, kind="stable")
    idx_s = idx[order]
    uniq, first_pos, counts = np.unique(idx_s, return_index=True, return_counts=True)
    prior = set(int(e) for e in lru_eids)
    add_hits = add_misses = 0
    for e, c in zip(uniq, counts):
        if int(e) in prior:
            add_hits += int(c)
        else:
            add_misses += 1
            add_hits += int(c) - 1
    slot_to_eid = {int(s): int(e) for e, s in zip(lru_eids, lru_slots)}
    eid_to_slot = {int(e): int(s) for e, s in zip(lru_eids, lru_slots)}
    chunks = []
    last_len = 0
    n = len(uniq)
    for u0 in range(0, n, capacity):
        u1 = min(n, u0 + capacity)
        ce = [int(e) for e in uniq[u0:u1]]
        last_len = len(ce)
        le, ls = [], []
        for s_idx, e in enumerate(ce):
            if slot_to_eid.get(s_idx) != e:
                old = slot_to_eid.get(s_idx)
                if old is not None and eid_to_slot.get(old) == s_idx:
                    del eid_to_slot[old]
                prev = eid_to_slot.get(e)
                if prev is not None and prev != s_idx:
                    slot_to_eid.pop(prev, None)
                slot_to_eid[s_idx] = e
                eid_to_slot[e] = s_idx
                le.append(e)
                ls.append(s_idx)
        chunks.append((u0, u1, le, ls))
    new_e, new_s = [], []
    for s_idx in list(range(last_len, capacity)) + list(range(last_len)):
        if s_idx in slot_to_eid:
            new_e.append(slot_to_eid[s_idx])
            new_s.append(s_idx)
    return dict(order=order, idx_sorted=idx_s, uniq=uniq, first_pos=first_pos, counts=counts,
                chunks=chunks, new_lru=(new_e, new_s), add_req=M, add_hits=add_hits,
                add_misses=add_misses)


def k_hdr(rows: int, cap: int) -> int:
    """prefill_qproj.py:25 -- slots visible to the sorted gather_qmm fast path."""
    return max(1, min(cap, max(rows, 16) // 4))
