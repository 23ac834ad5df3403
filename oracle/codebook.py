"""CPU restatement of the 2-bit codebook expert path (TEST INFRASTRUCTURE ONLY: what the tests
compare the HIP codebook kernels with; never imported by the product).

Restated behaviour.  The reference runs its Nemotron model (README.md:37: IQ2_XXS GGUF, 240
experts, top-9; non-gated up -> squared ReLU -> down) only inside llama.cpp's Metal backend,
which it patches but does not vendor (llamacpp-bolt/llama-moe-cache.patch; Makefile and
bench.py there point at an external checkout).  So this follows the published algorithm of the
format, with the workload's seeded grid in place of ggml's fixed table, not reference source:

  * dequantisation (ggml IQ2_XXS): per 32-weight sub-block db = d * (0.5 + s) / 4 with d the
    super-block's fp16 scale and s its 4-bit sub-scale; weight j of an 8-weight group =
    db * grid[idx][j] * sign, the sign from bit j of sign7 | parity(sign7) << 7;
  * the Metal matrix-vector path multiplies dequantised weights with float activations:
    u = U . x, h = relu(u)^2, y = D . h, combined as y = residual + sum_j score_j * y_j.

`expert` computes in fp64; with h_bf16 it rounds h to bf16 (round to nearest even) between the
two products, as the GPU path stores it.

Parity unpinned against the reference: no golden output of this path exists (llama.cpp is not
vendored).  Pinned instead by hand-computed known answers, a brute-force loop form, the format's
invariants (even number of negative weights per group, magnitudes in grid x db, pack/unpack
round trips) and planted-mistake controls (tests/test_oracle_codebook.py).
"""
from __future__ import annotations

import numpy as np

SUPER, SUB, GROUP = 256, 32, 8


def signs8(sign7: np.ndarray) -> np.ndarray:
    """7 stored sign bits -> 8 (bit 7 = parity of the 7), so every group has an even number of
    negative weights."""
    s = np.asarray(sign7, dtype=np.int64) & 0x7F
    par = np.zeros_like(s)
    for b in range(7):
        par ^= (s >> b) & 1
    return s | (par << 7)


def int_weights(idx: np.ndarray, sign7: np.ndarray, grid: np.ndarray) -> np.ndarray:
    """[rows, K/8] codes -> signed integer weights [rows, K] (magnitudes from the grid)."""
    rows, ng = idx.shape
    mag = grid[np.asarray(idx, dtype=np.int64)].astype(np.int64)            # [rows, ng, 8]
    s8 = signs8(sign7)
    neg = (s8[..., None] >> np.arange(8)) & 1
    return (mag * (1 - 2 * neg)).reshape(rows, ng * GROUP)


def sub_scales(sub: np.ndarray, d: np.ndarray) -> np.ndarray:
    """[rows, K/32] sub-scales and [rows, K/256] fp16 d -> db [rows, K/32] (fp32-exact)."""
    d32 = np.asarray(d, dtype=np.float16).astype(np.float32)
    dd = np.repeat(d32, SUPER // SUB, axis=1)
    return dd * (2 * np.asarray(sub, dtype=np.float32) + 1) * np.float32(0.125)


def dequantize(codes, grid) -> np.ndarray:
    """(idx, sign7, sub, d) -> fp64 weights [rows, K]."""
    idx, sign7, sub, d = codes
    w = int_weights(idx, sign7, grid).astype(np.float64)
    db = sub_scales(sub, d).astype(np.float64)
    return w * np.repeat(db, SUB, axis=1)


def round_bf16(v: np.ndarray) -> np.ndarray:
    """fp32 values rounded to bf16 (nearest, ties to even), returned as float64."""
    f = np.asarray(v, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    return u.astype(np.uint32).view(np.float32).astype(np.float64)


def expert(x: np.ndarray, up_codes, down_codes, grid, h_bf16: bool = False) -> np.ndarray:
    """One expert: down . relu(up . x)^2 in fp64 (h rounded to bf16 first when h_bf16)."""
    u = dequantize(up_codes, grid) @ np.asarray(x, dtype=np.float64)
    h = np.maximum(u, 0.0) ** 2
    if h_bf16:
        h = round_bf16(h)
    return dequantize(down_codes, grid) @ h


def moe_combine(x, ids, scores, experts, grid, residual=None, h_bf16=False) -> np.ndarray:
    """residual + sum_j scores[j] * expert(ids[j])(x); experts(e) -> (up_codes, down_codes)."""
    y = np.zeros(0)
    for j, e in enumerate(ids):
        up, down = experts(int(e))
        yj = float(scores[j]) * expert(x, up, down, grid, h_bf16)
        y = yj if y.size == 0 else y + yj
    if residual is not None:
        y = y + np.asarray(residual, dtype=np.float64)
    return y


def brute_matvec(codes, grid, x) -> np.ndarray:
    """Loop form of dequantize(codes) @ x straight from the format description (small sizes)."""
    idx, sign7, sub, d = codes
    rows, ng = idx.shape
    y = np.zeros(rows)
    for r in range(rows):
        for g in range(ng):
            s7 = int(sign7[r, g]) & 0x7F
            par = bin(s7).count("1") & 1
            s8 = s7 | (par << 7)
            k0 = g * GROUP
            sb = k0 // SUB
            db = float(np.float16(d[r, k0 // SUPER])) * (0.5 + int(sub[r, sb])) * 0.25
            for j in range(GROUP):
                sign = -1.0 if (s8 >> j) & 1 else 1.0
                y[r] += db * int(grid[int(idx[r, g]), j]) * sign * float(x[k0 + j])
    return y
