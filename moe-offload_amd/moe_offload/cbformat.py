"""2-bit codebook expert format (the Nemotron-style experts: non-gated up -> squared ReLU -> down).

Weights come in super-blocks of 256 along the input dimension, each with an fp16 super-scale d and
8 sub-blocks of 32 weights.  A sub-block holds four 8-weight groups: per group an 8-bit index into a
fixed seeded grid of 256 entries (8 magnitudes each, from {1, 3, 5}) and 7 sign bits, plus one 4-bit
sub-scale s for the sub-block.  Weight j of group g:

    w = d * (2 s + 1) / 8 * grid[idx_g][j] * (-1 if bit j of signs8_g else +1)
    signs8_g = sign7_g | (popcount(sign7_g) & 1) << 7      (an even number of negative weights)

This is the IQ2_XXS scheme of ggml (66 bytes per 256 weights) with the seeded grid of the workload
in place of ggml's fixed table.  The reference runs this format only inside llama.cpp
(llamacpp-bolt/llama-moe-cache.patch patches an unvendored llama.cpp), so the arithmetic above is
restated here and in the oracle, not compared with the reference.

Blob (one contiguous byte range per expert, in the HBM pool and in the host store), 16-byte aligned
planes, for hidden H and intermediate I (both multiples of 256):

    up_qs [I][H/256][8][8] | down_qs [H][I/256][8][8] | up_d [I][H/256] fp16 | down_d [H][I/256] fp16

where each 8-byte sub-block entry is 4 grid indices (bytes 0-3, group order) and a little-endian
u32 aux = sign7_0 | sign7_1 << 7 | sign7_2 << 14 | sign7_3 << 21 | s << 28.  At H=3072, I=1536 an
expert is 2,433,024 bytes.
"""
from __future__ import annotations

import numpy as np

SUPER = 256          # weights per super-block
SUB = 32             # weights per sub-block (4 groups of 8)
GRID_SEED = 240      # the workload's fixed grid: seeded, 256 entries x 8 magnitudes from {1, 3, 5}


def grid(seed: int = GRID_SEED) -> np.ndarray:
    """The seeded codebook: uint8 [256, 8] with values in {1, 3, 5}."""
    rng = np.random.default_rng(seed)
    return rng.choice(np.array([1, 3, 5], dtype=np.uint8), size=(256, 8))


def blob_offsets(hidden: int, inter: int) -> dict[str, int]:
    if hidden % SUPER or inter % SUPER:
        raise ValueError(f"hidden={hidden}, inter={inter} must be multiples of {SUPER}")
    up_qs = inter * (hidden // SUPER) * 64
    dn_qs = hidden * (inter // SUPER) * 64
    up_d = inter * (hidden // SUPER) * 2
    dn_d = hidden * (inter // SUPER) * 2
    return {"up_qs": 0, "down_qs": up_qs, "up_d": up_qs + dn_qs, "down_d": up_qs + dn_qs + up_d,
            "bytes": up_qs + dn_qs + up_d + dn_d}


def expert_bytes(hidden: int, inter: int) -> int:
    return blob_offsets(hidden, inter)["bytes"]


def pack_matrix(idx: np.ndarray, sign7: np.ndarray, sub_scale: np.ndarray, d: np.ndarray):
    """Codes of one [rows, K] matrix -> (qs uint8 [rows, K/256, 8, 8], d fp16 [rows, K/256]).

    idx, sign7: [rows, K/8] (group order along K); sub_scale: [rows, K/32] in 0..15;
    d: [rows, K/256]."""
    rows, ng = idx.shape
    nsb = ng // 32
    idx = idx.astype(np.uint32).reshape(rows, nsb, 8, 4)
    sg = sign7.astype(np.uint32).reshape(rows, nsb, 8, 4)
    ss = sub_scale.astype(np.uint32).reshape(rows, nsb, 8)
    qs = np.zeros((rows, nsb, 8, 8), dtype=np.uint8)
    qs[..., 0:4] = idx.astype(np.uint8)
    aux = sg[..., 0] | (sg[..., 1] << 7) | (sg[..., 2] << 14) | (sg[..., 3] << 21) | (ss << 28)
    qs[..., 4:8] = aux.astype("<u4")[..., None].view(np.uint8).reshape(rows, nsb, 8, 4)
    return qs, d.astype(np.float16).reshape(rows, nsb)


def unpack_matrix(qs: np.ndarray, d: np.ndarray):
    """Inverse of pack_matrix -> (idx, sign7, sub_scale, d)."""
    rows, nsb = qs.shape[:2]
    idx = qs[..., 0:4].reshape(rows, nsb * 32).astype(np.int32)
    aux = np.ascontiguousarray(qs[..., 4:8]).view("<u4")[..., 0].astype(np.uint32)     # [rows, nsb, 8]
    sign7 = np.stack([(aux >> (7 * g)) & 0x7F for g in range(4)], axis=-1).reshape(rows, nsb * 32)
    sub = (aux >> 28).reshape(rows, nsb * 8)
    return idx, sign7.astype(np.int32), sub.astype(np.int32), d


def to_blob(up: tuple, down: tuple, hidden: int, inter: int) -> np.ndarray:
    """One expert's (idx, sign7, sub_scale, d) for up [I, H] and down [H, I] -> blob bytes."""
    o = blob_offsets(hidden, inter)
    b = np.zeros(o["bytes"], dtype=np.uint8)
    uq, ud = pack_matrix(*up)
    dq, dd = pack_matrix(*down)
    b[o["up_qs"]:o["down_qs"]] = uq.reshape(-1)
    b[o["down_qs"]:o["up_d"]] = dq.reshape(-1)
    b[o["up_d"]:o["down_d"]] = ud.reshape(-1).view(np.uint8)
    b[o["down_d"]:] = dd.reshape(-1).view(np.uint8)
    return b


def from_blob(blob: np.ndarray, hidden: int, inter: int):
    """Blob -> ((idx, sign7, sub_scale, d) of up, same of down)."""
    o = blob_offsets(hidden, inter)
    blob = np.asarray(blob, dtype=np.uint8)
    nh, ni = hidden // SUPER, inter // SUPER
    uq = blob[o["up_qs"]:o["down_qs"]].reshape(inter, nh, 8, 8)
    dq = blob[o["down_qs"]:o["up_d"]].reshape(hidden, ni, 8, 8)
    ud = blob[o["up_d"]:o["down_d"]].view(np.float16).reshape(inter, nh)
    dd = blob[o["down_d"]:o["bytes"]].view(np.float16).reshape(hidden, ni)
    return unpack_matrix(uq, ud), unpack_matrix(dq, dd)


def random_codes(rows: int, k: int, rng: np.random.Generator, d_scale: float = 0.01):
    """Random codes for a [rows, k] matrix: uniform grid indices, signs and sub-scales, and
    d ~ |N(0, d_scale)| (fp16)."""
    ng = k // 8
    idx = rng.integers(0, 256, size=(rows, ng))
    sign7 = rng.integers(0, 128, size=(rows, ng))
    sub = rng.integers(0, 16, size=(rows, k // SUB))
    d = np.abs(rng.standard_normal((rows, k // SUPER)) * d_scale).astype(np.float16)
    return idx, sign7, sub, d


def random_blobs(n_exp: int, hidden: int, inter: int, seed: int = 0, d_scale: float = 0.01) -> np.ndarray:
    rng = np.random.default_rng(seed)
    out = np.zeros((n_exp, expert_bytes(hidden, inter)), dtype=np.uint8)
    for e in range(n_exp):
        out[e] = to_blob(random_codes(inter, hidden, rng, d_scale), random_codes(hidden, inter, rng, d_scale),
                         hidden, inter)
    return out
