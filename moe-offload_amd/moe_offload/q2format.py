"""Q2 expert blob format (host side): conversion from the MLX/safetensors tensor layout.

The reference stores each projection of a layer's routed experts as three tensors
(`mlx-qwen38/loader.py:332-366`): `weight` [E, out, in/16] uint32 (2-bit codes, LSB first),
`scales` and `biases` [E, out, in/group].  This build keeps one contiguous blob per expert
(the layout comment in csrc/moe_common.h): the three code arrays verbatim, then the
(scale, bias) pairs interleaved per group, so one miss is one copy and one kernel load
fetches a group's codes while one 32-bit load fetches its scale and bias.
"""
from __future__ import annotations

import numpy as np


def blob_offsets(hidden: int, inter: int, group: int = 64) -> dict[str, int]:
    gu = inter * hidden // 4
    dn = hidden * inter // 4
    gsb = inter * (hidden // group) * 4
    dsb = hidden * (inter // group) * 4
    o = {"gate_codes": 0, "up_codes": gu, "down_codes": 2 * gu, "gate_sb": 2 * gu + dn}
    o["up_sb"] = o["gate_sb"] + gsb
    o["down_sb"] = o["up_sb"] + gsb
    o["bytes"] = o["down_sb"] + dsb
    return o


def expert_bytes(hidden: int, inter: int, group: int = 64) -> int:
    return blob_offsets(hidden, inter, group)["bytes"]


def _sb(scales: np.ndarray, biases: np.ndarray) -> np.ndarray:
    s = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16).astype(np.uint32)
    b = np.ascontiguousarray(biases, dtype=np.float16).view(np.uint16).astype(np.uint32)
    return (s | (b << 16)).astype(np.uint32)


def to_blobs(gate, up, down, hidden: int, inter: int, group: int = 64, out: np.ndarray | None = None) -> np.ndarray:
    """gate/up/down = (w [E,out,in/16] u32, s [E,out,in/g] f16, b [E,out,in/g] f16) -> uint8 [E, bytes]."""
    n = gate[0].shape[0]
    o = blob_offsets(hidden, inter, group)
    if out is None:
        out = np.empty((n, o["bytes"]), np.uint8)
    for name, (w, s, b) in (("gate", gate), ("up", up), ("down", down)):
        cw = np.ascontiguousarray(w, dtype=np.uint32).reshape(n, -1).view(np.uint8)
        out[:, o[f"{name}_codes"]:o[f"{name}_codes"] + cw.shape[1]] = cw
        sb = _sb(s, b).reshape(n, -1).view(np.uint8)
        out[:, o[f"{name}_sb"]:o[f"{name}_sb"] + sb.shape[1]] = sb
    return out


def from_blob(blob: np.ndarray, hidden: int, inter: int, group: int = 64):
    """uint8 [bytes] -> ((w, s, b) gate, up, down) for one expert, in the MLX layout."""
    o = blob_offsets(hidden, inter, group)
    blob = np.asarray(blob, np.uint8)
    shapes = {"gate": (inter, hidden), "up": (inter, hidden), "down": (hidden, inter)}
    res = []
    for name in ("gate", "up", "down"):
        rows, cols = shapes[name]
        nw = rows * cols // 16
        w = blob[o[f"{name}_codes"]:o[f"{name}_codes"] + nw * 4].view(np.uint32).reshape(rows, cols // 16)
        ng = rows * cols // group
        sb = blob[o[f"{name}_sb"]:o[f"{name}_sb"] + ng * 4].view(np.uint32).reshape(rows, cols // group)
        s = (sb & 0xFFFF).astype(np.uint16).view(np.float16)
        b = (sb >> 16).astype(np.uint16).view(np.float16)
        res.append((w, s, b))
    return tuple(res)
