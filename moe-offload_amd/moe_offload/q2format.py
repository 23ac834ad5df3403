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


# ---- on-disk tier ------------------------------------------------------------------------------
#
# Expert blob file: a 4 KiB header, then [n_exp][blob] at offset 4096 (page aligned), so a miss is
# one pread of one contiguous blob.  Header (little endian): magic "MOEQ2BLB", u32 version (1),
# u32 n_exp, u32 hidden, u32 inter, u32 group, u32 reserved, u64 blob bytes, u64 data offset.

BLOB_MAGIC = b"MOEQ2BLB"
BLOB_DATA_OFFSET = 4096


def write_blob_file(path, blobs: np.ndarray, hidden: int, inter: int, group: int = 64) -> None:
    blobs = np.ascontiguousarray(blobs, np.uint8)
    n, nb = blobs.shape
    if nb != expert_bytes(hidden, inter, group):
        raise ValueError(f"blob size {nb} != {expert_bytes(hidden, inter, group)} for {hidden}x{inter} g{group}")
    hdr = np.zeros(BLOB_DATA_OFFSET, np.uint8)
    hdr[:8] = np.frombuffer(BLOB_MAGIC, np.uint8)
    hdr[8:32] = np.array([1, n, hidden, inter, group, 0], "<u4").view(np.uint8)
    hdr[32:48] = np.array([nb, BLOB_DATA_OFFSET], "<u8").view(np.uint8)
    with open(path, "wb") as f:
        f.write(hdr.tobytes())
        f.write(blobs.tobytes())


def read_blob_header(path) -> dict:
    with open(path, "rb") as f:
        raw = f.read(48)
    if len(raw) < 48 or raw[:8] != BLOB_MAGIC:
        raise ValueError(f"{path}: not an expert blob file")
    version, n, hidden, inter, group, _ = np.frombuffer(raw[8:32], "<u4").tolist()
    nb, off = np.frombuffer(raw[32:48], "<u8").tolist()
    if version != 1 or nb != expert_bytes(hidden, inter, group):
        raise ValueError(f"{path}: unsupported version {version} or inconsistent blob size")
    return {"n_exp": n, "hidden": hidden, "inter": inter, "group": group, "blob_bytes": nb, "data_offset": off}


def _safetensors_header(path):
    """(header dict, data start) of a safetensors file -- the same parse as loader.py:316-318."""
    import json
    with open(path, "rb") as f:
        hsize = int(np.frombuffer(f.read(8), "<u8")[0])
        hdr = json.loads(f.read(hsize))
    return hdr, 8 + hsize


def _half_from(raw: np.ndarray, dtype: str) -> np.ndarray:
    """bf16 / f16 bits (uint16) -> float16, refusing values that do not convert exactly."""
    if dtype == "F16":
        return raw.view(np.float16)
    if dtype != "BF16":
        raise ValueError(f"scales/biases dtype {dtype} unsupported (BF16 or F16)")
    f32 = (raw.astype(np.uint32) << 16).view(np.float32)
    h = f32.astype(np.float16)
    if not np.array_equal(h.astype(np.float32), f32):
        bad = int(np.sum(h.astype(np.float32) != f32))
        raise ValueError(f"{bad} bf16 scale/bias values are not exact in fp16")
    return h


def reference_layer_to_blobs(path, layer: int, hidden: int, inter: int, group: int = 64,
                             prefix: str = "language_model.model.layers.{layer}.mlp.switch_mlp") -> np.ndarray:
    """Blobs [E, bytes] of one layer from a reference `experts-XX.safetensors` shard.

    Tensor names and layout as `mlx-qwen38/loader.py:336-366`: `{prefix}.{gate,up,down}_proj.
    {weight,scales,biases}`, weight U32 [E, out, in/16], scales/biases BF16 (or F16) [E, out, in/g].
    Read with plain file reads at the header's offsets (nothing in the file is executed).
    """
    hdr, start = _safetensors_header(path)
    pre = prefix.format(layer=layer)
    shapes = {"gate_proj": (inter, hidden), "up_proj": (inter, hidden), "down_proj": (hidden, inter)}
    parts = {}
    with open(path, "rb") as f:
        for proj, (out_f, in_f) in shapes.items():
            trip = []
            for suffix in ("weight", "scales", "biases"):
                info = hdr[f"{pre}.{proj}.{suffix}"]
                a, b = info["data_offsets"]
                f.seek(start + a)
                raw = np.frombuffer(f.read(b - a), np.uint8)
                shp = tuple(info["shape"])
                if suffix == "weight":
                    if info["dtype"] != "U32" or shp[1:] != (out_f, in_f // 16):
                        raise ValueError(f"{pre}.{proj}.weight: {info['dtype']} {shp}")
                    trip.append(raw.view("<u4").reshape(shp))
                else:
                    if shp[1:] != (out_f, in_f // group):
                        raise ValueError(f"{pre}.{proj}.{suffix}: shape {shp}")
                    trip.append(_half_from(raw.view("<u2"), info["dtype"]).reshape(shp))
            parts[proj] = tuple(trip)
    return to_blobs(parts["gate_proj"], parts["up_proj"], parts["down_proj"], hidden, inter, group)
