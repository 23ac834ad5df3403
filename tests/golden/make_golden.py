#!/usr/bin/env python3
"""Extract the routed-expert golden vectors from the reference's own test fixture file.

Reads `mlx-qwen38/cpp/tests/fixtures.safetensors` (a data file that the reference's
`cpp/tests/test_kernels.cpp` checks against; written by `cpp/tests/gen_fixtures.py:474-573,680-703`)
purely as bytes -- safetensors is a JSON header plus raw little-endian arrays, so nothing in the
file is executed -- and keeps the tensors that pin the router, the prefetch predictor and the
2-bit SwitchGLU: `moe.*`, `pred_next.*` and the two hyper-connection mixer outputs that feed
the predictor (`hc.r1.m_nowrite`, `hc.r1.m_write`).

bf16 tensors are stored as their raw uint16 bit patterns.

Run in the build container only (the reference tree is not present on the GPU machines):
    python tests/golden/make_golden.py
"""
from __future__ import annotations

import json
import struct
import sys
from pathlib import Path

import numpy as np

SRC = Path("/root/reference/mlx-qwen38/cpp/tests/fixtures.safetensors")
OUT = Path(__file__).resolve().parent / "moe_fixture.npz"

_DT = {"BF16": np.uint16, "F16": np.float16, "F32": np.float32, "U32": np.uint32,
       "I32": np.int32, "I64": np.int64, "U8": np.uint8}


def read_safetensors(path: Path, keep) -> dict[str, np.ndarray]:
    raw = path.read_bytes()
    (hlen,) = struct.unpack("<Q", raw[:8])
    hdr = json.loads(raw[8:8 + hlen])
    base = 8 + hlen
    out = {}
    for name, info in hdr.items():
        if name == "__metadata__" or not keep(name):
            continue
        a, b = info["data_offsets"]
        arr = np.frombuffer(raw[base + a: base + b], dtype=_DT[info["dtype"]]).reshape(info["shape"])
        out[name] = arr.copy()
        out[name + "@dtype"] = np.array(info["dtype"])
    return out


def main() -> int:
    if not SRC.exists():
        print(f"missing {SRC}", file=sys.stderr)
        return 1
    keep = lambda n: n.startswith("moe.") or n.startswith("pred_next.") or n in (
        "hc.r1.m_nowrite", "hc.r1.m_write")
    t = read_safetensors(SRC, keep)
    np.savez_compressed(OUT, **t)
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes, {len(t) // 2} tensors)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
