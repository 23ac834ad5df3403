"""On-disk tier (host side): the reference's expert shard layout converted to blobs, and the
blob file format.

A synthetic `experts-XX.safetensors` shard is written with the reference's tensor names and
dtypes (`mlx-qwen38/loader.py:336-366`: U32 codes [E, out, in/16], BF16 scales/biases
[E, out, in/64]) by the safetensors library itself; the converter must give exactly the blobs of
the same tensors, and the blob file must round-trip.  No GPU needed.
"""
import numpy as np
import pytest

from moe_offload import q2format, synth

torch = pytest.importorskip("torch")
st_torch = pytest.importorskip("safetensors.torch")

H, I, E = 256, 128, 8


def _bf16_exact(shape, rng):
    # bf16 values in the fp16 normal range (exactly representable in fp16)
    v = (rng.standard_normal(shape) * 0.02).astype(np.float32)
    v = np.where(np.abs(v) < 1e-4, 1e-4, v).astype(np.float32)
    return torch.from_numpy(v).to(torch.bfloat16)


def _shard(tmp_path, layer, rng):
    gate, up, down = synth.q2_experts(E, H, I, seed=3)
    tensors, ref = {}, {}
    pre = f"language_model.model.layers.{layer}.mlp.switch_mlp"
    for name, (w, _, _) in (("gate_proj", gate), ("up_proj", up), ("down_proj", down)):
        s = _bf16_exact(w.shape[:2] + (w.shape[2] * 16 // 64,), rng)
        b = _bf16_exact(s.shape, rng)
        tensors[f"{pre}.{name}.weight"] = torch.from_numpy(w.view(np.int32)).view(torch.uint32) \
            if hasattr(torch, "uint32") else torch.from_numpy(w.view(np.int32))
        tensors[f"{pre}.{name}.scales"] = s
        tensors[f"{pre}.{name}.biases"] = b
        ref[name] = (w, s.float().numpy().astype(np.float16), b.float().numpy().astype(np.float16))
    path = tmp_path / "experts-00.safetensors"
    st_torch.save_file(tensors, str(path))
    return path, ref


def test_reference_shard_to_blobs(tmp_path):
    rng = np.random.default_rng(0)
    path, ref = _shard(tmp_path, 7, rng)
    got = q2format.reference_layer_to_blobs(path, 7, H, I)
    want = q2format.to_blobs(ref["gate_proj"], ref["up_proj"], ref["down_proj"], H, I)
    assert np.array_equal(got, want)
    g, u, d = q2format.from_blob(got[3], H, I)
    assert np.array_equal(g[0], ref["gate_proj"][0][3]) and np.array_equal(d[2], ref["down_proj"][2][3])


def test_blob_file_round_trip(tmp_path):
    blobs = np.random.default_rng(1).integers(0, 256, (E, q2format.expert_bytes(H, I)), dtype=np.uint8)
    p = tmp_path / "layer.q2blob"
    q2format.write_blob_file(p, blobs, H, I)
    h = q2format.read_blob_header(p)
    assert h == {"n_exp": E, "hidden": H, "inter": I, "group": 64, "blob_bytes": blobs.shape[1],
                 "data_offset": q2format.BLOB_DATA_OFFSET}
    raw = np.fromfile(p, np.uint8)
    assert np.array_equal(raw[h["data_offset"]:].reshape(E, -1), blobs)
    with pytest.raises(ValueError):
        q2format.write_blob_file(p, blobs[:, :-16], H, I)


def test_inexact_bf16_scales_are_refused():
    raw = (np.array([1e-7], np.float32).view(np.uint32) >> 16).astype(np.uint16)   # fp16 subnormal range
    with pytest.raises(ValueError):
        q2format._half_from(raw, "BF16")


def _u64(vals):
    import ctypes
    return (ctypes.c_uint64 * max(len(vals), 1))(*vals)


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_reader_threads_read_ranges(tmp_path, threads):
    """c_io_read_ranges: ragged, unaligned, overlapping and empty ranges land where asked, whatever
    the number of reader threads."""
    import os
    from moe_offload import _lib
    L = _lib.lib()
    data = np.random.default_rng(threads).integers(0, 256, 3_000_017, dtype=np.uint8)
    p = tmp_path / "blob.bin"
    data.tofile(p)
    rng = np.random.default_rng(40 + threads)
    offs = [int(v) for v in rng.integers(0, data.size - 70_000, 200)] + [0, data.size - 5, 17]
    lens = [int(v) for v in rng.integers(1, 70_000, 200)] + [5, 5, 0]
    out = np.zeros(sum(lens) + 1, dtype=np.uint8)
    dsts, pos = [], 0
    for n in lens:
        dsts.append(out.ctypes.data + pos)
        pos += n
    L.c_io_init(threads)
    assert L.c_io_threads() == threads
    fd = os.open(p, os.O_RDONLY)
    try:
        assert L.c_io_read_ranges(fd, _u64(offs), _u64(lens), _u64(dsts), len(offs)) == 0, _lib.last_error()
    finally:
        os.close(fd)
    pos = 0
    for o, n in zip(offs, lens):
        assert np.array_equal(out[pos:pos + n], data[o:o + n]), (o, n)
        pos += n
    assert out[-1] == 0


def test_reader_threads_report_short_and_failed_reads(tmp_path):
    import os
    from moe_offload import _lib
    L = _lib.lib()
    p = tmp_path / "small.bin"
    p.write_bytes(bytes(range(256)) * 4)
    buf = np.zeros(4096, dtype=np.uint8)
    L.c_io_init(4)
    fd = os.open(p, os.O_RDONLY)
    try:
        L.c_clear_error()
        assert L.c_io_read_ranges(fd, _u64([1000]), _u64([100]), _u64([buf.ctypes.data]), 1) == -1
        assert "short read" in _lib.last_error()
        assert np.array_equal(buf[:24], np.frombuffer(bytes(range(256)) * 4, np.uint8)[1000:1024])
    finally:
        os.close(fd)
    L.c_clear_error()
    assert L.c_io_read_ranges(fd, _u64([0]), _u64([10]), _u64([buf.ctypes.data]), 1) == -1   # closed fd
    assert "pread" in _lib.last_error()
    L.c_clear_error()
    assert L.c_io_read_ranges(fd, _u64([]), _u64([]), _u64([]), 0) == 0
    L.c_io_init(0)
    assert L.c_io_threads() == 8


@pytest.mark.parametrize("scale_dtype", ["bf16", "f16"])
def test_reference_shard_layout_in_place(tmp_path, scale_dtype):
    """ShardExpertStore lists the shard's 9 tensors by ascending file offset with their roles, and
    reading expert e's row of each (offset + e * bytes per expert, by the reader threads) gives the
    bytes of that expert's slice of the tensor the safetensors library wrote."""
    from helpers import experts_bf16, role_arrays, write_reference_shard
    from moe_offload import _lib
    from moe_offload.loader import ShardExpertStore
    Hs, Is, Es, layer = 512, 192, 12, 9
    mlx = experts_bf16(Es, Hs, Is, seed=4)
    path = write_reference_shard(tmp_path / f"experts-{layer:02d}.safetensors", layer, mlx, scale_dtype)
    want = role_arrays(mlx)
    store = ShardExpertStore(tmp_path, layers=[layer])
    try:
        lay = store.layout[layer]
        assert (store.n_exp, store.hidden, store.inter, store.group) == (Es, Hs, Is, 64)
        assert lay["scale_bf16"] == (scale_dtype == "bf16")
        assert sorted(lay["roles"]) == list(range(9)) and lay["offsets"] == sorted(lay["offsets"])
        assert lay["row_bytes"] == [want[r].shape[1] for r in lay["roles"]]
        assert store.blob_bytes == sum(a.shape[1] for a in want)
        L = _lib.lib()
        L.c_io_init(8)
        eids = [0, 5, 6, 7, 11]
        bufs = [np.zeros((len(eids), want[r].shape[1]), np.uint8) for r in lay["roles"]]
        offs, lens, dsts = [], [], []
        for t, r in enumerate(lay["roles"]):
            for i, e in enumerate(eids):
                offs.append(lay["offsets"][t] + e * lay["row_bytes"][t])
                lens.append(lay["row_bytes"][t])
                dsts.append(bufs[t].ctypes.data + i * lay["row_bytes"][t])
        assert L.c_io_read_ranges(store.fds[layer], _u64(offs), _u64(lens), _u64(dsts), len(offs)) == 0
        for t, r in enumerate(lay["roles"]):
            assert np.array_equal(bufs[t], want[r][eids]), t
    finally:
        store.close()


def test_reference_shard_rejects_malformed(tmp_path):
    from helpers import experts_bf16, write_reference_shard
    from moe_offload.loader import ShardExpertStore
    mlx = experts_bf16(4, 256, 128, seed=5)
    write_reference_shard(tmp_path / "experts-03.safetensors", 3, mlx)
    with pytest.raises(KeyError):
        ShardExpertStore({4: str(tmp_path / "experts-03.safetensors")})     # layer 4's names absent
    pre = "language_model.model.layers.3.mlp.switch_mlp"
    t = {f"{pre}.{p}.{s}": torch.zeros((4, 8, 4), dtype=torch.float32)
         for p in ("gate_proj", "up_proj", "down_proj") for s in ("weight", "scales", "biases")}
    st_torch.save_file(t, str(tmp_path / "bad.safetensors"))
    with pytest.raises(ValueError):
        ShardExpertStore({3: str(tmp_path / "bad.safetensors")})
