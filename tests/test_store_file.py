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
