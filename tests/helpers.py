"""Shared helpers for the GPU parity tests (inputs are seeded; results are compared with the oracle)."""
from __future__ import annotations

import numpy as np

from moe_offload import q2format, synth
from oracle import q2

H, E, K, I, G = 2048, 512, 10, 512, 64


def experts_np(n_exp=E, hidden=H, inter=I, seed=1, scale_std=0.02):
    """MLX-layout experts and their blobs."""
    gate, up, down = synth.q2_experts(n_exp, hidden, inter, seed=seed, scale_std=scale_std)
    blobs = q2format.to_blobs(gate, up, down, hidden, inter)
    return (gate, up, down), blobs


def expert_fn(mlx):
    gate, up, down = mlx
    return lambda e: ((gate[0][e], gate[1][e], gate[2][e]), (up[0][e], up[1][e], up[2][e]),
                      (down[0][e], down[1][e], down[2][e]))


def oracle_moe(x16, inds, scores16, mlx, residual=None):
    """fp64 oracle of sum_j s_j SwitchGLU_{e_j}(x) (+ residual)."""
    y = q2.moe_combine(x16.astype(np.float64), inds, scores16.astype(np.float64), expert_fn(mlx),
                       bits=2, group=64)
    if residual is not None:
        y = y + residual.astype(np.float64)
    return y


def assert_close_rms(got, want, tol=1e-2, what=""):
    """max|err| <= tol * RMS(want) -- the decode output bar."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    rms = np.sqrt(np.mean(want ** 2))
    err = np.abs(got - want).max()
    assert err <= tol * rms, f"{what}: max|err| {err:.3e} > {tol} x RMS {rms:.3e}"
    return err / rms


def experts_bf16(n_exp, hidden, inter, seed=1, scale_std=0.02):
    """MLX-layout experts with bf16 scales and biases, as the reference's checkpoints hold them:
    per projection (w uint32 [E, out, in/16], scales / biases bf16 bits uint16 [E, out, in/64])."""
    rng = np.random.default_rng(seed)

    def proj(out_f, in_f):
        w = rng.integers(0, 2**32, size=(n_exp, out_f, in_f // 16), dtype=np.uint32)
        s = q2.f32_to_bf16_bits((rng.standard_normal((n_exp, out_f, in_f // 64)) * scale_std).astype(np.float32))
        b = q2.f32_to_bf16_bits(-1.5 * q2.bf16_bits_to_f32(s))
        return w, s, b

    return proj(inter, hidden), proj(inter, hidden), proj(hidden, inter)


ROLE_NAMES = [(p, s) for p in ("gate_proj", "up_proj", "down_proj") for s in ("weight", "scales", "biases")]


def role_arrays(mlx):
    """The 9 tensors of MLX-layout experts in role order, each as uint8 [E, bytes per expert]."""
    out = []
    for w, s, b in mlx:
        n = w.shape[0]
        out += [np.ascontiguousarray(a).view(np.uint8).reshape(n, -1) for a in (w, s, b)]
    return out


def write_reference_shard(path, layer, mlx, scale_dtype="bf16"):
    """An experts-XX.safetensors shard in the reference checkpoint's form (U32 codes; BF16 or F16
    scales and biases, given as their 16-bit patterns), written by the safetensors library."""
    import torch
    from safetensors.torch import save_file
    half = torch.bfloat16 if scale_dtype == "bf16" else torch.float16
    pre = f"language_model.model.layers.{layer}.mlp.switch_mlp"
    tensors = {}
    for (proj, suffix), a in zip(ROLE_NAMES, [t for p in mlx for t in p]):
        a = np.ascontiguousarray(a)
        if suffix == "weight":
            tensors[f"{pre}.{proj}.{suffix}"] = torch.from_numpy(a.view(np.int32)).view(torch.uint32)
        else:
            tensors[f"{pre}.{proj}.{suffix}"] = torch.from_numpy(a.view(np.int16)).view(half)
    save_file(tensors, str(path))
    return path


def router_q8(n_exp, hidden, rng, equal_rows=False):
    """An 8-bit affine group-64 router as the checkpoint stores it: codes uint32 [E, H/4], bf16 bits
    uint16 scales / biases [E, H/64] (scales ~2e-4, biases ~ -128 x scale: logits of order one)."""
    rows = 1 if equal_rows else n_exp
    codes = rng.integers(0, 2**32, size=(rows, hidden // 4), dtype=np.uint32)
    scales = q2.f32_to_bf16_bits((rng.standard_normal((rows, hidden // 64)) * 2e-4).astype(np.float32))
    biases = q2.f32_to_bf16_bits((-128 * q2.to_f64(scales, "bf16")
                                  + rng.standard_normal((rows, hidden // 64)) * 1e-4).astype(np.float32))
    if equal_rows:
        codes, scales, biases = (np.repeat(a, n_exp, axis=0) for a in (codes, scales, biases))
    return codes, scales, biases


def write_model_dir(root, n_layers, n_exp, hidden, inter, seed=1):
    """A model directory in the reference's layout: experts-{l:02d}.safetensors per layer (the 9
    switch_mlp tensors, bf16 scales) and base-00.safetensors with every layer's 8-bit router
    `language_model.model.layers.{l}.mlp.gate.{weight,scales,biases}`.  Returns
    ({layer: MLX-layout experts}, {layer: (codes, scales, biases)})."""
    import torch
    from safetensors.torch import save_file
    from pathlib import Path
    root = Path(root)
    root.mkdir(parents=True, exist_ok=True)
    rng = np.random.default_rng(seed)
    experts, routers, base = {}, {}, {}
    for l in range(n_layers):
        experts[l] = experts_bf16(n_exp, hidden, inter, seed=seed * 100 + l)
        write_reference_shard(root / f"experts-{l:02d}.safetensors", l, experts[l])
        routers[l] = router_q8(n_exp, hidden, rng)
        c, s, b = routers[l]
        pre = f"language_model.model.layers.{l}.mlp.gate"
        base[f"{pre}.weight"] = torch.from_numpy(c.view(np.int32)).view(torch.uint32)
        base[f"{pre}.scales"] = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
        base[f"{pre}.biases"] = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    save_file(base, str(root / "base-00.safetensors"))
    return experts, routers
