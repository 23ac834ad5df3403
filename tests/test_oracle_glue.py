"""Pins two oracle/host functions that no golden vector covers.

* `oracle.q2.rmsnorm`, the reference for every GPU RMSNorm (router prologue, stack glue, codebook
  stack): against torch's own `rms_norm` and against closed forms chosen so that a plausible
  mistake fails one of them (eps outside the square root, a missing weight, a sum instead of a
  mean).  A planted mistake must fail.
* `moe_offload.loader.compute_layer_capacities` (mlx-qwen38/loader.py:245-303): hand-computed
  totals and remainder splits for the percentage, byte-budget and proportional paths and the
  16 / num_experts clamps.
"""
import json

import numpy as np
import pytest

from moe_offload.loader import compute_layer_capacities
from oracle import q2

torch = pytest.importorskip("torch")


# ---- RMSNorm -----------------------------------------------------------------------------------


def _eps_outside_sqrt(h, w, eps=1e-6):
    """A plausible wrong restatement: eps added after the square root."""
    h = np.asarray(h, np.float64)
    return h / (np.sqrt(np.mean(h * h, axis=-1, keepdims=True)) + eps) * np.asarray(w, np.float64)


def _no_weight(h, w, eps=1e-6):
    h = np.asarray(h, np.float64)
    return h / np.sqrt(np.mean(h * h, axis=-1, keepdims=True) + eps)


def _sum_not_mean(h, w, eps=1e-6):
    h = np.asarray(h, np.float64)
    return h / np.sqrt(np.sum(h * h, axis=-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def _closed_form_checks(fn):
    """Each returns True when fn passes it."""
    rng = np.random.default_rng(0)
    H = 2048
    w = 1.0 + 0.1 * rng.standard_normal(H)
    out = {}
    # torch's rms_norm (float64, the same eps)
    for scale in (1.0, 1e-3, 40.0):
        h = scale * rng.standard_normal((4, H))
        want = torch.nn.functional.rms_norm(torch.from_numpy(h), (H,), torch.from_numpy(w), eps=1e-6).numpy()
        out.setdefault("torch", True)
        out["torch"] &= bool(np.allclose(fn(h, w), want, rtol=1e-12, atol=0))
    # a constant vector c: rms = sqrt(c^2 + eps), so the output is c / sqrt(c^2 + eps) * w
    c = 3.0
    got = fn(np.full(H, c), w)
    out["constant"] = bool(np.allclose(got, c / np.sqrt(c * c + 1e-6) * w, rtol=1e-14, atol=0))
    # eps-dominated input: |h| ~ 1e-9 so mean(h^2) ~ 1e-18 << eps; output -> h / sqrt(eps) * w = 1000 h w
    h = 1e-9 * rng.standard_normal(H)
    out["eps_dominated"] = bool(np.allclose(fn(h, w), 1000.0 * h * w, rtol=1e-9, atol=0))
    # weight scaling is linear; input scaling cancels when eps is negligible
    h = rng.standard_normal(H)
    out["weight_linear"] = bool(np.allclose(fn(h, 2.5 * w), 2.5 * fn(h, w), rtol=1e-14, atol=0))
    out["scale_invariant"] = bool(np.allclose(fn(1e3 * h, w), fn(1e6 * h, w), rtol=1e-9, atol=0))
    # unit weight, +-1 entries: every output is +-1 / sqrt(1 + eps)
    h = np.where(rng.standard_normal(H) > 0, 1.0, -1.0)
    out["signs"] = bool(np.allclose(fn(h, np.ones(H)), h / np.sqrt(1 + 1e-6), rtol=1e-15, atol=0))
    return out


def test_rmsnorm_matches_torch_and_closed_forms():
    res = _closed_form_checks(q2.rmsnorm)
    assert all(res.values()), res


@pytest.mark.parametrize("wrong", [_eps_outside_sqrt, _no_weight, _sum_not_mean])
def test_rmsnorm_checks_catch_planted_mistakes(wrong):
    res = _closed_form_checks(wrong)
    assert not all(res.values()), f"{wrong.__name__} passed every check: {res}"


def test_rmsnorm_eps_outside_sqrt_fails_eps_closed_form():
    # the specific mistake named for this function must fail the eps-dominated closed form
    assert not _closed_form_checks(_eps_outside_sqrt)["eps_dominated"]


# ---- compute_layer_capacities ------------------------------------------------------------------


def test_capacities_percentage_path():
    # 20% of 512 = 102.4 -> 102 slots on each of layers 1..47 (the workload's 102-slot pools)
    caps = compute_layer_capacities(budget_pct=20)
    assert sorted(caps) == list(range(1, 48)) and set(caps.values()) == {102}
    # a fraction <= 1 is taken as-is: 0.2 -> 102; 1.0 -> every expert
    assert set(compute_layer_capacities(budget_pct=0.2).values()) == {102}
    assert set(compute_layer_capacities(budget_pct=1.0).values()) == {512}
    # 20.1% -> 102.912 -> 103; 30% -> 153.6 -> 154
    assert set(compute_layer_capacities(budget_pct=20.1).values()) == {103}
    assert set(compute_layer_capacities(budget_pct=30).values()) == {154}
    # clamps: 2% -> 10.24 -> 10 -> 16 (floor); 150% -> 768 -> 512 (ceiling)
    assert set(compute_layer_capacities(budget_pct=2).values()) == {16}
    assert set(compute_layer_capacities(budget_pct=150).values()) == {512}


def test_capacities_byte_budget_path():
    # the reference's expert size (loader.py:88-92): 7.5e9 / 1,536,000 = 4882.81 -> 4883 slots;
    # 4883 = 47 * 103 + 42: layers 1..42 take 104, layers 43..47 take 103
    caps = compute_layer_capacities(budget_gb=7.5, expert_bytes=1_536_000)
    assert [caps[l] for l in range(1, 43)] == [104] * 42
    assert [caps[l] for l in range(43, 48)] == [103] * 5
    assert sum(caps.values()) == 4883
    # no budget at all means 7.5 GB
    assert compute_layer_capacities(expert_bytes=1_536_000) == caps
    # the workload's expert size: 7.5e9 / 983,040 = 7629.39 -> 7629 = 47 * 162 + 15
    caps = compute_layer_capacities(budget_gb=7.5, expert_bytes=983_040)
    assert [caps[l] for l in range(1, 16)] == [163] * 15 and [caps[l] for l in range(16, 48)] == [162] * 32
    # clamps on the total: 0.1 GB -> 65 slots -> at least 16 per layer; 1000 GB -> at most 512
    assert set(compute_layer_capacities(budget_gb=0.1, expert_bytes=1_536_000).values()) == {16}
    assert set(compute_layer_capacities(budget_gb=1000, expert_bytes=1_536_000).values()) == {512}


def _summary(tmp_path, weights):
    per_layer = [{"active_experts_decode": 0.0}] + [{"active_experts_decode": float(w)} for w in weights]
    p = tmp_path / "analysis_summary.json"
    p.write_text(json.dumps({"expert_concentration": {"per_layer": per_layer}}))
    return p


def test_capacities_proportional_path(tmp_path):
    kw = dict(budget_pct=50, alloc_mode="proportional", num_layers=5, num_experts=64)
    # total = 4 layers * round(0.5 * 64) = 128.  weights 1:2:3:4 -> raw 12.8, 25.6, 38.4, 51.2;
    # floors clamped to >= 16: 16, 25, 38, 51 (130, two too many); the two smallest fractional
    # parts (51.2, then 38.4) give one back each -> 16, 25, 37, 50
    caps = compute_layer_capacities(analysis_summary=_summary(tmp_path, [1, 2, 3, 4]), **kw)
    assert caps == {1: 16, 2: 25, 3: 37, 4: 50}
    # weights 3:3:2:2 -> raw 38.4, 38.4, 25.6, 25.6; floors sum to 126, the two largest
    # fractional parts (the 25.6s) take the two missing slots
    caps = compute_layer_capacities(analysis_summary=_summary(tmp_path, [3, 3, 2, 2]), **kw)
    assert caps == {1: 38, 2: 38, 3: 26, 4: 26}
    # weights 10:1:1:1 -> raw 98.5, 9.8, 9.8, 9.8 -> clamped 64, 16, 16, 16 (16 short); one pass
    # in fractional order adds one to each of the three layers below the ceiling and stops:
    # the total stays 13 short, as in the reference
    caps = compute_layer_capacities(analysis_summary=_summary(tmp_path, [10, 1, 1, 1]), **kw)
    assert caps == {1: 64, 2: 17, 3: 17, 4: 17}
    # a missing summary falls back to the even split
    caps = compute_layer_capacities(analysis_summary=tmp_path / "absent.json", **kw)
    assert caps == {1: 32, 2: 32, 3: 32, 4: 32}


def test_offload_engine_model_path_is_never_ignored(tmp_path):
    """OffloadEngine(model_path=...) binds that directory or raises: it never falls back to the
    synthetic model (no GPU needed: the directory is checked before any device work)."""
    import pytest
    from moe_offload.loader import OffloadEngine
    with pytest.raises(FileNotFoundError):
        OffloadEngine(model_path=tmp_path / "missing")
    (tmp_path / "empty").mkdir()
    with pytest.raises(FileNotFoundError):
        OffloadEngine(model_path=tmp_path / "empty")


def test_model_directory_routers_are_read_and_checked(tmp_path):
    """ckpt.load_routers reads each layer's 8-bit router from base-*.safetensors with the shapes
    the reference's loader checks (loader.cpp:398-404, 450) and rejects a wrong shape."""
    import numpy as np
    import pytest
    import torch
    from safetensors.torch import save_file

    from helpers import router_q8
    from moe_offload import ckpt
    rng = np.random.default_rng(1)
    E, Hd = 16, 256
    base = {}
    want = {}
    for l in range(3):
        c, s, b = router_q8(E, Hd, rng)
        want[l] = (c, s, b)
        pre = f"language_model.model.layers.{l}.mlp.gate"
        base[f"{pre}.weight"] = torch.from_numpy(c.view(np.int32)).view(torch.uint32)
        base[f"{pre}.scales"] = torch.from_numpy(s.view(np.int16)).view(torch.bfloat16)
        base[f"{pre}.biases"] = torch.from_numpy(b.view(np.int16)).view(torch.bfloat16)
    save_file(base, str(tmp_path / "base-00.safetensors"))
    got = ckpt.load_routers(tmp_path, 3, E, Hd)
    for l in range(3):
        assert np.array_equal(got[l][0].view(np.uint32), want[l][0])
        assert np.array_equal(got[l][1].view(np.uint16), want[l][1])
        assert np.array_equal(got[l][2].view(np.uint16), want[l][2])
    with pytest.raises(ValueError):
        ckpt.load_routers(tmp_path, 3, E, 2 * Hd)     # experts of another hidden size
    with pytest.raises(KeyError):
        ckpt.load_routers(tmp_path, 4, E, Hd)         # a layer without a router
