"""The codebook format (moe_offload.cbformat) and its oracle (oracle/codebook.py) on the CPU.

The reference runs this path only inside llama.cpp (not vendored), so nothing here is a golden
vector of the reference: parity of this path is unpinned.  The oracle is pinned instead by hand
computed known answers, a loop form written straight from the format description, the format's
invariants and planted mistakes that those checks must catch."""
import numpy as np
import pytest

from moe_offload import cbformat
from oracle import codebook as cb

GRID = cbformat.grid()


def one_block(idx0, sign0, sub0, d0, grid=GRID):
    """A [1, 256] matrix whose first group has the given codes; the other groups have
    magnitudes grid[0], no signs, sub-scale 0."""
    idx = np.zeros((1, 32), np.int64)
    sign7 = np.zeros((1, 32), np.int64)
    sub = np.zeros((1, 8), np.int64)
    idx[0, 0], sign7[0, 0], sub[0, 0] = idx0, sign0, sub0
    d = np.array([[d0]], np.float16)
    return idx, sign7, sub, d


def test_grid_is_seeded_and_in_range():
    g = cbformat.grid()
    assert g.shape == (256, 8) and g.dtype == np.uint8
    assert set(np.unique(g)) == {1, 3, 5}
    assert np.array_equal(g, cbformat.grid(cbformat.GRID_SEED))
    assert not np.array_equal(g, cbformat.grid(cbformat.GRID_SEED + 1))


def test_known_answers():
    """Hand-computed weights of one group: d = 0.5, sub-scale 3 -> db = 0.5 * 7 / 8 = 0.4375."""
    grid = GRID.copy()
    grid[17] = [1, 3, 5, 1, 3, 5, 1, 3]
    db = 0.4375
    # sign7 = 0b0000101: two negatives, parity 0 -> weights 0 and 2 negative
    w = cb.dequantize(one_block(17, 0b0000101, 3, 0.5, grid), grid)[0, :8]
    assert w.tolist() == [db * v for v in (-1, 3, -5, 1, 3, 5, 1, 3)]
    # sign7 = 0b0000001: one negative, parity 1 -> the 8th weight is negative too
    w = cb.dequantize(one_block(17, 0b0000001, 3, 0.5, grid), grid)[0, :8]
    assert w.tolist() == [db * v for v in (-1, 3, 5, 1, 3, 5, 1, -3)]
    # sign7 = 0b0000011: weights 0 and 1 negative (an asymmetric pattern: bit order matters)
    w = cb.dequantize(one_block(17, 0b0000011, 3, 0.5, grid), grid)[0, :8]
    assert w.tolist() == [db * v for v in (-1, -3, 5, 1, 3, 5, 1, 3)]
    # sub-scale 0 and 15: db = d / 8 and d * 31 / 8
    assert cb.dequantize(one_block(17, 0, 0, 2.0, grid), grid)[0, 0] == 0.25
    assert cb.dequantize(one_block(17, 0, 15, 2.0, grid), grid)[0, 0] == 7.75


def planted(codes, grid, mistake):
    """The dequantiser with one plausible mistake (a control, not a product path)."""
    idx, sign7, sub, d = codes
    rows, ng = idx.shape
    mag = grid[np.asarray(idx, np.int64)].astype(np.float64)
    s8 = np.asarray(sign7, np.int64) & 0x7F if mistake == "no_parity" else cb.signs8(sign7)
    bits = (s8[..., None] >> np.arange(8)) & 1
    if mistake == "msb_first":
        bits = bits[..., ::-1]
    w = (mag * (1 - 2 * bits)).reshape(rows, ng * 8)
    d32 = np.repeat(np.asarray(d, np.float16).astype(np.float64), 8, axis=1)
    db = d32 * ((np.asarray(sub) + 1) if mistake == "scale" else (2 * np.asarray(sub) + 1)) / 8
    return w * np.repeat(db, 32, axis=1)


@pytest.mark.parametrize("mistake", ["no_parity", "scale", "msb_first"])
def test_planted_mistakes_fail_the_known_answers(mistake):
    grid = GRID.copy()
    grid[17] = [1, 3, 5, 1, 3, 5, 1, 3]
    for sign7 in (0b0000001, 0b0000011):
        codes = one_block(17, sign7, 3, 0.5, grid)
        assert np.array_equal(planted(codes, grid, None), cb.dequantize(codes, grid))   # faithful control
    failed = [not np.array_equal(planted(c, grid, mistake), cb.dequantize(c, grid))
              for c in (one_block(17, 0b0000001, 3, 0.5, grid), one_block(17, 0b0000011, 3, 0.5, grid))]
    assert any(failed)


def test_vectorised_matches_loop_form():
    rng = np.random.default_rng(3)
    for rows, k in [(3, 256), (5, 512), (2, 1024)]:
        codes = cbformat.random_codes(rows, k, rng, d_scale=0.1)
        x = rng.standard_normal(k)
        np.testing.assert_allclose(cb.dequantize(codes, GRID) @ x, cb.brute_matvec(codes, GRID, x), rtol=1e-12,
                                   atol=1e-12)


def test_format_invariants():
    rng = np.random.default_rng(4)
    codes = cbformat.random_codes(64, 512, rng, d_scale=0.1)
    w = cb.int_weights(codes[0], codes[1], GRID)
    neg = (w < 0).reshape(64, -1, 8).sum(-1)
    assert (neg % 2 == 0).all()                                  # parity: even negatives per group
    assert set(np.unique(np.abs(w))) <= {1, 3, 5}
    full = cb.dequantize(codes, GRID)
    db = np.repeat(cb.sub_scales(codes[2], codes[3]), 32, axis=1)
    assert np.array_equal(full, w * db)


@pytest.mark.parametrize("hidden,inter", [(3072, 1536), (512, 256)])
def test_blob_pack_unpack_round_trip(hidden, inter):
    rng = np.random.default_rng(5)
    up = cbformat.random_codes(inter, hidden, rng)
    down = cbformat.random_codes(hidden, inter, rng)
    blob = cbformat.to_blob(up, down, hidden, inter)
    assert blob.size == cbformat.expert_bytes(hidden, inter)
    u2, d2 = cbformat.from_blob(blob, hidden, inter)
    for a, b in zip(up, u2):
        assert np.array_equal(np.asarray(a), np.asarray(b))
    for a, b in zip(down, d2):
        assert np.array_equal(np.asarray(a), np.asarray(b))


def test_expert_bytes_at_the_workload_shape():
    # 256 weights -> 64 code bytes + 2 scale bytes (66 B, 2.0625 bits per weight)
    assert cbformat.expert_bytes(3072, 1536) == 2 * 3072 * 1536 // 256 * 66 == 2_433_024


def test_bf16_rounding_closed_forms():
    v = np.array([1.0, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -9, 1.0 + 2 ** -9, 3.0 * 2 ** 20], np.float32)
    r = cb.round_bf16(v)
    # bf16 keeps 7 fraction bits: the step at 1 is 2^-7, so 1 + 2^-8 is a tie
    assert r[0] == 1.0
    assert r[1] == 1.0                        # tie -> even (1.0)
    assert r[2] == 1.0 + 2 ** -7              # above the tie -> up
    assert r[3] == 1.0                        # below the tie -> down
    assert r[4] == 3.0 * 2 ** 20


def test_expert_forward_closed_form():
    """The expert equals down . relu(up . x)^2 over the dequantised matrices, is quadratic in
    the up scales and linear in the down scales."""
    rng = np.random.default_rng(6)
    hidden, inter = 256, 256
    up = cbformat.random_codes(inter, hidden, rng, d_scale=0.05)
    down = cbformat.random_codes(hidden, inter, rng, d_scale=0.05)
    x = rng.standard_normal(hidden)
    U, D = cb.dequantize(up, GRID), cb.dequantize(down, GRID)
    want = D @ np.maximum(U @ x, 0) ** 2
    np.testing.assert_allclose(cb.expert(x, up, down, GRID), want, rtol=1e-12)
    # linear in the down scale, quadratic in the up scale
    up2 = (up[0], up[1], up[2], (up[3].astype(np.float32) * 2).astype(np.float16))
    np.testing.assert_allclose(cb.expert(x, up2, down, GRID), 4 * want, rtol=1e-12)
