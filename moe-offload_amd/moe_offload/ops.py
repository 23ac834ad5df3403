"""torch-facing wrappers of the HIP compute entry points (tensors in, tensors out).

Every function calls straight into libmoe_offload.so on torch's current HIP stream; there is
no PyTorch fallback for any of them.
"""
from __future__ import annotations

import torch

from . import _lib

_ROUTER_WS: dict[tuple[int, int], torch.Tensor] = {}


def _stream(stream=None) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _p(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def router_workspace(n_exp: int, device=None) -> torch.Tensor:
    """Zeroed scratch for one router launch site (logits + the block-done counter)."""
    dev = torch.device(device or "cuda")
    key = (dev.index if dev.index is not None else torch.cuda.current_device(), n_exp)
    ws = _ROUTER_WS.get(key)
    if ws is None:
        nb = _lib.lib().moe_router_workspace_bytes(n_exp)
        ws = torch.zeros(int(nb), dtype=torch.uint8, device=dev)
        _ROUTER_WS[key] = ws
    return ws


def router(w: torch.Tensor, k: int, *, x: torch.Tensor | None = None, h: torch.Tensor | None = None,
           norm_w: torch.Tensor | None = None, eps: float = 1e-6, w_next: torch.Tensor | None = None,
           m: int = 12, x_out: torch.Tensor | None = None, ids: torch.Tensor | None = None,
           scores: torch.Tensor | None = None, pred: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None):
    """Fused router for one token.

    x: fp16 [hidden] input, or h: fp32 [hidden] residual to RMSNorm first (written to x_out).
    w: fp16 [n_exp, hidden].  Returns (ids int32 [k] ascending-gate order, scores fp16 [k],
    pred int32 [m] (next-layer prediction, descending) or None).
    """
    n_exp, hidden = w.shape
    assert w.dtype == torch.float16 and w.is_contiguous()
    assert (x is None) != (h is None)
    if x is not None:
        assert x.dtype == torch.float16 and x.numel() == hidden and x.is_contiguous()
    if h is not None:
        assert h.dtype == torch.float32 and h.numel() == hidden and h.is_contiguous()
    if w_next is not None:
        assert w_next.shape == w.shape and w_next.dtype == torch.float16 and w_next.is_contiguous()
    dev = w.device
    ids = ids if ids is not None else torch.empty(k, dtype=torch.int32, device=dev)
    scores = scores if scores is not None else torch.empty(k, dtype=torch.float16, device=dev)
    if w_next is not None and pred is None:
        pred = torch.empty(m, dtype=torch.int32, device=dev)
    ws = workspace if workspace is not None else router_workspace(n_exp, dev)
    rc = _lib.lib().moe_router(_p(h), _p(norm_w), eps, _p(x), _p(x_out), _p(w), _p(w_next), hidden, n_exp, k,
                               m if w_next is not None else 0, _p(ws), _p(ids), _p(scores), _p(pred), _stream())
    _lib.check(rc, "moe_router")
    return ids, scores, (pred if w_next is not None else None)


def rmsnorm(h: torch.Tensor, norm_w: torch.Tensor | None, eps: float = 1e-6, out: torch.Tensor | None = None):
    """fp16 RMSNorm of an fp32 vector (fp64 math, one rounding)."""
    assert h.dtype == torch.float32 and h.is_contiguous()
    out = out if out is not None else torch.empty(h.numel(), dtype=torch.float16, device=h.device)
    rc = _lib.lib().moe_rmsnorm(_p(h), _p(norm_w), eps, h.numel(), _p(out), _stream())
    _lib.check(rc, "moe_rmsnorm")
    return out


def q2_switch_glu(x: torch.Tensor, pool: torch.Tensor, slots: torch.Tensor, hidden: int, inter: int,
                  group: int = 64, scores: torch.Tensor | None = None, residual: torch.Tensor | None = None,
                  per_expert: bool = False, h_ws: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """SwitchGLU over the Q2 blobs pool[slots[j]] for one token.

    Returns fp32 [hidden] = residual + sum_j scores[j] * expert_j(x), or fp32 [k, hidden] of
    per-expert outputs when per_expert.
    """
    k = slots.numel()
    assert x.dtype == torch.float16 and x.numel() == hidden and x.is_contiguous()
    assert pool.dtype == torch.uint8 and pool.dim() == 2 and pool.is_contiguous()
    assert slots.dtype == torch.int32 and slots.is_contiguous()
    dev = x.device
    if h_ws is None:
        h_ws = torch.empty(k * inter, dtype=torch.float16, device=dev)
    if out is None:
        out = torch.empty((k, hidden) if per_expert else (hidden,), dtype=torch.float32, device=dev)
    rc = _lib.lib().moe_q2_switch_glu(_p(x), _p(pool), pool.shape[1], pool.shape[0], _p(slots), _p(scores), k,
                                      hidden, inter,
                                      group, _p(residual), _p(h_ws), _p(out), int(per_expert), _stream())
    _lib.check(rc, "moe_q2_switch_glu")
    return out


def q2_gate_up(x, pool, slots, hidden, inter, group=64, h_out=None):
    k = slots.numel()
    h_out = h_out if h_out is not None else torch.empty(k * inter, dtype=torch.float16, device=x.device)
    rc = _lib.lib().moe_q2_gate_up(_p(x), _p(pool), pool.shape[1], pool.shape[0], _p(slots), k, hidden, inter,
                                   group, _p(h_out), _stream())
    _lib.check(rc, "moe_q2_gate_up")
    return h_out


def q2_down(h, pool, slots, hidden, inter, group=64, scores=None, residual=None, per_expert=False, out=None):
    k = slots.numel()
    if out is None:
        out = torch.empty((k, hidden) if per_expert else (hidden,), dtype=torch.float32, device=h.device)
    rc = _lib.lib().moe_q2_down(_p(h), _p(pool), pool.shape[1], pool.shape[0], _p(slots), _p(scores), k, hidden,
                                inter, group,
                                _p(residual), _p(out), int(per_expert), _stream())
    _lib.check(rc, "moe_q2_down")
    return out


def q2_grouped_gate_up(x, row_token, seg_start, pool, hidden, inter, group=64, seg_slot=None, h_out=None):
    """h[r] = silu(G x[row_token[r]]) * (U x[row_token[r]]) for rows sorted by expert.

    x: fp16 [n_tok, hidden]; row_token int32 [M]; seg_start int32 [n_seg + 1] (segment u = rows
    seg_start[u]:seg_start[u+1], weights pool[seg_slot[u]], or pool[u] when seg_slot is None).
    Returns fp16 [M, inter].
    """
    n_tok, M, n_seg = x.shape[0], row_token.numel(), seg_start.numel() - 1
    h_out = h_out if h_out is not None else torch.empty((M, inter), dtype=torch.float16, device=x.device)
    rc = _lib.lib().moe_q2_grouped_gate_up(_p(x), n_tok, _p(row_token), M, _p(seg_start), _p(seg_slot), n_seg,
                                           _p(pool), pool.shape[1], pool.shape[0], hidden, inter, group, _p(h_out),
                                           _stream())
    _lib.check(rc, "moe_q2_grouped_gate_up")
    return h_out


def q2_grouped_down(h, seg_start, pool, hidden, inter, group=64, row_out=None, n_out_rows=None, seg_slot=None,
                    out=None):
    """y[row_out[r]] = D h[r] (fp16) for rows sorted by expert; row_out None writes row r."""
    M, n_seg = h.shape[0], seg_start.numel() - 1
    n_out = n_out_rows if n_out_rows is not None else M
    out = out if out is not None else torch.empty((n_out, hidden), dtype=torch.float16, device=h.device)
    rc = _lib.lib().moe_q2_grouped_down(_p(h), M, _p(row_out), n_out, _p(seg_start), _p(seg_slot), n_seg, _p(pool),
                                        pool.shape[1], pool.shape[0], hidden, inter, group, _p(out), _stream())
    _lib.check(rc, "moe_q2_grouped_down")
    return out


def q2_grouped_switch_glu(x, row_token, seg_start, pool, hidden, inter, group=64, row_out=None, n_out_rows=None,
                          seg_slot=None, h_ws=None, out=None):
    """Both grouped projections: fp16 [n_out_rows, hidden] per-(token, k) SwitchGLU outputs."""
    n_tok, M, n_seg = x.shape[0], row_token.numel(), seg_start.numel() - 1
    n_out = n_out_rows if n_out_rows is not None else M
    h_ws = h_ws if h_ws is not None else torch.empty((M, inter), dtype=torch.float16, device=x.device)
    out = out if out is not None else torch.empty((n_out, hidden), dtype=torch.float16, device=x.device)
    rc = _lib.lib().moe_q2_grouped_switch_glu(_p(x), n_tok, _p(row_token), _p(row_out), M, n_out, _p(seg_start),
                                              _p(seg_slot), n_seg, _p(pool), pool.shape[1], pool.shape[0], hidden,
                                              inter, group, _p(h_ws), _p(out), _stream())
    _lib.check(rc, "moe_q2_grouped_switch_glu")
    return out


def pair_combine(y, scores, residual=None, out=None):
    """out fp32 [n_tok, hidden] = residual + sum_j scores[t, j] * y[t*k + j]."""
    n_tok, k = scores.shape
    hidden = y.shape[-1]
    out = out if out is not None else torch.empty((n_tok, hidden), dtype=torch.float32, device=y.device)
    rc = _lib.lib().moe_pair_combine(_p(y), _p(scores), _p(residual), n_tok, k, hidden, _p(out), _stream())
    _lib.check(rc, "moe_pair_combine")
    return out


# ---- 2-bit codebook experts (non-gated: up -> squared ReLU -> down) ---------------------------

def cb_moe(x: torch.Tensor, pool: torch.Tensor, slots: torch.Tensor, grid: torch.Tensor, hidden: int, inter: int,
           scores: torch.Tensor | None = None, residual: torch.Tensor | None = None, per_expert: bool = False,
           h_ws: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """Codebook experts pool[slots[j]] (format of moe_offload.cbformat) for one token.

    Returns fp32 [hidden] = residual + sum_j scores[j] * down_j(relu(up_j x)^2), or fp32
    [k, hidden] per-expert outputs when per_expert.  grid: device uint8 [256, 8]."""
    k = slots.numel()
    assert x.dtype == torch.float16 and x.numel() == hidden and x.is_contiguous()
    assert pool.dtype == torch.uint8 and pool.dim() == 2 and pool.is_contiguous()
    assert slots.dtype == torch.int32 and slots.is_contiguous()
    assert grid.dtype == torch.uint8 and grid.numel() == 256 * 8 and grid.is_cuda
    dev = x.device
    if h_ws is None:
        h_ws = torch.empty(k * inter, dtype=torch.bfloat16, device=dev)
    if out is None:
        out = torch.empty((k, hidden) if per_expert else (hidden,), dtype=torch.float32, device=dev)
    rc = _lib.lib().moe_cb_moe(_p(x), _p(pool), pool.shape[1], pool.shape[0], _p(slots), _p(scores), k, hidden, inter,
                               _p(grid), _p(residual), _p(h_ws), _p(out), int(per_expert), _stream())
    _lib.check(rc, "moe_cb_moe")
    return out


def cb_up(x, pool, slots, grid, hidden, inter, h_out=None):
    """bf16 [k, inter] = relu(up_j x)^2."""
    k = slots.numel()
    h_out = h_out if h_out is not None else torch.empty((k, inter), dtype=torch.bfloat16, device=x.device)
    rc = _lib.lib().moe_cb_up(_p(x), _p(pool), pool.shape[1], pool.shape[0], _p(slots), k, hidden, inter, _p(grid),
                              _p(h_out), _stream())
    _lib.check(rc, "moe_cb_up")
    return h_out
