"""Merge statistics and the two-phase schedule on MI355X.

The paper's Algorithm 1 splits a layer's sources into an inter-block group
(shared by every layer of the block, so evaluated for all of them in one
batched pass) and an intra-block group, and merges the two partial results
with an online softmax. That needs each phase to return its unnormalised
output together with the running max and sum of exponentials
(reference src/switchyard/reference.py:194-233, ``attn_with_stats`` and
``merge_online_softmax``). The reference has these only as a float64 oracle
and its batched API returns no statistics; here they are HIP operators:

* ``attn_with_stats(v, w)`` -> ``(o, m, l)``, with autograd through all three;
* ``merge_online_softmax(o1, m1, l1, o2, m2, l2)`` -> ``(o, m, l)``, with autograd;
* ``block_attn_res_batched_with_stats(v, queries)`` -> ``(o, m, l)`` per query,
  one read of ``v`` for all queries (output only);
* ``attn_with_stats_merge(v, w, o1, m1, l1)`` -> ``(out, m, l)``: phase 2 of
  the schedule in one pass, this group's sources merged with a prior group's
  triple before anything is written (normalised by default), with autograd;
* ``block_attn_res_two_phase(v, w, split)`` composes them; it equals the
  single-pass operator up to rounding.

Per token, with ``p_n = exp(logit_n - m)``: ``m = max_n logit_n``,
``l = sum_n p_n``, ``o = sum_n p_n v_n``; ``o`` has ``v``'s dtype, ``m`` and
``l`` are fp32 ``[B, T]``.
"""

from __future__ import annotations

import torch

from . import _lib
from .hip_op import _ptr, _validate, _validate_batched
from .reference import DEFAULT_EPS

__all__ = [
    "attn_with_stats",
    "merge_online_softmax",
    "attn_with_stats_merge",
    "block_attn_res_batched_with_stats",
    "block_attn_res_two_phase",
]


class _AttnWithStats(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v: torch.Tensor, w: torch.Tensor, eps: float):
        n, b, t, d = _validate(v, w)
        v = v.contiguous()
        w = w.contiguous()
        n_tok = b * t
        o = torch.empty(b, t, d, device=v.device, dtype=v.dtype)
        m = torch.empty(b, t, device=v.device, dtype=torch.float32)
        ell = torch.empty(b, t, device=v.device, dtype=torch.float32)
        want_grad = bool(ctx.needs_input_grad[0] or ctx.needs_input_grad[1])
        stats = (
            torch.empty(2, n, n_tok, device=v.device, dtype=torch.float32)
            if want_grad and n_tok > 0 and d > 0
            else None
        )
        if n_tok > 0 and d > 0:
            with torch.cuda.device(v.device):
                rc = _lib.lib().sy_attn_with_stats(
                    _ptr(v), _ptr(w), _ptr(o), _ptr(m), _ptr(ell), _ptr(stats), n, n_tok, d,
                    n_tok * d, _lib.dtype_code(v.dtype), _lib.dtype_code(w.dtype), float(eps),
                    _lib.stream_ptr(v.device),
                )
            _lib.check(rc, "sy_attn_with_stats")
        ctx.save_for_backward(v, w, stats)
        ctx.eps = float(eps)
        return o, m, ell

    @staticmethod
    def backward(ctx, go, gm, gl):
        v, w, stats = ctx.saved_tensors
        n, b, t, d = v.shape
        n_tok = b * t
        go = torch.zeros(b, t, d, device=v.device, dtype=v.dtype) if go is None else go.to(v.dtype).contiguous()
        zeros = torch.zeros(b, t, device=v.device, dtype=torch.float32)
        gm = zeros if gm is None else gm.float().contiguous()
        gl = zeros if gl is None else gl.float().contiguous()
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
        dw = torch.empty(d, device=v.device, dtype=w.dtype)
        if d == 0:
            return dv, dw, None
        lib = _lib.lib()
        vt, wt = _lib.dtype_code(v.dtype), _lib.dtype_code(w.dtype)
        with torch.cuda.device(v.device):
            ws_bytes = lib.sy_bwd_workspace_bytes(n, n_tok, d, vt, wt)
            if ws_bytes < 0:
                _lib.check(int(ws_bytes), "sy_bwd_workspace_bytes")
            ws = torch.empty(max(1, (ws_bytes + 3) // 4), device=v.device, dtype=torch.float32)
            rc = lib.sy_attn_with_stats_bwd(
                _ptr(v), _ptr(w), _ptr(go), _ptr(gm), _ptr(gl), _ptr(stats), _ptr(dv), _ptr(dw),
                _ptr(ws), ws.numel() * 4, n, n_tok, d, n_tok * d, vt, wt, ctx.eps,
                _lib.stream_ptr(v.device),
            )
        _lib.check(rc, "sy_attn_with_stats_bwd")
        return dv, dw, None


def attn_with_stats(v: torch.Tensor, w: torch.Tensor, eps: float = DEFAULT_EPS):
    """``(o, m, l)`` of one source group (reference.py:194-215), with autograd.

    ``o / l[..., None]`` equals ``block_attn_res_triton(v, w)``; two groups
    combine exactly with :func:`merge_online_softmax`.
    """
    return _AttnWithStats.apply(v, w, eps)


def _validate_triple(o: torch.Tensor, m: torch.Tensor, ell: torch.Tensor, name: str) -> None:
    if o.ndim != 3:
        raise ValueError(f"{name}: o must be [B, T, D], got {tuple(o.shape)}")
    if m.shape != o.shape[:2] or ell.shape != o.shape[:2]:
        raise ValueError(f"{name}: m and l must be [B, T] = {tuple(o.shape[:2])}")
    if m.dtype != torch.float32 or ell.dtype != torch.float32:
        raise ValueError(f"{name}: m and l must be float32")
    if not (o.is_cuda and m.is_cuda and ell.is_cuda):
        raise ValueError(f"{name}: tensors must be on a CUDA device")
    _lib.dtype_code(o.dtype)


class _MergeStats(torch.autograd.Function):
    @staticmethod
    def forward(ctx, o1, m1, l1, o2, m2, l2):
        _validate_triple(o1, m1, l1, "group 1")
        _validate_triple(o2, m2, l2, "group 2")
        if o1.shape != o2.shape or o1.dtype != o2.dtype or o1.device != o2.device:
            raise ValueError("both groups must have the same shape, dtype and device")
        o1, m1, l1, o2, m2, l2 = (x.contiguous() for x in (o1, m1, l1, o2, m2, l2))
        b, t, d = o1.shape
        o = torch.empty_like(o1)
        m = torch.empty_like(m1)
        ell = torch.empty_like(l1)
        if b * t and d:
            with torch.cuda.device(o1.device):
                rc = _lib.lib().sy_merge_stats(
                    _ptr(o1), _ptr(m1), _ptr(l1), _ptr(o2), _ptr(m2), _ptr(l2), _ptr(o), _ptr(m),
                    _ptr(ell), b * t, d, _lib.dtype_code(o1.dtype), _lib.stream_ptr(o1.device),
                )
            _lib.check(rc, "sy_merge_stats")
        ctx.save_for_backward(o1, m1, l1, o2, m2, l2)
        return o, m, ell

    @staticmethod
    def backward(ctx, go, gm, gl):
        o1, m1, l1, o2, m2, l2 = ctx.saved_tensors
        b, t, d = o1.shape
        go = torch.zeros_like(o1) if go is None else go.to(o1.dtype).contiguous()
        gm = torch.zeros_like(m1) if gm is None else gm.float().contiguous()
        gl = torch.zeros_like(l1) if gl is None else gl.float().contiguous()
        outs = [torch.empty_like(x) for x in (o1, m1, l1, o2, m2, l2)]
        if b * t and d:
            with torch.cuda.device(o1.device):
                rc = _lib.lib().sy_merge_stats_bwd(
                    _ptr(o1), _ptr(m1), _ptr(l1), _ptr(o2), _ptr(m2), _ptr(l2), _ptr(go), _ptr(gm),
                    _ptr(gl), *[_ptr(x) for x in outs], b * t, d, _lib.dtype_code(o1.dtype),
                    _lib.stream_ptr(o1.device),
                )
            _lib.check(rc, "sy_merge_stats_bwd")
        return tuple(outs)


def merge_online_softmax(o1, m1, l1, o2, m2, l2):
    """The ``(o, m, l)`` of the union of two disjoint source groups
    (reference.py:218-233), with autograd. The max goes to group 1 on a tie."""
    return _MergeStats.apply(o1, m1, l1, o2, m2, l2)


class _AttnWithStatsMerge(torch.autograd.Function):
    """Forward: one launch of ``sy_attn_with_stats_merge``. Backward: the
    gradient of the same function, evaluated through the two kernels it fuses
    (``attn_with_stats`` of this group, then the merge and the division),
    which recomputes this group's partial result once."""

    @staticmethod
    def forward(ctx, v, w, o1, m1, l1, eps: float, normalize: bool):
        n, b, t, d = _validate(v, w)
        _validate_triple(o1, m1, l1, "prior group")
        if o1.shape != (b, t, d) or o1.dtype != v.dtype or o1.device != v.device:
            raise ValueError(f"prior group: o1 must be [B, T, D] = {(b, t, d)} in v's dtype and device")
        v, w, o1, m1, l1 = (x.contiguous() for x in (v, w, o1, m1, l1))
        n_tok = b * t
        out = torch.empty(b, t, d, device=v.device, dtype=v.dtype)
        m = torch.empty(b, t, device=v.device, dtype=torch.float32)
        ell = torch.empty(b, t, device=v.device, dtype=torch.float32)
        if n_tok > 0 and d > 0:
            with torch.cuda.device(v.device):
                rc = _lib.lib().sy_attn_with_stats_merge(
                    _ptr(v), _ptr(w), _ptr(o1), _ptr(m1), _ptr(l1), _ptr(out), _ptr(m), _ptr(ell), n, n_tok,
                    d, n_tok * d, _lib.dtype_code(v.dtype), _lib.dtype_code(w.dtype), float(eps),
                    int(bool(normalize)), _lib.stream_ptr(v.device),
                )
            _lib.check(rc, "sy_attn_with_stats_merge")
        ctx.save_for_backward(v, w, o1, m1, l1)
        ctx.eps = float(eps)
        ctx.normalize = bool(normalize)
        return out, m, ell

    @staticmethod
    def backward(ctx, gout, gm, gl):
        v, w, o1, m1, l1 = ctx.saved_tensors
        leaves = [x.detach().requires_grad_(need) for x, need in zip((v, w, o1, m1, l1), ctx.needs_input_grad)]
        with torch.enable_grad():
            o2, m2, l2 = attn_with_stats(leaves[0], leaves[1], ctx.eps)
            o, m, ell = merge_online_softmax(leaves[2], leaves[3], leaves[4], o2, m2, l2)
            out = (o.float() / ell.unsqueeze(-1)).to(v.dtype) if ctx.normalize else o
            pairs = [(y, g) for y, g in ((out, gout), (m, gm), (ell, gl)) if g is not None]
            wanted = [x for x in leaves if x.requires_grad]
            grads = torch.autograd.grad([y for y, _ in pairs], wanted, [g for _, g in pairs], allow_unused=True)
        it = iter(grads)
        res = [next(it) if x.requires_grad else None for x in leaves]
        return (*res, None, None)


def attn_with_stats_merge(v: torch.Tensor, w: torch.Tensor, o1: torch.Tensor, m1: torch.Tensor, l1: torch.Tensor,
                          eps: float = DEFAULT_EPS, normalize: bool = True):
    """Phase 2 of the two-phase schedule (the paper's Algorithm 1, lines 10-12;
    reference.py:194-233) in one pass: ``attn_with_stats(v, w)`` merged with a
    prior group's ``(o1, m1, l1)`` by the online softmax before anything is
    written. Returns ``(out, m, l)`` -- ``out`` is the operator's output over
    both groups when ``normalize`` (the default), else the merged unnormalised
    ``o``. Differentiable in every tensor argument."""
    return _AttnWithStatsMerge.apply(v, w, o1, m1, l1, eps, normalize)


def block_attn_res_batched_with_stats(v: torch.Tensor, queries: torch.Tensor, eps: float = DEFAULT_EPS):
    """``(o [S, B, T, D], m [S, B, T], l [S, B, T])``: ``attn_with_stats`` for
    ``S`` pseudo-queries sharing one read of ``v`` -- the batched inter-block
    phase of the two-phase schedule. Output only, like
    ``block_attn_res_batched``."""
    _validate_batched(v, queries)
    if torch.is_grad_enabled() and (v.requires_grad or queries.requires_grad):
        raise RuntimeError("block_attn_res_batched_with_stats has no backward; run it under torch.no_grad()")
    dt = _lib.dtype_code(v.dtype)
    n, b, t, d = v.shape
    s = queries.shape[0]
    v = v.contiguous()
    queries = queries.contiguous()
    o = torch.empty(s, b, t, d, device=v.device, dtype=v.dtype)
    m = torch.empty(s, b, t, device=v.device, dtype=torch.float32)
    ell = torch.empty(s, b, t, device=v.device, dtype=torch.float32)
    n_tok = b * t
    if n_tok == 0:
        return o, m, ell
    with torch.cuda.device(v.device):
        rc = _lib.lib().sy_batched_with_stats(
            _ptr(v), _ptr(queries), _ptr(o), _ptr(m), _ptr(ell), n, s, n_tok, d, n_tok * d, dt,
            float(eps), _lib.stream_ptr(v.device),
        )
    _lib.check(rc, "sy_batched_with_stats")
    return o, m, ell


def block_attn_res_two_phase(v: torch.Tensor, w: torch.Tensor, split: int, eps: float = DEFAULT_EPS):
    """The two-phase schedule for one query: sources ``[0, split)`` reduced to
    their ``(o, m, l)``, then sources ``[split, N)`` reduced and merged with
    them in one pass and normalised (two launches). Differentiable; equals
    ``block_attn_res_triton(v, w)`` up to rounding (reference
    test_reference.py:139-150 states the exactness)."""
    n = v.shape[0] if v.ndim == 4 else 0
    if not 0 < split < n:
        raise ValueError(f"split must be in (0, {n}), got {split}")
    out, _, _ = attn_with_stats_merge(v[split:], w, *attn_with_stats(v[:split], w, eps), eps=eps)
    return out
