"""Block AttnRes over a list of source tensors (pointer-table input).

The reference's operator takes one stacked ``[N, B, T, D]`` tensor, so a
model whose sources are separate tensors pays for a stacking copy or keeps an
arena it writes every sublayer output into. The reference's report names a
per-source pointer table (fla's API) as the better design on that axis
(docs/report.md:401-404). ``block_attn_res_sources`` is that input: the
kernels find row ``n`` of token ``t`` at ``sources[n].data_ptr() + t*D``
through a table carried in the kernel arguments, and the backward writes each
source's gradient through a second table. Same kernels, same bytes and the
same numerics as the stacked operator; at most 16 sources (the table size).
"""

from __future__ import annotations

from typing import Sequence

import torch

from . import _lib
from .hip_op import _ptr
from .reference import DEFAULT_EPS

__all__ = ["block_attn_res_sources", "MAX_SOURCES"]

#: Most sources one call takes (SY_MAX_TABLE_ROWS of include/switchyard.h).
MAX_SOURCES = _lib.MAX_TABLE_ROWS


def _validate_sources(sources: Sequence[torch.Tensor], w: torch.Tensor) -> tuple[int, int, int, int]:
    if len(sources) == 0:
        raise ValueError("sources must hold at least one [B, T, D] tensor")
    if len(sources) > MAX_SOURCES:
        raise ValueError(
            f"at most {MAX_SOURCES} sources per call, got {len(sources)}; stack them into "
            "[N, B, T, D] and call block_attn_res_triton"
        )
    first = sources[0]
    if first.ndim != 3:
        raise ValueError(f"each source must be [B, T, D], got {tuple(first.shape)}")
    b, t, d = first.shape
    for s in sources:
        if s.shape != first.shape:
            raise ValueError(f"every source must be [{b}, {t}, {d}], got {tuple(s.shape)}")
        if not s.is_cuda:
            raise ValueError("sources must be on a CUDA device")
        if s.device != first.device:
            raise ValueError("every source must be on the same CUDA device")
        if s.dtype != first.dtype:
            raise ValueError("every source must have the same dtype")
    if w.shape != (d,):
        raise ValueError(f"w must be [{d}], got {tuple(w.shape)}")
    if w.device != first.device:
        raise ValueError("w must be on the same CUDA device as the sources")
    _lib.dtype_code(first.dtype)
    _lib.dtype_code(w.dtype)
    return len(sources), b, t, d


class _BlockAttnResSources(torch.autograd.Function):
    @staticmethod
    def forward(ctx, w: torch.Tensor, eps: float, *sources: torch.Tensor):
        n, b, t, d = _validate_sources(sources, w)
        sources = tuple(s.contiguous() for s in sources)
        w = w.contiguous()
        dev = sources[0].device
        out = torch.empty(b, t, d, device=dev, dtype=sources[0].dtype)
        n_tok = b * t
        want_grad = any(ctx.needs_input_grad)
        stats = (
            torch.empty(2, n, n_tok, device=dev, dtype=torch.float32)
            if want_grad and n_tok > 0 and d > 0
            else None
        )
        if n_tok > 0 and d > 0:
            table = _lib.pointer_table(sources)
            with torch.cuda.device(dev):
                rc = _lib.lib().sy_fwd_table(
                    table, _ptr(w), _ptr(out), _ptr(stats), n, n_tok, d,
                    _lib.dtype_code(out.dtype), _lib.dtype_code(w.dtype), float(eps),
                    _lib.stream_ptr(dev),
                )
            _lib.check(rc, "sy_fwd_table")
        ctx.save_for_backward(w, stats, *sources)
        ctx.eps = float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        w, stats, *sources = ctx.saved_tensors
        n = len(sources)
        b, t, d = sources[0].shape
        n_tok = b * t
        dev = sources[0].device
        dt = sources[0].dtype
        grad_out = grad_out.to(dt).contiguous()
        # One allocation; each source's gradient is a [B, T, D] slice of it.
        dv = torch.empty(n, b, t, d, device=dev, dtype=dt)
        dvs = dv.unbind(0)
        dw = torch.empty(d, device=dev, dtype=w.dtype)
        if d == 0:
            return (dw, None, *dvs)
        lib = _lib.lib()
        vt, wt = _lib.dtype_code(dt), _lib.dtype_code(w.dtype)
        with torch.cuda.device(dev):
            ws_bytes = lib.sy_bwd_workspace_bytes(n, n_tok, d, vt, wt)
            if ws_bytes < 0:
                _lib.check(int(ws_bytes), "sy_bwd_workspace_bytes")
            ws = torch.empty(max(1, (ws_bytes + 3) // 4), device=dev, dtype=torch.float32)
            rc = lib.sy_bwd_table(
                _lib.pointer_table(sources), _ptr(w), _ptr(grad_out), _ptr(stats),
                _lib.pointer_table(dvs), _ptr(dw), _ptr(ws), ws.numel() * 4, n, n_tok, d, vt, wt,
                ctx.eps, _lib.stream_ptr(dev),
            )
        _lib.check(rc, "sy_bwd_table")
        return (dw, None, *dvs)


def block_attn_res_sources(
    sources: Sequence[torch.Tensor], w: torch.Tensor, eps: float = DEFAULT_EPS
) -> torch.Tensor:
    """Block AttnRes over ``N`` separate ``[B, T, D]`` source tensors, with autograd.

    Equals ``block_attn_res_triton(torch.stack(sources), w, eps)`` bit for bit
    (the same kernels see the same rows), without the stack. Each source gets
    its own ``[B, T, D]`` gradient; ``dw`` is reduced in fp32 and returned in
    ``w.dtype``. ``1 <= N <= 16``.
    """
    return _BlockAttnResSources.apply(w, eps, *sources)
