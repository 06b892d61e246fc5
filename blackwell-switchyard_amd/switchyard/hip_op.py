"""Block AttnRes on MI355X: the autograd operator and the batched forward.

Drop-in for the reference's ``switchyard.triton_op`` (src/switchyard/
triton_op.py of sabdulmajid/blackwell-switchyard): same names, argument
meaning, validation messages and gradient contract, backed by hand-written
HIP kernels for gfx950 behind the C ABI of ``include/switchyard.h``.

Per token ``(b, t)`` with sources ``v_0..v_{N-1}`` and pseudo-query ``w``::

    r_n    = rsqrt(mean(v_n ** 2) + eps)
    alpha  = softmax_n(r_n * <w, v_n>)       # no 1/sqrt(D)
    out    = sum_n alpha_n * v_n             # raw sources

The forward reads ``v`` once and writes ``out`` once (one kernel). When a
gradient is needed it also writes the per-(source, token) logits and inverse
RMS (``[2, N, B*T]`` fp32) so the backward need only reduce ``<g, v_n>``.
The backward is one persistent kernel that writes ``dv`` and per-workgroup
fp32 ``dw`` partials, then a fixed-order reduction writes ``dw`` in
``w.dtype``: two kernels, no float atomics, bit-reproducible.

There is no fallback: when the HIP library is missing, or a tensor is not on
a GPU, these functions raise.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from .reference import DEFAULT_EPS

__all__ = [
    "block_attn_res_hip",
    "block_attn_res_batched",
    "block_attn_res_batched_train",
    "BlockAttnResHIP",
    "speed_of_light",
    "bandwidth_probe",
    "bwd_workspace_bytes",
]


def _ptr(t: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _validate(v: torch.Tensor, w: torch.Tensor) -> tuple[int, int, int, int]:
    """The reference's checks and messages (triton_op.py:507-513), plus the
    ones a C ABI needs (same device, supported dtypes, N >= 1)."""
    if v.ndim != 4:
        raise ValueError(f"v must be [N, B, T, D], got {tuple(v.shape)}")
    n, b, t, d = v.shape
    if w.shape != (d,):
        raise ValueError(f"w must be [{d}], got {tuple(w.shape)}")
    if not v.is_cuda:
        raise ValueError("v must be on a CUDA device")
    if w.device != v.device:
        raise ValueError("w must be on the same CUDA device as v")
    _lib.dtype_code(v.dtype)
    _lib.dtype_code(w.dtype)
    if n == 0:
        raise ValueError("N (the number of sources) must be positive")
    return n, b, t, d


class _BlockAttnResHIP(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v: torch.Tensor, w: torch.Tensor, eps: float):
        n, b, t, d = _validate(v, w)
        # Tokens are walked with one stride, so B and T must be flattenable;
        # a strided input is copied rather than misread (triton_op.py:515-519).
        v = v.contiguous()
        w = w.contiguous()
        out = torch.empty(b, t, d, device=v.device, dtype=v.dtype)
        n_tok = b * t
        want_grad = bool(ctx.needs_input_grad[0] or ctx.needs_input_grad[1])
        stats = (
            torch.empty(2, n, n_tok, device=v.device, dtype=torch.float32)
            if want_grad and n_tok > 0 and d > 0
            else None
        )
        if n_tok > 0 and d > 0:
            lib = _lib.lib()
            with torch.cuda.device(v.device):
                rc = lib.sy_fwd(
                    _ptr(v), _ptr(w), _ptr(out), _ptr(stats), n, n_tok, d, n_tok * d,
                    _lib.dtype_code(v.dtype), _lib.dtype_code(w.dtype), float(eps),
                    _lib.stream_ptr(v.device),
                )
            _lib.check(rc, "sy_fwd")
        ctx.save_for_backward(v, w, stats)
        ctx.eps = float(eps)
        return out

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        v, w, stats = ctx.saved_tensors
        n, b, t, d = v.shape
        n_tok = b * t
        grad_out = grad_out.to(v.dtype).contiguous()
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
            rc = lib.sy_bwd(
                _ptr(v), _ptr(w), _ptr(grad_out), _ptr(stats), _ptr(dv), _ptr(dw), _ptr(ws),
                ws.numel() * 4, n, n_tok, d, n_tok * d, vt, wt, ctx.eps, _lib.stream_ptr(v.device),
            )
        _lib.check(rc, "sy_bwd")
        return dv, dw, None


def block_attn_res_hip(v: torch.Tensor, w: torch.Tensor, eps: float = DEFAULT_EPS) -> torch.Tensor:
    """Fused Block AttnRes with autograd; same contract as the reference's
    ``block_attn_res_triton`` (triton_op.py:592-594).

    Args:
        v: ``[N, B, T, D]`` sources on a GPU (bf16, fp16 or fp32).
        w: ``[D]`` pseudo-query, any of those dtypes (upcast in the kernel).
        eps: RMSNorm epsilon.

    Returns:
        ``[B, T, D]`` in ``v.dtype``. Gradients: ``dv`` in ``v.dtype``, ``dw``
        accumulated in fp32 and returned in ``w.dtype``.
    """
    return _BlockAttnResHIP.apply(v, w, eps)


def _validate_batched(v: torch.Tensor, queries: torch.Tensor) -> None:
    """The reference's batched checks and messages (triton_op.py:438-462)."""
    if v.ndim != 4:
        raise ValueError(f"v must be [N, B, T, D], got {tuple(v.shape)}")
    if queries.ndim != 2 or queries.shape[1] != v.shape[-1]:
        raise ValueError(f"queries must be [S, {v.shape[-1]}], got {tuple(queries.shape)}")
    if not v.is_cuda or not queries.is_cuda:
        raise ValueError("v and queries must be CUDA tensors")
    if v.device != queries.device:
        raise ValueError("v and queries must be on the same CUDA device")
    if v.dtype != queries.dtype:
        raise ValueError("v and queries must have the same dtype")
    if v.shape[0] == 0 or queries.shape[0] == 0 or v.shape[-1] == 0:
        raise ValueError("N, S, and D must be positive")
    _lib.dtype_code(v.dtype)


def _batched_forward(v: torch.Tensor, queries: torch.Tensor, eps: float) -> torch.Tensor:
    n, b, t, d = v.shape
    s = queries.shape[0]
    out = torch.empty(s, b, t, d, device=v.device, dtype=v.dtype)
    n_tok = b * t
    if n_tok == 0:
        return out
    with torch.cuda.device(v.device):
        rc = _lib.lib().sy_fwd_batched(
            _ptr(v), _ptr(queries), _ptr(out), n, s, n_tok, d, n_tok * d,
            _lib.dtype_code(v.dtype), float(eps), _lib.stream_ptr(v.device),
        )
    _lib.check(rc, "sy_fwd_batched")
    return out


class _BlockAttnResBatched(torch.autograd.Function):
    @staticmethod
    def forward(ctx, v: torch.Tensor, queries: torch.Tensor, eps: float):
        _validate_batched(v, queries)
        v = v.contiguous()
        queries = queries.contiguous()
        ctx.save_for_backward(v, queries)
        ctx.eps = float(eps)
        return _batched_forward(v, queries, eps)

    @staticmethod
    def backward(ctx, grad_out: torch.Tensor):
        v, queries = ctx.saved_tensors
        n, b, t, d = v.shape
        s = queries.shape[0]
        n_tok = b * t
        grad_out = grad_out.to(v.dtype).contiguous()
        dv = torch.empty_like(v, memory_format=torch.contiguous_format)
        dq = torch.empty_like(queries)
        lib = _lib.lib()
        dt = _lib.dtype_code(v.dtype)
        with torch.cuda.device(v.device):
            ws_bytes = lib.sy_bwd_batched_workspace_bytes(n, s, n_tok, d, dt)
            if ws_bytes < 0:
                _lib.check(int(ws_bytes), "sy_bwd_batched_workspace_bytes")
            ws = torch.empty(max(1, (ws_bytes + 3) // 4), device=v.device, dtype=torch.float32)
            rc = lib.sy_bwd_batched(
                _ptr(v), _ptr(queries), _ptr(grad_out), _ptr(dv), _ptr(dq), _ptr(ws), ws.numel() * 4,
                n, s, n_tok, d, n_tok * d, dt, ctx.eps, _lib.stream_ptr(v.device),
            )
        _lib.check(rc, "sy_bwd_batched")
        return dv, dq, None


def block_attn_res_batched_train(
    v: torch.Tensor, queries: torch.Tensor, eps: float = DEFAULT_EPS
) -> torch.Tensor:
    """``block_attn_res_batched`` with a backward: ``out[s] = AttnRes(v, queries[s])``.

    The reference's batched API is output-only and raises under autograd
    (triton_op.py:463-467, kept as is in ``block_attn_res_batched``); this is
    its training contract. Forward: the same single read of ``v`` for all
    queries. Backward: one persistent kernel reads ``v`` and the ``S``
    output gradients once, writes ``dv = sum_s dv_s`` rounded once and fp32
    per-workgroup ``dq`` partials, then the fixed-order reduction writes
    ``dq`` -- two kernels, bit-reproducible.
    """
    return _BlockAttnResBatched.apply(v, queries, eps)


def block_attn_res_batched(
    v: torch.Tensor, queries: torch.Tensor, eps: float = DEFAULT_EPS
) -> torch.Tensor:
    """``S`` pseudo-queries against one shared read of ``v`` (output only).

    Same contract as the reference's ``block_attn_res_batched``
    (triton_op.py:438-501): ``out[s] == block_attn_res_triton(v, queries[s])``,
    ``[S, B, T, D]``, no backward. For N, D, dtype the resident kernel holds
    and S <= 16 one kernel reads ``v`` once; other shapes issue one forward
    launch per query, written straight into ``out[s]`` (no stack).
    """
    _validate_batched(v, queries)
    if v.requires_grad or queries.requires_grad:
        raise RuntimeError(
            "block_attn_res_batched has no backward; use block_attn_res_triton per query "
            "for training, or run this under torch.no_grad() for inference"
        )
    return _batched_forward(v.contiguous(), queries.contiguous(), eps)


class BlockAttnResHIP(torch.nn.Module):
    """Module form (reference triton_op.py:597-609): zero-initialised query
    ``w`` and unit RMSNorm gain ``g``; the kernel sees ``w * g``."""

    def __init__(self, d_model: int, norm_affine: bool = True, eps: float = DEFAULT_EPS) -> None:
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.w = torch.nn.Parameter(torch.zeros(d_model))
        self.g = torch.nn.Parameter(torch.ones(d_model)) if norm_affine else None

    def forward(self, v: torch.Tensor) -> torch.Tensor:
        q = self.w if self.g is None else self.w * self.g
        return block_attn_res_hip(v, q, self.eps)


def speed_of_light(v: torch.Tensor) -> torch.Tensor:
    """The traffic-only ceiling (triton_op.py:153-191): reads every source
    element and writes ``sum_n v_n`` per token with the forward's geometry."""
    if v.ndim != 4 or not v.is_cuda:
        raise ValueError("v must be a [N, B, T, D] CUDA tensor")
    n, b, t, d = v.shape
    v = v.contiguous()
    out = torch.empty(b, t, d, device=v.device, dtype=v.dtype)
    if b * t and d:
        with torch.cuda.device(v.device):
            rc = _lib.lib().sy_sol(_ptr(v), _ptr(out), n, b * t, d, b * t * d,
                                   _lib.dtype_code(v.dtype), _lib.stream_ptr(v.device))
        _lib.check(rc, "sy_sol")
    return out


def bandwidth_probe(kind: str, src: torch.Tensor | None, dst: torch.Tensor) -> None:
    """HBM probe (reference bench/machine.py:41-61): ``read`` streams ``src``
    (``dst`` receives one float per workgroup, see ``probe_grid``), ``write``
    fills ``dst``, ``copy`` copies ``src`` into ``dst``, ``mix`` reads ``src``
    and writes ``dst`` (a ninth of its size) as one linear stream -- the
    forward's 9:1 read:write ratio without its row stride."""
    code = {"read": 0, "write": 1, "copy": 2, "mix": 3}[kind]
    nbytes = (src if code != 1 else dst).numel() * (src if code != 1 else dst).element_size()
    with torch.cuda.device(dst.device):
        rc = _lib.lib().sy_bw_probe(code, _ptr(src), _ptr(dst), nbytes, _lib.stream_ptr(dst.device))
    _lib.check(rc, "sy_bw_probe")


def probe_grid(nbytes: int) -> int:
    """Workgroups the read probe uses (floats ``dst`` must hold)."""
    return int(_lib.lib().sy_probe_grid(nbytes))


def bwd_workspace_bytes(n: int, n_tok: int, d: int, v_dtype: torch.dtype,
                        w_dtype: torch.dtype | None = None) -> int:
    """Device workspace the backward needs on the current device."""
    r = _lib.lib().sy_bwd_workspace_bytes(n, n_tok, d, _lib.dtype_code(v_dtype),
                                          _lib.dtype_code(w_dtype or v_dtype))
    if r < 0:
        _lib.check(int(r), "sy_bwd_workspace_bytes")
    return int(r)


# --------------------------------------------------------------------------
# Dispatch introspection, mirroring the reference's helpers that its tests
# import (triton_op.py:130-150, :267-276, :420-435). Pure host arithmetic.
# --------------------------------------------------------------------------


def _launch_config(n: int, d: int, dtype: torch.dtype = torch.bfloat16) -> tuple[bool, int, int, int]:
    """Forward plan: ``(resident, waves_per_token, chunks_per_lane, rows_per_tile)``.
    ``resident`` means the whole token tile is held in registers (one read of v,
    one softmax). Unlike the reference, ``n`` is the real source count."""
    p = _lib.plan(_lib.OP_FWD, n, d, dtype)
    return p["family_name"] == "resident", p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]


def _bwd_launch(n: int, d: int, dtype: torch.dtype = torch.bfloat16) -> tuple[bool, int, int, int]:
    """Backward plan: ``(resident, tokens_per_block, waves_per_token, rows_per_tile)``."""
    p = _lib.plan(_lib.OP_BWD, n, d, dtype)
    return p["family_name"] == "resident", p["tokens_per_block"], p["waves_per_token"], p["rows_per_tile"]


def _batched_launch(n: int, d: int, s: int, dtype: torch.dtype = torch.bfloat16) -> tuple[bool, int, int, int]:
    """Batched plan: ``(one_kernel, waves_per_token, chunks_per_lane, rows_per_tile)``;
    one_kernel is the reference's "resident" flag (one launch for all queries),
    true for the register-tiled and the matrix-core kernels."""
    p = _lib.plan(_lib.OP_BATCHED, n, d, dtype, n_q=s)
    one = p["family_name"] in ("resident", "matrix")
    return one, p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]
