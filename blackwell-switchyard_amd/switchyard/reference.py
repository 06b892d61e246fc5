"""Constants, the per-layer parameter module and the byte/FLOP model.

Mirrors the product-facing parts of the reference's ``switchyard.reference``
(src/switchyard/reference.py of sabdulmajid/blackwell-switchyard):
``DEFAULT_EPS`` (:93-95), the ``BlockAttnRes`` parameter module (:149-183) and
the roofline denominators (:236-271). The float64 oracle itself is test
infrastructure and lives in ``oracle/reference.py`` at the repository root;
nothing here calls it.

The operator, per token with sources ``v_0..v_{N-1}`` and query ``w``::

    k_n   = v_n / sqrt(mean(v_n ** 2) + eps)
    alpha = softmax_n(<w, k_n>)              # no 1/sqrt(D)
    out   = sum_n alpha_n v_n                # raw, not normalised, sources
"""

from __future__ import annotations

import torch
import torch.nn as nn

__all__ = [
    "DEFAULT_EPS",
    "BlockAttnRes",
    "attn_res_flops",
    "attn_res_min_bytes",
    "attn_res_train_bytes",
    "attn_res_batched_bytes",
    "arithmetic_intensity",
    "ridge_point",
]

#: RMSNorm epsilon. The paper states none; 1e-6 is the Llama / Kimi Linear
#: convention the reference adopts (reference.py:93-95).
DEFAULT_EPS = 1e-6


class BlockAttnRes(nn.Module):
    """One layer's Block AttnRes parameters: the pseudo-query ``w``, initialised
    to zeros so attention starts uniform (paper Sec. 5), and an RMSNorm gain
    ``g`` that is mathematically redundant with ``w`` (``<w, g*x> = <w*g, x>``)
    and folded into ``w`` before the operator runs (reference.py:149-183).

    ``forward`` evaluates the eager framework formulation
    (:func:`switchyard.baselines.folded_form`), as the reference's module
    evaluates its eager paper form; the fused HIP path is
    :class:`switchyard.hip_op.BlockAttnResHIP`.
    """

    def __init__(self, d_model: int, norm_affine: bool = True, eps: float = DEFAULT_EPS) -> None:
        super().__init__()
        self.d_model = d_model
        self.eps = eps
        self.w = nn.Parameter(torch.zeros(d_model))
        self.g = nn.Parameter(torch.ones(d_model)) if norm_affine else None

    def extra_repr(self) -> str:
        return f"d_model={self.d_model}, norm_affine={self.g is not None}, eps={self.eps}"

    def effective_query(self) -> torch.Tensor:
        """``w * g``, the single vector the kernels consume."""
        return self.w if self.g is None else self.w * self.g

    def forward(self, v: torch.Tensor) -> torch.Tensor:
        from .baselines import folded_form

        return folded_form(v, self.effective_query(), self.eps)


def attn_res_flops(n: int, b: int, t: int, d: int) -> int:
    """Sum of squares, query dot and weighted sum: 3 multiply-adds per source
    element, 2 FLOP each (reference.py:236-244)."""
    return 2 * n * b * t * d * 3


def attn_res_min_bytes(n: int, b: int, t: int, d: int, itemsize: int = 2) -> int:
    """Forward traffic lower bound: every source read once, the output written
    once, ``(N + 1)`` slabs of ``B*T*D`` (reference.py:247-255)."""
    return (n * b * t * d + b * t * d) * itemsize


def attn_res_train_bytes(n: int, b: int, t: int, d: int, itemsize: int = 2) -> int:
    """Forward + backward lower bound, ``(3N + 2)`` slabs: the forward reads v
    and writes out; the backward reads v and grad_out and writes dv."""
    return (3 * n + 2) * b * t * d * itemsize


def attn_res_batched_bytes(n: int, s: int, b: int, t: int, d: int, itemsize: int = 2) -> int:
    """Batched forward lower bound, ``(N + S)`` slabs plus the queries
    (reference bench/bench_third_party.py:328-331)."""
    return (n + s) * b * t * d * itemsize + s * d * itemsize


def arithmetic_intensity(n: int, b: int, t: int, d: int, itemsize: int = 2) -> float:
    """FLOP per byte at the traffic lower bound; depends on N only
    (reference.py:258-266)."""
    return attn_res_flops(n, b, t, d) / attn_res_min_bytes(n, b, t, d, itemsize)


def ridge_point(peak_flops: float, peak_bandwidth: float) -> float:
    """Machine balance in FLOP per byte (reference.py:269-271)."""
    return peak_flops / peak_bandwidth
