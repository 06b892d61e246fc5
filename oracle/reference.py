"""TEST INFRASTRUCTURE: float64 torch restatement of the reference's oracle.

Follows ``src/switchyard/reference.py`` of sabdulmajid/blackwell-switchyard
(the paper's Eq. 2-4/6, Kimi Team, arXiv:2603.15031) and the eager
formulations of ``src/switchyard/baselines.py``; the parity metric follows
``bench/harness.py:295-358``. Written from the published mathematics; every
function cites the reference lines it restates.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's cpu_baseline leg use
this module.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

#: The paper states no epsilon; the reference uses 1e-6 (reference.py:93-95).
DEFAULT_EPS = 1e-6


def rms_norm(x: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """RMS normalisation over the last axis, no gain (reference.py:98-104)."""
    return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)


def block_attn_res_reference(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """Block AttnRes as the paper writes it (reference.py:107-133).

    ``v: [N, B, T, D]``, ``w: [D]`` -> ``[B, T, D]``: keys are RMS-normalised
    sources, logits are ``<w, k>`` with no 1/sqrt(D), the softmax runs over the
    source axis and the weighted sum uses the raw sources.
    """
    if v.ndim != 4:
        raise ValueError(f"v must be [N, B, T, D], got shape {tuple(v.shape)}")
    if w.ndim != 1:
        raise ValueError(f"w must be [D], got shape {tuple(w.shape)}")
    if w.shape[0] != v.shape[-1]:
        raise ValueError(f"w has D={w.shape[0]} but v has D={v.shape[-1]}")
    k = rms_norm(v, eps)
    logits = torch.einsum("d,nbtd->nbt", w, k)
    alpha = logits.softmax(0)
    return torch.einsum("nbt,nbtd->btd", alpha, v)


def block_attn_res_oracle(
    v: Tensor, w: Tensor, eps: float = DEFAULT_EPS, dtype: torch.dtype = torch.float64
) -> Tensor:
    """The high-precision oracle (reference.py:136-146): promote, then evaluate."""
    return block_attn_res_reference(v.to(dtype), w.to(dtype), eps)


def attn_with_stats(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> tuple[Tensor, Tensor, Tensor]:
    """``(o, m, ell)`` of the paper's Algorithm 1 (reference.py:195-216)."""
    k = rms_norm(v, eps)
    logits = torch.einsum("d,nbtd->nbt", w, k)
    m = logits.amax(0)
    p = (logits - m).exp()
    o = torch.einsum("nbt,nbtd->btd", p, v)
    return o, m, p.sum(0)


def merge_online_softmax(o1, m1, l1, o2, m2, l2):
    """Exact merge of two partial results (reference.py:219-233)."""
    m = torch.maximum(m1, m2)
    s1 = (m1 - m).exp()
    s2 = (m2 - m).exp()
    return o1 * s1.unsqueeze(-1) + o2 * s2.unsqueeze(-1), m, l1 * s1 + l2 * s2


def paper_form(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """Eager transcription that materialises k (baselines.py:57-61)."""
    k = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    logits = torch.einsum("d,nbtd->nbt", w, k)
    return torch.einsum("nbt,nbtd->btd", logits.softmax(0), v)


def folded_form(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """Eager form with the RMS scale folded into the score (baselines.py:64-73).

    This is the CPU baseline bench.py times (fp32, forward and backward).
    """
    dots = torch.einsum("d,nbtd->nbt", w, v)
    inv_rms = torch.rsqrt(v.pow(2).mean(-1) + eps)
    alpha = (dots * inv_rms).softmax(0)
    return torch.einsum("nbt,nbtd->btd", alpha, v)


def batched_folded_form(v: Tensor, queries: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """``S`` queries against shared sources (baselines.py:76-81)."""
    dots = torch.einsum("sd,nbtd->snbt", queries, v)
    inv_rms = torch.rsqrt(v.pow(2).mean(-1) + eps)
    alpha = (dots * inv_rms.unsqueeze(0)).softmax(1)
    return torch.einsum("snbt,nbtd->sbtd", alpha, v)


def oracle_grads(v: Tensor, w: Tensor, g: Tensor, eps: float = DEFAULT_EPS) -> tuple[Tensor, Tensor]:
    """``(dv, dw)`` of the paper form by float64 autograd, as the reference's
    backward test computes them (tests/test_triton_op.py:151-165)."""
    vv = v.detach().to(torch.float64).clone().requires_grad_(True)
    ww = w.detach().to(torch.float64).clone().requires_grad_(True)
    k = vv * torch.rsqrt(vv.pow(2).mean(-1, keepdim=True) + eps)
    out = torch.einsum("nbt,nbtd->btd", torch.einsum("d,nbtd->nbt", ww, k).softmax(0), vv)
    out.backward(g.detach().to(torch.float64))
    return vv.grad, ww.grad


# --------------------------------------------------------------------------
# Byte / FLOP model (reference.py:236-271)
# --------------------------------------------------------------------------


def attn_res_flops(n: int, b: int, t: int, d: int) -> int:
    """Three multiply-add passes over ``[N, B, T, D]`` (reference.py:236-244)."""
    return 2 * n * b * t * d * 3


def attn_res_min_bytes(n: int, b: int, t: int, d: int, itemsize: int = 2) -> int:
    """Read every source once, write the output once (reference.py:247-255)."""
    return (n * b * t * d + b * t * d) * itemsize


def arithmetic_intensity(n: int, b: int, t: int, d: int, itemsize: int = 2) -> float:
    """FLOP per byte at minimum traffic (reference.py:258-266)."""
    return attn_res_flops(n, b, t, d) / attn_res_min_bytes(n, b, t, d, itemsize)


# --------------------------------------------------------------------------
# Parity metric (bench/harness.py:295-358, tests/test_triton_op.py:35-44)
# --------------------------------------------------------------------------


def rel_l2(got: Tensor, oracle: Tensor) -> float:
    """``||got - oracle|| / ||oracle||`` in float64."""
    g = got.detach().to(torch.float64).cpu()
    o = oracle.detach().to(torch.float64).cpu()
    return ((g - o).norm() / o.norm()).item()


def dtype_floor(oracle: Tensor, dtype: torch.dtype) -> float:
    """What rounding the exact answer to ``dtype`` alone costs, in rel-L2."""
    o = oracle.detach().to(torch.float64).cpu()
    return ((o.to(dtype).to(torch.float64) - o).norm() / o.norm()).item()


def check_against(got: Tensor, oracle: Tensor, *, rel_l2_tol: float) -> dict:
    """Report of one candidate against the oracle (harness.py:295-358)."""
    if tuple(got.shape) != tuple(oracle.shape):
        return {"ok": False, "error": f"shape {tuple(got.shape)} != {tuple(oracle.shape)}"}
    o = oracle.detach().to(torch.float64).cpu()
    g = got.detach().to(torch.float64).cpu()
    diff = g - o
    o_norm = o.norm().item()
    o_rms = o.pow(2).mean().sqrt().item()
    err = diff.norm().item() / o_norm if o_norm > 0 else math.inf
    floor = dtype_floor(o, got.dtype) if o_norm > 0 else 0.0
    has_nan = bool(torch.isnan(g).any().item())
    return {
        "ok": bool(err <= rel_l2_tol) and not has_nan,
        "rel_l2": err,
        "rel_l2_tol": rel_l2_tol,
        "dtype_floor_rel_l2": floor,
        "err_vs_dtype_floor": err / floor if floor > 0 else None,
        "max_abs_err": diff.abs().max().item() if diff.numel() else 0.0,
        "max_abs_err_over_rms": (diff.abs().max().item() / o_rms) if o_rms > 0 else None,
        "output_rms": o_rms,
        "has_nan": has_nan,
        "has_inf": bool(torch.isinf(g).any().item()),
    }
