"""Framework-native (eager PyTorch) Block AttnRes formulations.

The comparators the fused HIP operator is measured against, and the operator
the Transformer's ``"attnres"`` residual mode evaluates. Same names and
arithmetic arrangement as the reference's ``switchyard.baselines``
(src/switchyard/baselines.py:57-104). They run on any device torch supports;
the HIP operator never calls them.
"""

from __future__ import annotations

import torch
from torch import Tensor

from .reference import DEFAULT_EPS

__all__ = ["paper_form", "folded_form", "batched_folded_form", "chunked_form", "FORMULATIONS"]


def paper_form(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """Paper pseudocode: materialises the normalised keys (baselines.py:57-61)."""
    keys = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    scores = torch.einsum("d,nbtd->nbt", w, keys)
    return torch.einsum("nbt,nbtd->btd", scores.softmax(0), v)


def folded_form(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """RMS scale folded into the score, ``<w, v/rms> = <w, v>/rms``; the
    normalised tensor is never formed (baselines.py:64-73)."""
    qdot = torch.einsum("d,nbtd->nbt", w, v)
    rinv = torch.rsqrt(v.pow(2).mean(-1) + eps)
    weights = (qdot * rinv).softmax(0)
    return torch.einsum("nbt,nbtd->btd", weights, v)


def batched_folded_form(v: Tensor, queries: Tensor, eps: float = DEFAULT_EPS) -> Tensor:
    """``S`` queries sharing the sources (baselines.py:76-81)."""
    qdot = torch.einsum("sd,nbtd->snbt", queries, v)
    rinv = torch.rsqrt(v.pow(2).mean(-1) + eps)
    weights = (qdot * rinv.unsqueeze(0)).softmax(1)
    return torch.einsum("snbt,nbtd->sbtd", weights, v)


def chunked_form(v: Tensor, w: Tensor, eps: float = DEFAULT_EPS, chunk: int = 2048) -> Tensor:
    """``folded_form`` over token-axis tiles of ``chunk`` positions
    (baselines.py:84-96)."""
    t = v.shape[2]
    if chunk >= t:
        return folded_form(v, w, eps)
    return torch.cat([folded_form(v[:, :, i : i + chunk], w, eps) for i in range(0, t, chunk)], dim=1)


#: Name -> callable, for benchmark iteration (baselines.py:99-104).
FORMULATIONS = {
    "paper_form": paper_form,
    "folded_form": folded_form,
    "chunked_form": chunked_form,
}
