"""Decoder-only Transformer with a switchable residual mechanism.

Restates the reference's ``switchyard.model`` (src/switchyard/model.py of
sabdulmajid/blackwell-switchyard): the same three residual modes, the same
Block AttnRes wiring (paper Eq. 6, two sites per layer plus a readout site),
and the same source arena, with the ``"switchyard"`` mode calling the HIP
operator.

Residual modes (model.py:132-143):
  ``standard``    PreNorm ``x = x + sublayer(norm(x))`` -- the control.
  ``attnres``     Block AttnRes through the eager ``folded_form``.
  ``switchyard``  Block AttnRes through the HIP operator.

Block AttnRes wiring (model.py:26-57). A sublayer is the paper's "layer"; the
``2 * n_layers`` sublayers are split into ``n_blocks`` blocks. ``blocks[0]`` is
the embedding, ``blocks[j]`` the completed block ``j``; ``partial`` is the
unweighted running sum of the current block's sublayer outputs. Sublayer ``i``
attends over ``blocks[0..n]`` (plus ``partial`` unless it opens its block);
its output replaces the residual stream input. A readout site over every block
feeds the LM head.

Source arena (model.py:59-104). Instead of ``torch.stack`` at every site, one
``[n_blocks + 1, B, T, D]`` buffer holds the embedding in slot 0, block ``j``
in slot ``j`` and the running partial in the next free slot (whose final value
*is* the next block, so a block boundary writes nothing). Each site hands the
operator ``arena[:n_src]`` -- a contiguous prefix, which the HIP op reads in
place through its source stride. The prefix is an alias made with
``Tensor.set_`` so it has its own autograd version counter; the partial slot,
the only slot rewritten later, is restored from the saved partial before the
site's backward runs. Sites' backwards run in reverse order, so each restore
happens after every later site is done with the slot.
"""

from __future__ import annotations

import contextlib
import math
from collections.abc import Callable
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F
from torch import Tensor

from .baselines import folded_form
from .reference import DEFAULT_EPS, BlockAttnRes

__all__ = [
    "ModelConfig",
    "Transformer",
    "RESIDUAL_MODES",
    "SOURCE_MODES",
    "source_count_schedule",
    "slab_copies",
]

RESIDUAL_MODES = ("standard", "attnres", "switchyard")
SOURCE_MODES = ("arena", "stack")


def _hip_impl(v: Tensor, w: Tensor, eps: float) -> Tensor:
    from .hip_op import block_attn_res_hip

    return block_attn_res_hip(v, w, eps)


#: Residual mode -> operator ``(v, w, eps) -> [B, T, D]``.
_IMPLS: dict[str, Callable[[Tensor, Tensor, float], Tensor]] = {
    "attnres": folded_form,
    "switchyard": _hip_impl,
}


@dataclass
class ModelConfig:
    """Model shape (model.py:151-202). Defaults: the 1.3B configuration of
    BASELINE.json (24 layers, d_model 2048, 16 heads, 8 blocks, vocab 32000;
    the reference used 32768)."""

    vocab_size: int = 32000
    d_model: int = 2048
    n_layers: int = 24
    n_heads: int = 16
    d_ff: int = 5632
    n_blocks: int = 8
    max_seq_len: int = 4096
    rope_theta: float = 10000.0
    norm_eps: float = DEFAULT_EPS
    tie_embeddings: bool = True
    residual: str = "standard"
    sources: str = "arena"

    def __post_init__(self) -> None:
        if self.residual not in RESIDUAL_MODES:
            raise ValueError(f"residual must be one of {RESIDUAL_MODES}, got {self.residual!r}")
        if self.sources not in SOURCE_MODES:
            raise ValueError(f"sources must be one of {SOURCE_MODES}, got {self.sources!r}")
        if self.d_model % self.n_heads:
            raise ValueError(f"d_model {self.d_model} not divisible by n_heads {self.n_heads}")
        if self.n_sublayers % self.n_blocks:
            raise ValueError(
                f"n_blocks {self.n_blocks} must divide the sublayer count {self.n_sublayers} "
                "(= 2 * n_layers); a block is a whole number of sublayers"
            )

    @property
    def n_sublayers(self) -> int:
        return 2 * self.n_layers

    @property
    def block_size(self) -> int:
        return self.n_sublayers // self.n_blocks

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def uses_attnres(self) -> bool:
        return self.residual != "standard"


def source_count_schedule(n_sublayers: int, n_blocks: int) -> list[int]:
    """Sources each AttnRes site attends over (paper Eq. 6, model.py:205-219):
    sublayer ``i`` of block ``k = i // block_size`` sees ``k + 1`` blocks, plus
    the partial unless it opens its block; the last entry is the readout."""
    per_block = n_sublayers // n_blocks
    counts = []
    for i in range(n_sublayers):
        k, opens = divmod(i, per_block)
        counts.append(k + 1 + (0 if opens == 0 else 1))
    return counts + [n_blocks + 1]


def slab_copies(n_sublayers: int, n_blocks: int, sources: str) -> int:
    """``B*T*D`` slabs copied to stage sources in one forward (model.py:222-235):
    stacking copies every source at every site; the arena writes the embedding
    once and the partial once per sublayer."""
    if sources == "stack":
        return sum(source_count_schedule(n_sublayers, n_blocks))
    return n_sublayers + 1


# --------------------------------------------------------------------------
# Standard decoder pieces (identical in every mode)
# --------------------------------------------------------------------------


class RMSNorm(nn.Module):
    def __init__(self, d: int, eps: float) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x: Tensor) -> Tensor:
        scale = torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + self.eps).to(x.dtype)
        return x * scale * self.weight


def _rope_tables(max_len: int, head_dim: int, theta: float) -> tuple[Tensor, Tensor]:
    freqs = theta ** (-torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim)
    ang = torch.arange(max_len, dtype=torch.float32)[:, None] * freqs[None, :]
    return ang.cos(), ang.sin()


def _rotate(x: Tensor, cos: Tensor, sin: Tensor) -> Tensor:
    """``x: [B, H, T, hd]``; rotation of the two halves in fp32."""
    t = x.shape[-2]
    a, b = x.float().chunk(2, dim=-1)
    c, s = cos[:t], sin[:t]
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1).to(x.dtype)


class CausalSelfAttention(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.n_heads, self.head_dim = cfg.n_heads, cfg.head_dim
        self.q_proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.k_proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.v_proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)
        self.o_proj = nn.Linear(cfg.d_model, cfg.d_model, bias=False)

    def forward(self, x: Tensor, rope: tuple[Tensor, Tensor]) -> Tensor:
        b, t, _ = x.shape

        def heads(y: Tensor) -> Tensor:
            # Contiguous [B, H, T, hd]: attention's math path never sees a
            # transposed operand.
            return y.view(b, t, self.n_heads, self.head_dim).transpose(1, 2).contiguous()

        q = _rotate(heads(self.q_proj(x)), *rope)
        k = _rotate(heads(self.k_proj(x)), *rope)
        v = heads(self.v_proj(x))
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.o_proj(y.transpose(1, 2).reshape(b, t, -1))


class SwiGLU(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.gate_proj = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.up_proj = nn.Linear(cfg.d_model, cfg.d_ff, bias=False)
        self.down_proj = nn.Linear(cfg.d_ff, cfg.d_model, bias=False)

    def forward(self, x: Tensor, rope=None) -> Tensor:
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class Sublayer(nn.Module):
    def __init__(self, norm: RMSNorm, op: nn.Module) -> None:
        super().__init__()
        self.norm = norm
        self.op = op

    def forward(self, x: Tensor, rope) -> Tensor:
        return self.op(self.norm(x), rope)


# --------------------------------------------------------------------------
# The arena
# --------------------------------------------------------------------------


def _alias(arena: Tensor, n_src: int) -> Tensor:
    """``arena[:n_src]`` sharing storage but with its own version counter
    (model.py:325-337)."""
    view = torch.empty(0, dtype=arena.dtype, device=arena.device)
    view.set_(arena.untyped_storage(), arena.storage_offset(), (n_src, *arena.shape[1:]), arena.stride())
    return view


class _ArenaAttnRes(torch.autograd.Function):
    """``impl(arena[:n_src], w)`` whose gradient flows to the live source
    tensors (model.py:340-369). The operator's inner graph is built in forward
    and replayed in backward; only the partial slot is restored first."""

    @staticmethod
    def forward(ctx, w, arena, n_src, has_partial, impl, eps, *sources):
        with torch.enable_grad():
            v = _alias(arena, n_src).requires_grad_(True)
            q = w.detach().requires_grad_(True)
            out = impl(v, q, eps)
        ctx.inner = (v, q, out)
        ctx.arena, ctx.n_src, ctx.has_partial = arena, n_src, has_partial
        ctx.save_for_backward(*((sources[-1],) if has_partial else ()))
        return out.detach()

    @staticmethod
    def backward(ctx, grad_out):
        if ctx.has_partial:
            with torch.no_grad():
                ctx.arena[ctx.n_src - 1].copy_(ctx.saved_tensors[0])
        v, q, out = ctx.inner
        ctx.inner = None
        dv, dw = torch.autograd.grad(out, (v, q), grad_out)
        return (dw, None, None, None, None, None, *(dv[j] for j in range(ctx.n_src)))


# --------------------------------------------------------------------------
# The model
# --------------------------------------------------------------------------


class Transformer(nn.Module):
    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        ops: list[nn.Module] = []
        for _ in range(cfg.n_layers):
            ops += [CausalSelfAttention(cfg), SwiGLU(cfg)]
        self.sublayers = nn.ModuleList(Sublayer(RMSNorm(cfg.d_model, cfg.norm_eps), op) for op in ops)
        # One pseudo-query and gain per sublayer plus the readout site; the
        # modules carry parameters only, the operator comes from _IMPLS.
        self.attn_res = (
            nn.ModuleList(BlockAttnRes(cfg.d_model, eps=cfg.norm_eps) for _ in range(cfg.n_sublayers + 1))
            if cfg.uses_attnres
            else None
        )
        self.final_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        if cfg.tie_embeddings:
            self.lm_head.weight = self.embed.weight
        cos, sin = _rope_tables(cfg.max_seq_len, cfg.head_dim, cfg.rope_theta)
        self.register_buffer("rope_cos", cos, persistent=False)
        self.register_buffer("rope_sin", sin, persistent=False)
        # Only Linear/Embedding draw from the RNG, so every mode built after the
        # same seed shares identical weights (model.py:437-442).
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)):
                nn.init.normal_(mod.weight, mean=0.0, std=0.02)
        depth_scale = 1.0 / math.sqrt(2 * cfg.n_layers)
        with torch.no_grad():
            for sub in self.sublayers:
                proj = sub.op.o_proj if isinstance(sub.op, CausalSelfAttention) else sub.op.down_proj
                proj.weight.mul_(depth_scale)
        self.last_source_counts: list[int] = []
        self.last_alphas: list[Tensor] = []
        self.profile_regions = False

    def param_counts(self) -> dict:
        total = sum(p.numel() for p in self.parameters())
        attnres = sum(p.numel() for m in self.attn_res for p in m.parameters()) if self.attn_res is not None else 0
        return {"total": total, "attnres": attnres, "non_attnres": total - attnres,
                "embedding": self.embed.weight.numel(), "tied_head": self.cfg.tie_embeddings}

    def forward(self, idx: Tensor, targets: Tensor | None = None, collect_alphas: bool = False):
        _, t = idx.shape
        if t > self.cfg.max_seq_len:
            raise ValueError(f"sequence length {t} exceeds max_seq_len {self.cfg.max_seq_len}")
        rope = (self.rope_cos[:t], self.rope_sin[:t])
        x0 = self.embed(idx)
        self.last_alphas = []
        h = self._forward_attnres(x0, rope, collect_alphas) if self.cfg.uses_attnres else self._forward_standard(x0, rope)
        logits = self.lm_head(self.final_norm(h))
        if targets is None:
            return logits
        return logits, F.cross_entropy(logits.float().flatten(0, 1), targets.flatten())

    def _forward_standard(self, x: Tensor, rope) -> Tensor:
        for sub in self.sublayers:
            x = x + sub(x, rope)
        self.last_source_counts = []
        return x

    def _forward_attnres(self, x0: Tensor, rope, collect_alphas: bool) -> Tensor:
        cfg = self.cfg
        b, t, d = x0.shape
        arena = None
        if cfg.sources == "arena":
            # Fresh per forward: a second forward before backward must not
            # overwrite the first one's saved slots.
            arena = torch.empty(cfg.n_blocks + 1, b, t, d, device=x0.device, dtype=x0.dtype)
            with torch.no_grad():
                arena[0].copy_(x0)
        blocks: list[Tensor] = [x0]
        partial: Tensor | None = None
        counts: list[int] = []
        for i, sub in enumerate(self.sublayers):
            if i and i % cfg.block_size == 0:
                blocks.append(partial)  # already sitting in its arena slot
                partial = None
            sources = blocks if partial is None else [*blocks, partial]
            counts.append(len(sources))
            h = self._site(i, arena, sources, partial is not None, collect_alphas)
            y = sub(h, rope)
            partial = y if partial is None else partial + y
            if arena is not None:
                with self._region("attnres_stage"), torch.no_grad():
                    arena[len(blocks)].copy_(partial)
        blocks.append(partial)
        counts.append(len(blocks))
        self.last_source_counts = counts
        return self._site(len(self.sublayers), arena, blocks, False, collect_alphas)

    def _site(self, i: int, arena: Tensor | None, sources: list[Tensor], has_partial: bool,
              collect_alphas: bool) -> Tensor:
        site = self.attn_res[i]
        q = site.effective_query()
        impl = _IMPLS[self.cfg.residual]
        if collect_alphas:
            self.last_alphas.append(_mean_alpha(sources, q, self.cfg.norm_eps))
        if arena is None:
            with self._region("attnres_stage"):
                v = torch.stack(sources, 0)
            with self._region("attnres_op"):
                return impl(v, q, self.cfg.norm_eps)
        with self._region("attnres_op"):
            return _ArenaAttnRes.apply(q, arena, len(sources), has_partial, impl, self.cfg.norm_eps, *sources)

    def _region(self, name: str):
        return torch.profiler.record_function(name) if self.profile_regions else contextlib.nullcontext()


@torch.no_grad()
def _mean_alpha(sources: list[Tensor], q: Tensor, eps: float) -> Tensor:
    """Mean attention weight per source over batch and positions (model.py:571-581)."""
    v = torch.stack(sources, 0).float()
    keys = v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + eps)
    return torch.einsum("d,nbtd->nbt", q.float(), keys).softmax(0).mean(dim=(1, 2))
