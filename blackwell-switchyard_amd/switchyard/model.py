"""Decoder-only Transformer whose residual stream can be Block AttnRes.

This is the operator's training caller (the reference's ``switchyard.model``,
src/switchyard/model.py of sabdulmajid/blackwell-switchyard): the same public
names (``ModelConfig``, ``Transformer``, ``source_count_schedule``,
``slab_copies``), the same three residual mechanisms and the same wiring of
the paper's Eq. 6, so that the step-time comparison between mechanisms means
the same thing here.

Residual mechanisms (``ModelConfig.residual``):
  ``standard``    PreNorm, ``x <- x + f(norm(x))``: the control.
  ``attnres``     Block AttnRes evaluated by the eager ``folded_form``.
  ``switchyard``  Block AttnRes evaluated by the HIP operator.

Wiring. A "layer" of the paper is a sublayer here (attention or MLP, each
behind its own RMSNorm), and the ``2 * n_layers`` sublayers are cut into
``n_blocks`` equal blocks. The stream keeps the completed block
representations (the embedding first) and the running, unweighted sum of the
current block's sublayer outputs. Each sublayer reads ``AttnRes`` over the
completed blocks plus the running sum (absent for the first sublayer of a
block) and adds its output to the running sum; when a block ends, its running
sum becomes its representation. A final site over every completed block feeds
the LM head. Each site owns a pseudo-query and an RMSNorm gain, both of width
``d_model`` (2 * d_model parameters a site).

How a site's sources reach the operator (``ModelConfig.sources``):
  ``stack``  ``torch.stack`` of the live tensors at every site: N slab copies
             per site (the paper's pseudocode).
  ``arena``  one ``[n_blocks + 1, B, T, D]`` buffer per forward. The
             embedding is copied into slot 0 and each new running sum into the
             slot of the block being built, so a site's sources are always the
             buffer's first N slots, read in place: one slab copy per sublayer.
  ``table``  (HIP operator only) the site passes the live tensors' addresses
             to the pointer-table entry points; nothing is copied. At most 16
             sources per site (the table size); wider sites stack.

Autograd over the arena. The running-sum slot is overwritten by every later
sublayer of its block while earlier sites still need, for their backward, the
value they read. Two mechanisms handle that:
  * HIP sites call the C ABI themselves. The forward reads the buffer prefix
    through its source stride; the backward addresses the completed-block
    slots in the buffer (each written once, when its block ended, and never
    again) and the site's running sum through the tensor itself, with the
    pointer-table backward -- so no slot is ever restored or copied back.
  * Eager sites hand ``folded_form`` a view of the prefix. Every tensor that
    autograd saves out of the buffer passes through a saved-tensor hook whose
    unpack puts the site's running sum back into its slot before handing the
    view over. The backward of a site runs only after every later site that
    reads the slot has finished its own (each later site depends on this
    site's output through the running sum), so the restored value is never
    needed elsewhere. Saved-tensor hooks also bypass autograd's storage-wide
    version check, which the slot writes would otherwise trip.
"""

from __future__ import annotations

import contextlib
import math
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
SOURCE_MODES = ("arena", "stack", "table")


# --------------------------------------------------------------------------
# Configuration and the Eq. 6 bookkeeping
# --------------------------------------------------------------------------


@dataclass
class ModelConfig:
    """Model shape and residual mechanism (field names and meaning as the
    reference's ``ModelConfig``, model.py:151-202). Defaults: the 1.3B
    benchmark decoder -- 24 layers, d_model 2048, 16 heads, d_ff 5632, 8
    blocks, vocab 32000 (the reference used 32768)."""

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
        problems = []
        if self.residual not in RESIDUAL_MODES:
            problems.append(f"residual must be one of {RESIDUAL_MODES}, got {self.residual!r}")
        if self.sources not in SOURCE_MODES:
            problems.append(f"sources must be one of {SOURCE_MODES}, got {self.sources!r}")
        elif self.sources == "table" and self.residual == "attnres":
            problems.append("sources='table' passes device pointers to the HIP operator; "
                            "the eager 'attnres' mechanism needs 'arena' or 'stack'")
        if self.d_model % self.n_heads != 0:
            problems.append(f"d_model {self.d_model} is not a multiple of n_heads {self.n_heads}")
        if (2 * self.n_layers) % self.n_blocks != 0:
            problems.append(f"n_blocks {self.n_blocks} does not divide the {2 * self.n_layers} "
                            "sublayers (2 * n_layers) into whole blocks")
        if problems:
            raise ValueError("; ".join(problems))

    @property
    def n_sublayers(self) -> int:
        """Attention and MLP of every layer: the paper's "layers"."""
        return 2 * self.n_layers

    @property
    def block_size(self) -> int:
        return self.n_sublayers // self.n_blocks

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads

    @property
    def uses_attnres(self) -> bool:
        return self.residual in ("attnres", "switchyard")


def source_count_schedule(n_sublayers: int, n_blocks: int) -> list[int]:
    """Source count of every AttnRes site in order (paper Eq. 6; the reference
    states it at model.py:205-219): in block ``j`` the opening sublayer sees
    the embedding and the ``j`` completed blocks, every other sublayer also the
    running sum; the readout site sees all ``n_blocks + 1`` representations."""
    size = n_sublayers // n_blocks
    counts: list[int] = []
    for j in range(n_blocks):
        counts += [j + 1] + [j + 2] * (size - 1)
    return counts + [n_blocks + 1]


def slab_copies(n_sublayers: int, n_blocks: int, sources: str) -> int:
    """``B*T*D`` slabs copied to present the sources over one forward
    (model.py:222-235): ``stack`` copies every source at every site, ``arena``
    the embedding once plus one running sum per sublayer, ``table`` nothing."""
    if sources == "stack":
        return sum(source_count_schedule(n_sublayers, n_blocks))
    if sources == "arena":
        return n_sublayers + 1
    if sources == "table":
        return 0
    raise ValueError(f"unknown source mode {sources!r}")


# --------------------------------------------------------------------------
# Decoder blocks (the same in every residual mode)
# --------------------------------------------------------------------------


class RMSNorm(nn.Module):
    """``x / rms(x) * weight``, the statistic in fp32."""

    def __init__(self, d: int, eps: float) -> None:
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))

    def forward(self, x: Tensor) -> Tensor:
        inv = x.float().square().mean(dim=-1, keepdim=True).add(self.eps).rsqrt()
        return x * inv.to(x.dtype) * self.weight


class Rotary(nn.Module):
    """Rotary position embedding on ``[B, T, H, hd]``: channel ``i`` of the
    first half turns with channel ``i`` of the second half by ``t * theta^(-2i/hd)``."""

    def __init__(self, head_dim: int, max_len: int, theta: float) -> None:
        super().__init__()
        half = head_dim // 2
        inv_freq = torch.pow(theta, -torch.arange(half, dtype=torch.float32) * 2.0 / head_dim)
        phase = torch.arange(max_len, dtype=torch.float32)[:, None] * inv_freq[None, :]
        self.register_buffer("cos", phase.cos()[:, None, :], persistent=False)  # [T, 1, half]
        self.register_buffer("sin", phase.sin()[:, None, :], persistent=False)

    def forward(self, x: Tensor) -> Tensor:
        t = x.shape[1]
        c, s = self.cos[:t], self.sin[:t]
        lo, hi = x.float().chunk(2, dim=-1)
        return torch.cat((lo * c - hi * s, lo * s + hi * c), dim=-1).to(x.dtype)


class Attention(nn.Module):
    """Causal multi-head attention: one fused QKV projection (one GEMM),
    rotary positions, ``scaled_dot_product_attention`` on contiguous
    ``[B, H, T, hd]`` operands, and the output projection."""

    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.heads, self.hd = cfg.n_heads, cfg.head_dim
        self.qkv = nn.Linear(cfg.d_model, 3 * cfg.d_model, bias=False)
        self.out = nn.Linear(cfg.d_model, cfg.d_model, bias=False)

    def forward(self, x: Tensor, rotary: Rotary) -> Tensor:
        b, t, d = x.shape
        q, k, v = self.qkv(x).view(b, t, 3, self.heads, self.hd).unbind(2)
        q, k = rotary(q), rotary(k)
        q, k, v = (y.transpose(1, 2).contiguous() for y in (q, k, v))
        y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
        return self.out(y.transpose(1, 2).reshape(b, t, d))


class GatedMLP(nn.Module):
    """SwiGLU: ``down(silu(gate x) * (up x))`` with gate and up as one GEMM."""

    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.gate_up = nn.Linear(cfg.d_model, 2 * cfg.d_ff, bias=False)
        self.down = nn.Linear(cfg.d_ff, cfg.d_model, bias=False)

    def forward(self, x: Tensor, rotary: Rotary | None = None) -> Tensor:
        gate, up = self.gate_up(x).chunk(2, dim=-1)
        return self.down(F.silu(gate) * up)


class DecoderLayer(nn.Module):
    """Two sublayers, each a pre-norm and a transform: attention, then MLP."""

    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.attn_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.attn = Attention(cfg)
        self.mlp_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.mlp = GatedMLP(cfg)

    def sublayers(self):
        yield self.attn_norm, self.attn
        yield self.mlp_norm, self.mlp


# --------------------------------------------------------------------------
# Source staging
# --------------------------------------------------------------------------


class _SlotBuffer:
    """The arena of one forward: ``[n_blocks + 1, B, T, D]`` slots and, per
    slot, the running-sum value it carries now. Everything the backward keeps
    (HIP sites hold the buffer, saved-tensor hooks the buffer and a value)
    lives here, and none of it belongs to the autograd graph: the values are
    detached aliases and the buffer is written under ``no_grad``. A reference
    from saved state back into the graph would close a cycle through
    autograd's C++ nodes, which Python's garbage collector cannot see, and
    leak every forward's activations."""

    def __init__(self, x0: Tensor, n_blocks: int) -> None:
        self.slots = x0.new_empty((n_blocks + 1, *x0.shape))
        self.holds: dict[int, Tensor] = {}
        self.write(0, x0.detach())

    def write(self, k: int, value: Tensor) -> None:
        with torch.no_grad():
            self.slots[k].copy_(value)
        self.holds[k] = value

    def restore(self, k: int, value: Tensor) -> None:
        if self.holds.get(k) is not value:
            self.write(k, value)


class _Stream:
    """The residual stream of one AttnRes forward: completed block
    representations, the running sum of the current block, and (arena mode)
    the slot buffer that mirrors them, with ``running_alias`` the detached
    alias the buffer's running slot was written from."""

    def __init__(self, x0: Tensor, n_blocks: int, arena: bool) -> None:
        self.blocks: list[Tensor] = [x0]
        self.running: Tensor | None = None
        self.running_alias: Tensor | None = None
        self.buf = _SlotBuffer(x0, n_blocks) if arena else None

    def sources(self) -> list[Tensor]:
        return self.blocks if self.running is None else [*self.blocks, self.running]

    def accumulate(self, y: Tensor, region=contextlib.nullcontext) -> None:
        """Add a sublayer output to the running sum; in arena mode also copy
        the new sum into its slot (the staging cost, inside ``region``)."""
        self.running = y if self.running is None else self.running + y
        if self.buf is not None:
            self.running_alias = self.running.detach()
            with region():
                self.buf.write(len(self.blocks), self.running_alias)

    def close_block(self) -> None:
        self.blocks.append(self.running)
        self.running = self.running_alias = None

    def saving(self):
        """Hooks under which an eager site may save views of the buffer: a
        saved view is kept detached, with the value its running slot held,
        and the slot is restored before the view is handed back."""
        buf, slot, value = self.buf, len(self.blocks), self.running_alias
        storage = buf.slots.untyped_storage().data_ptr()

        def pack(t: Tensor):
            if value is not None and t.untyped_storage().data_ptr() == storage:
                return (_BufferView, t.detach(), slot, value)
            return t

        def unpack(x):
            if isinstance(x, tuple) and x and x[0] is _BufferView:
                _, t, k, v = x
                buf.restore(k, v)
                return t
            return x

        return torch.autograd.graph.saved_tensors_hooks(pack, unpack)


class _BufferView(torch.autograd.Function):
    """``slots[:n]`` as a differentiable function of the ``n`` live sources,
    with no copy: the forward returns the prefix view, the backward hands each
    source its slice of the gradient."""

    @staticmethod
    def forward(ctx, slots: Tensor, n: int, *sources: Tensor) -> Tensor:
        return slots[:n]

    @staticmethod
    def backward(ctx, grad: Tensor):
        return (None, None, *grad.unbind(0))


class _SlotSiteHIP(torch.autograd.Function):
    """One HIP site over the slot buffer. Forward: ``sy_fwd`` on the prefix
    (source stride = one slot). Backward: ``sy_bwd_table`` with the
    completed-block slots and the site's running-sum tensor as rows, and each
    source's gradient as its own dv row."""

    @staticmethod
    def forward(ctx, q: Tensor, stream: _Stream, n: int, eps: float, *sources: Tensor) -> Tensor:
        from . import _lib
        from .hip_op import _ptr

        slots = stream.buf.slots
        _, b, t, d = slots.shape
        n_tok = b * t
        q = q.contiguous()
        out = slots.new_empty((b, t, d))
        stats = torch.empty(2, n, n_tok, device=slots.device, dtype=torch.float32)
        with torch.cuda.device(slots.device):
            rc = _lib.lib().sy_fwd(_ptr(slots), _ptr(q), _ptr(out), _ptr(stats), n, n_tok, d, n_tok * d,
                                   _lib.dtype_code(slots.dtype), _lib.dtype_code(q.dtype), float(eps),
                                   _lib.stream_ptr(slots.device))
        _lib.check(rc, "sy_fwd")
        running = stream.running
        # The buffer, not the stream: the stream holds graph tensors.
        ctx.buf, ctx.n, ctx.eps = stream.buf, n, float(eps)
        ctx.n_fixed = n - (1 if running is not None else 0)
        ctx.save_for_backward(q, stats, *((running,) if running is not None else ()))
        return out

    @staticmethod
    def backward(ctx, grad_out: Tensor):
        from . import _lib
        from .hip_op import _ptr

        q, stats, *running = ctx.saved_tensors
        buf, n = ctx.buf, ctx.n
        slots = buf.slots
        _, b, t, d = slots.shape
        n_tok = b * t
        dev, dt = slots.device, slots.dtype
        grad_out = grad_out.to(dt).contiguous()
        dv = torch.empty(n, b, t, d, device=dev, dtype=dt)
        dq = torch.empty(d, device=dev, dtype=q.dtype)
        lib = _lib.lib()
        vt, wt = _lib.dtype_code(dt), _lib.dtype_code(q.dtype)
        with torch.cuda.device(dev):
            ws_bytes = lib.sy_bwd_workspace_bytes(n, n_tok, d, vt, wt)
            if ws_bytes < 0:
                _lib.check(int(ws_bytes), "sy_bwd_workspace_bytes")
            ws = torch.empty(max(1, (ws_bytes + 3) // 4), device=dev, dtype=torch.float32)
            st = _lib.stream_ptr(dev)
            if n <= _lib.MAX_TABLE_ROWS:
                rows = [slots[j] for j in range(ctx.n_fixed)] + running
                rc = lib.sy_bwd_table(_lib.pointer_table(rows), _ptr(q), _ptr(grad_out), _ptr(stats),
                                      _lib.pointer_table(dv.unbind(0)), _ptr(dq), _ptr(ws), ws.numel() * 4,
                                      n, n_tok, d, vt, wt, ctx.eps, st)
                what = "sy_bwd_table"
            else:
                if running:
                    buf.restore(n - 1, running[0].detach())
                rc = lib.sy_bwd(_ptr(slots), _ptr(q), _ptr(grad_out), _ptr(stats), _ptr(dv), _ptr(dq),
                                _ptr(ws), ws.numel() * 4, n, n_tok, d, n_tok * d, vt, wt, ctx.eps, st)
                what = "sy_bwd"
        _lib.check(rc, what)
        return (dq, None, None, None, *dv.unbind(0))


def _hip_stacked(v: Tensor, q: Tensor, eps: float) -> Tensor:
    from .hip_op import block_attn_res_hip

    return block_attn_res_hip(v, q, eps)


def _hip_table(sources: list[Tensor], q: Tensor, eps: float) -> Tensor:
    from .table_op import MAX_SOURCES, block_attn_res_sources

    if len(sources) > MAX_SOURCES:
        return _hip_stacked(torch.stack(sources), q, eps)
    return block_attn_res_sources(sources, q, eps)


# --------------------------------------------------------------------------
# The model
# --------------------------------------------------------------------------


class Transformer(nn.Module):
    """Decoder-only LM: embedding, ``n_layers`` decoder layers, final norm,
    LM head (tied to the embedding by default). With an AttnRes mechanism,
    ``attn_res[i]`` holds the pseudo-query and gain of site ``i``
    (``n_sublayers`` sites plus the readout)."""

    def __init__(self, cfg: ModelConfig) -> None:
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.layers = nn.ModuleList(DecoderLayer(cfg) for _ in range(cfg.n_layers))
        self.attn_res = (nn.ModuleList(BlockAttnRes(cfg.d_model, eps=cfg.norm_eps)
                                       for _ in range(cfg.n_sublayers + 1))
                         if cfg.uses_attnres else None)
        self.final_norm = RMSNorm(cfg.d_model, cfg.norm_eps)
        self.lm_head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)
        if cfg.tie_embeddings:
            self.lm_head.weight = self.embed.weight
        self.rotary = Rotary(cfg.head_dim, cfg.max_seq_len, cfg.rope_theta)
        self._init_parameters()
        self.last_source_counts: list[int] = []
        self.last_alphas: list[Tensor] = []
        #: Wrap staging and operator calls in profiler regions
        #: (``attnres_stage``, ``attnres_op``) for attribution runs.
        self.profile_regions = False

    def _init_parameters(self) -> None:
        # N(0, 0.02) for every projection and the embedding, in module order;
        # the AttnRes parameters (zeros, ones) draw nothing from the RNG, so a
        # seed gives every residual mechanism the same shared weights. The
        # projections that write into the residual stream are scaled by
        # 1/sqrt(2 n_layers).
        seen = set()
        for mod in self.modules():
            if isinstance(mod, (nn.Linear, nn.Embedding)) and id(mod.weight) not in seen:
                seen.add(id(mod.weight))
                nn.init.normal_(mod.weight, mean=0.0, std=0.02)
        with torch.no_grad():
            for layer in self.layers:
                for proj in (layer.attn.out, layer.mlp.down):
                    proj.weight.mul_(1.0 / math.sqrt(2 * self.cfg.n_layers))

    def param_counts(self) -> dict:
        total = sum(p.numel() for p in self.parameters())
        own = sum(p.numel() for p in self.attn_res.parameters()) if self.attn_res is not None else 0
        return {"total": total, "attnres": own, "non_attnres": total - own,
                "embedding": self.embed.weight.numel(), "tied_head": self.cfg.tie_embeddings}

    def _sublayers(self):
        for layer in self.layers:
            yield from layer.sublayers()

    def forward(self, idx: Tensor, targets: Tensor | None = None, collect_alphas: bool = False):
        """``idx [B, T]`` -> logits ``[B, T, V]``, or ``(logits, loss)`` with
        ``targets``. ``collect_alphas`` records each site's mean attention
        weight per source in ``last_alphas`` (a diagnostic; it costs time)."""
        if idx.shape[1] > self.cfg.max_seq_len:
            raise ValueError(f"sequence length {idx.shape[1]} exceeds max_seq_len {self.cfg.max_seq_len}")
        x = self.embed(idx)
        self.last_alphas = []
        if self.cfg.uses_attnres:
            h = self._attnres_stream(x, collect_alphas)
        else:
            for norm, fn in self._sublayers():
                x = x + fn(norm(x), self.rotary)
            self.last_source_counts = []
            h = x
        logits = self.lm_head(self.final_norm(h))
        if targets is None:
            return logits
        return logits, F.cross_entropy(logits.float().flatten(0, 1), targets.flatten())

    def _attnres_stream(self, x0: Tensor, collect_alphas: bool) -> Tensor:
        cfg = self.cfg
        with self._region("attnres_stage"):
            stream = _Stream(x0, cfg.n_blocks, arena=cfg.sources == "arena")
        counts = []
        for i, (norm, fn) in enumerate(self._sublayers()):
            if i > 0 and i % cfg.block_size == 0:
                stream.close_block()
            h = self._site(i, stream, collect_alphas)
            counts.append(len(stream.sources()))
            y = fn(norm(h), self.rotary)
            stream.accumulate(y, lambda: self._region("attnres_stage"))
        stream.close_block()
        counts.append(len(stream.sources()))
        self.last_source_counts = counts
        return self._site(cfg.n_sublayers, stream, collect_alphas)

    def _site(self, i: int, stream: _Stream, collect_alphas: bool) -> Tensor:
        cfg = self.cfg
        q = self.attn_res[i].effective_query()
        sources = stream.sources()
        n = len(sources)
        if collect_alphas:
            self.last_alphas.append(_mean_alpha(sources, q, cfg.norm_eps))
        hip = cfg.residual == "switchyard"
        if cfg.sources == "stack":
            with self._region("attnres_stage"):
                v = torch.stack(sources)
            with self._region("attnres_op"):
                return _hip_stacked(v, q, cfg.norm_eps) if hip else folded_form(v, q, cfg.norm_eps)
        if cfg.sources == "table":
            with self._region("attnres_op"):
                return _hip_table(sources, q, cfg.norm_eps)
        with self._region("attnres_op"):
            if hip:
                return _SlotSiteHIP.apply(q, stream, n, cfg.norm_eps, *sources)
            with stream.saving():
                return folded_form(_BufferView.apply(stream.buf.slots, n, *sources), q, cfg.norm_eps)

    def _region(self, name: str):
        return torch.profiler.record_function(name) if self.profile_regions else contextlib.nullcontext()


@torch.no_grad()
def _mean_alpha(sources: list[Tensor], q: Tensor, eps: float) -> Tensor:
    """Mean softmax weight of each source over batch and positions, in fp32
    (the reference's diagnostic, model.py:571-581)."""
    logits = torch.stack([
        (s.float() @ q.float()) * s.float().square().mean(-1).add(eps).rsqrt() for s in sources
    ])
    return logits.softmax(0).mean(dim=(1, 2))
