"""The Transformer integration (reference tests/test_model.py, restated).

Architecture and framework-mode checks run on the CPU; everything that runs
the HIP operator (``residual="switchyard"``) is marked ``gpu``.
"""

from __future__ import annotations

import pytest
import torch

from switchyard.model import ModelConfig, Transformer, slab_copies, source_count_schedule

HAS_GPU = torch.cuda.is_available()


def _cfg(**kw):
    base = dict(vocab_size=512, d_model=128, n_heads=4, d_ff=256, n_layers=6, n_blocks=3, max_seq_len=64)
    base.update(kw)
    return ModelConfig(**base)


def _build(residual, sources, dev="cpu", seed=0):
    torch.manual_seed(seed)
    return Transformer(_cfg(residual=residual, sources=sources)).to(dev)


def _batch(dev="cpu", b=2, t=32, vocab=512):
    g = torch.Generator().manual_seed(99)
    return (torch.randint(0, vocab, (b, t), generator=g).to(dev),
            torch.randint(0, vocab, (b, t), generator=g).to(dev))


def _grads(m):
    return torch.cat([p.grad.flatten() for _, p in sorted(m.named_parameters())])


# -- architecture (CPU) -----------------------------------------------------


def test_source_count_schedule_matches_equation_6():  # test_model.py:54-64
    got = source_count_schedule(12, 3)
    assert got == [1, 2, 2, 2, 2, 3, 3, 3, 3, 4, 4, 4, 4]
    big = source_count_schedule(48, 8)
    assert len(big) == 49 and sum(big) == 265 and max(big) == 9


def test_model_actually_produces_that_schedule():  # :67-74
    m = _build("attnres", "arena")
    idx, tgt = _batch()
    m(idx, tgt)
    assert m.last_source_counts == source_count_schedule(m.cfg.n_sublayers, m.cfg.n_blocks)


def test_two_attnres_sites_per_transformer_block():  # :77-82
    m = _build("attnres", "arena")
    assert len(m.attn_res) == m.cfg.n_sublayers + 1 == 2 * m.cfg.n_layers + 1


def test_pseudo_queries_are_zero_initialized():  # :85-89
    for site in _build("attnres", "arena").attn_res:
        assert torch.count_nonzero(site.w) == 0


def test_arena_saves_the_stacking_copies():  # :92-99
    assert slab_copies(12, 3, "stack") == sum(source_count_schedule(12, 3))
    assert slab_copies(12, 3, "arena") == 13
    assert slab_copies(48, 8, "stack") == 265 and slab_copies(48, 8, "arena") == 49


def test_attnres_modes_have_identical_parameter_counts():  # :165-172
    counts = {r: sum(p.numel() for p in _build(r, "arena").parameters()) for r in ("attnres", "switchyard")}
    assert counts["attnres"] == counts["switchyard"]


def test_attnres_adds_only_the_parameters_the_paper_says():  # :175-182
    std = sum(p.numel() for p in _build("standard", "arena").parameters())
    att = _build("attnres", "arena")
    assert sum(p.numel() for p in att.parameters()) - std == 2 * att.cfg.d_model * (att.cfg.n_sublayers + 1)


def test_table_sources_need_the_hip_operator():
    with pytest.raises(ValueError, match="table"):
        ModelConfig(residual="attnres", sources="table")
    ModelConfig(residual="switchyard", sources="table")
    assert slab_copies(48, 8, "table") == 0


def test_config_rejects_bad_structure():
    with pytest.raises(ValueError, match="residual"):
        ModelConfig(residual="nope")
    with pytest.raises(ValueError, match="n_blocks"):
        ModelConfig(n_layers=5, n_blocks=4)
    with pytest.raises(ValueError, match="n_heads"):
        ModelConfig(d_model=100, n_heads=16)


def test_arena_and_stack_agree_for_the_framework_operator():  # :107-144
    idx, tgt = _batch()
    outs = {}
    for sources in ("stack", "arena"):
        m = _build("attnres", sources)
        logits, loss = m(idx, tgt)
        loss.backward()
        outs[sources] = (loss, logits, _grads(m))
    torch.testing.assert_close(outs["arena"][0], outs["stack"][0], rtol=0, atol=0)
    torch.testing.assert_close(outs["arena"][1], outs["stack"][1], rtol=0, atol=0)
    ga, gs = outs["arena"][2], outs["stack"][2]
    assert ((ga - gs).norm() / gs.norm()).item() < 1e-6


def test_initial_attention_is_uniform():  # :211-221
    m = _build("attnres", "arena")
    idx, tgt = _batch()
    m(idx, tgt, collect_alphas=True)
    for a in m.last_alphas:
        torch.testing.assert_close(a, torch.full_like(a, 1.0 / a.shape[0]), rtol=1e-4, atol=1e-4)


@pytest.mark.parametrize("residual", ["standard", "attnres"])
def test_framework_modes_overfit_a_fixed_batch(residual):  # :190-208
    torch.manual_seed(0)
    m = Transformer(_cfg(residual=residual, sources="arena"))
    opt = torch.optim.AdamW(m.parameters(), lr=3e-3)
    idx, tgt = _batch()
    first = None
    for _ in range(60):
        opt.zero_grad(set_to_none=True)
        _, loss = m(idx, tgt)
        loss.backward()
        opt.step()
        first = loss.item() if first is None else first
    assert torch.isfinite(loss) and loss.item() < 0.5 * first


def _live(cls):
    import gc

    gc.collect()
    return sum(type(o) is cls for o in gc.get_objects())


def _steps_leave_no_stream(residual, sources, dev):
    """A forward keeps its stream (block tensors, running sums, slot buffer)
    only until its backward has run: anything the backward keeps that points
    back into the autograd graph would form a cycle through autograd's C++
    nodes, invisible to Python's collector, and leak one forward's activations
    per step."""
    from switchyard.model import _SlotBuffer, _Stream

    m = _build(residual, sources, dev)
    idx, tgt = _batch(dev)
    before = (_live(_Stream), _live(_SlotBuffer))
    for _ in range(3):
        m.zero_grad(set_to_none=True)
        m(idx, tgt)[1].backward()  # the logits, kept, would keep the graph
    assert (_live(_Stream), _live(_SlotBuffer)) == before


@pytest.mark.parametrize("sources", ["arena", "stack"])
def test_framework_steps_free_their_stream(sources):
    _steps_leave_no_stream("attnres", sources, "cpu")


# -- the HIP operator inside the model (GPU) --------------------------------


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
@pytest.mark.parametrize("sources", ["arena", "table", "stack"])
def test_hip_steps_free_their_stream_and_device_memory(sources):
    _steps_leave_no_stream("switchyard", sources, "cuda")
    m = _build("switchyard", sources, "cuda")
    idx, tgt = _batch("cuda")

    def step():
        m.zero_grad(set_to_none=True)
        m(idx, tgt)[1].backward()

    step()
    torch.cuda.synchronize()
    base = torch.cuda.memory_allocated()
    for _ in range(3):
        step()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == base


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
@pytest.mark.parametrize("sources", ["arena", "table"])
def test_source_modes_agree_with_stacking_for_the_hip_operator(sources):
    idx, tgt = _batch("cuda")
    outs = {}
    for mode in ("stack", sources):
        m = _build("switchyard", mode, "cuda")
        logits, loss = m(idx, tgt)
        loss.backward()
        outs[mode] = (loss, logits, _grads(m))
    # Same source rows reach the same kernels: bitwise forward.
    torch.testing.assert_close(outs[sources][0], outs["stack"][0], rtol=0, atol=0)
    torch.testing.assert_close(outs[sources][1], outs["stack"][1], rtol=0, atol=0)
    ga, gs = outs[sources][2], outs["stack"][2]
    assert ((ga - gs).norm() / gs.norm()).item() < 1e-6


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
def test_arena_with_more_sources_than_the_table_holds():
    """17 sources at the readout site: the arena's HIP backward restores the
    running-sum slot and takes the stacked path instead of the table."""
    idx, tgt = _batch("cuda", t=16)
    outs = {}
    for mode in ("stack", "arena"):
        torch.manual_seed(0)
        m = Transformer(_cfg(residual="switchyard", sources=mode, n_layers=16, n_blocks=16)).cuda()
        logits, loss = m(idx, tgt)
        loss.backward()
        assert max(m.last_source_counts) == 17
        outs[mode] = (loss, _grads(m))
    torch.testing.assert_close(outs["arena"][0], outs["stack"][0], rtol=0, atol=0)
    ga, gs = outs["arena"][1], outs["stack"][1]
    assert ((ga - gs).norm() / gs.norm()).item() < 1e-6


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
def test_framework_and_fused_modes_agree():  # :147-162
    idx, tgt = _batch("cuda")
    ref = _build("attnres", "arena", "cuda")
    ours = _build("switchyard", "arena", "cuda")
    _, l1 = ref(idx, tgt)
    _, l2 = ours(idx, tgt)
    l1.backward()
    l2.backward()
    torch.testing.assert_close(l2, l1, rtol=1e-5, atol=1e-5)
    g1, g2 = _grads(ref), _grads(ours)
    assert ((g2 - g1).norm() / g1.norm()).item() < 1e-5


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
def test_hip_mode_overfits_a_fixed_batch():
    torch.manual_seed(0)
    m = Transformer(_cfg(residual="switchyard", sources="arena")).cuda()
    opt = torch.optim.AdamW(m.parameters(), lr=3e-3)
    idx, tgt = _batch("cuda")
    first = None
    for _ in range(60):
        opt.zero_grad(set_to_none=True)
        _, loss = m(idx, tgt)
        loss.backward()
        opt.step()
        first = loss.item() if first is None else first
    assert torch.isfinite(loss) and loss.item() < 0.5 * first


@pytest.mark.gpu
@pytest.mark.skipif(not HAS_GPU, reason="needs a HIP device")
def test_bf16_model_step_with_the_hip_operator():
    """One bf16 AdamW step of a mid-size model: HIP mode runs and tracks the
    framework mode's loss."""
    cfg = dict(vocab_size=1024, d_model=512, n_heads=8, d_ff=1408, n_layers=4, n_blocks=4, max_seq_len=256)
    losses = {}
    for residual in ("attnres", "switchyard"):
        torch.manual_seed(0)
        m = Transformer(ModelConfig(**cfg, residual=residual)).cuda().to(torch.bfloat16)
        opt = torch.optim.AdamW(m.parameters(), lr=1e-3)
        idx, tgt = _batch("cuda", b=2, t=256, vocab=1024)
        _, loss = m(idx, tgt)
        loss.backward()
        opt.step()
        losses[residual] = loss.item()
    assert abs(losses["switchyard"] - losses["attnres"]) < 2e-2 * abs(losses["attnres"])
