"""The 1.3B decoder the end-to-end benchmark times, at its real size (GPU).

24 layers, d_model 2048, 16 heads, d_ff 5632, 8 AttnRes blocks, vocab 32000,
bf16 weights, batch 4 x 2048 uniform-random token ids, AdamW. Built on the
device from one seed, so every residual mechanism starts from the same
weights.

* The HIP mechanism tracks the eager framework mechanism through one AdamW
  step: the loss before and after the step and the gradient norm of every
  parameter group agree within bars set by how far two bf16 evaluations of
  the same model drift apart (both are also compared with an fp32 evaluation
  of the framework mechanism, and the HIP mechanism must be no further from
  it than the framework's own bf16 evaluation is, with slack for bf16 noise).
* The three ways of presenting sources (stack, arena, pointer table) give
  bit-identical logits: the same rows reach the same kernel.
"""

from __future__ import annotations

import gc

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from switchyard.model import ModelConfig, Transformer  # noqa: E402

DEV = torch.device("cuda")
SHAPE = dict(vocab_size=32000, d_model=2048, n_layers=24, n_heads=16, d_ff=5632, n_blocks=8,
             max_seq_len=2048)
BATCH, SEQ = 4, 2048


def _build(residual: str, sources: str, dtype=torch.bfloat16) -> Transformer:
    torch.manual_seed(0)
    with DEV:
        m = Transformer(ModelConfig(**SHAPE, residual=residual, sources=sources))
    return m.to(dtype)


def _batch():
    g = torch.Generator().manual_seed(5)
    idx = torch.randint(0, SHAPE["vocab_size"], (BATCH, SEQ), generator=g)
    tgt = torch.randint(0, SHAPE["vocab_size"], (BATCH, SEQ), generator=g)
    return idx.to(DEV), tgt.to(DEV)


def _group(name: str) -> str:
    if name.startswith("attn_res"):
        return "attnres_" + name.rsplit(".", 1)[1]  # w or g
    if name.startswith("embed"):
        return "embedding"
    for key in ("qkv", "attn.out", "gate_up", "mlp.down", "norm"):
        if key in name:
            return key
    return "other"


def _step(residual: str, dtype=torch.bfloat16) -> dict:
    m = _build(residual, "arena", dtype)
    opt = torch.optim.AdamW(m.parameters(), lr=1e-4, weight_decay=0.0)
    idx, tgt = _batch()
    _, loss = m(idx, tgt)
    loss.backward()
    sq: dict[str, float] = {}
    for name, p in m.named_parameters():
        sq[_group(name)] = sq.get(_group(name), 0.0) + p.grad.float().pow(2).sum().item()
    opt.step()
    with torch.no_grad():
        _, after = m(idx, tgt)
    rec = {"loss": loss.item(), "after": after.item(), "norms": {k: v ** 0.5 for k, v in sq.items()}}
    del m, opt
    gc.collect()
    torch.cuda.empty_cache()
    return rec


def test_hip_mechanism_tracks_the_framework_through_an_adamw_step():
    print("config 5: one AdamW step, attnres (bf16, fp32) and switchyard (bf16)", flush=True)
    ref32 = _step("attnres", torch.float32)
    fw = _step("attnres")
    hip = _step("switchyard")
    print(f"  fp32 attnres {ref32}\n  bf16 attnres {fw}\n  bf16 switchyard {hip}", flush=True)
    # Observed on MI355X: losses within 1.3e-4 (relative) of each other and
    # 4e-4 of fp32; group norms within 1.5e-3 of each other and 1.8e-3 of
    # fp32. The bars leave several times that.
    for key in ("loss", "after"):
        assert abs(hip[key] - fw[key]) <= 1e-3 * abs(fw[key]), key
        # no further from the fp32 evaluation than the framework's bf16 is
        assert abs(hip[key] - ref32[key]) <= 2.0 * abs(fw[key] - ref32[key]) + 1e-3 * abs(ref32[key]), key
    assert set(hip["norms"]) == set(fw["norms"])
    for grp, ref in fw["norms"].items():
        got, truth = hip["norms"][grp], ref32["norms"][grp]
        assert abs(got - ref) <= 1e-2 * ref, (grp, got, ref)
        assert abs(got - truth) <= 2.0 * abs(ref - truth) + 5e-3 * truth, (grp, got, ref, truth)


def test_source_modes_give_bit_identical_logits():
    print("config 5: stack / arena / table forward, switchyard", flush=True)
    idx, _ = _batch()
    out = {}
    for sources in ("stack", "arena", "table"):
        m = _build("switchyard", sources)
        with torch.no_grad():
            out[sources] = m(idx)
        del m
        gc.collect()
        torch.cuda.empty_cache()
    assert torch.equal(out["arena"], out["stack"])
    assert torch.equal(out["table"], out["stack"])
