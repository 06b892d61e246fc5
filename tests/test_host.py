"""Host-side behaviour of the Python operator layer (no GPU needed): the
reference's validation messages, the parameter module, the eager comparators
and the byte model the benchmark divides by."""

from __future__ import annotations

import subprocess
import sys

import pytest
import torch

from oracle.reference import block_attn_res_reference
from switchyard import baselines, reference
from switchyard.hip_op import BlockAttnResHIP, block_attn_res_batched, block_attn_res_hip
from switchyard.triton_op import BlockAttnResTriton, block_attn_res_triton

F64 = dict(dtype=torch.float64)


def test_alias_module_exposes_the_reference_names():
    assert block_attn_res_triton is block_attn_res_hip
    assert BlockAttnResTriton is BlockAttnResHIP


@pytest.mark.parametrize("bad", ["rank", "query", "cpu", "empty_n"])
def test_operator_validation_messages(bad):
    """Pinned by the reference's tests (test_triton_op.py:256-268)."""
    v = torch.randn(4, 1, 8, 32)
    w = torch.randn(32)
    if bad == "rank":
        with pytest.raises(ValueError, match=r"\[N, B, T, D\]"):
            block_attn_res_triton(v[0], w)
    elif bad == "query":
        with pytest.raises(ValueError, match="w must be"):
            block_attn_res_triton(v, torch.randn(31))
    elif bad == "cpu":
        with pytest.raises(ValueError, match="CUDA"):
            block_attn_res_triton(v, w)
    else:
        with pytest.raises(ValueError, match=r"\[N, B, T, D\]|CUDA|positive"):
            block_attn_res_triton(v[:0], w)


def test_batched_validation_messages():
    """triton_op.py:463-479."""
    v = torch.randn(4, 1, 8, 32)
    q = torch.randn(3, 32)
    with pytest.raises(ValueError, match=r"\[N, B, T, D\]"):
        block_attn_res_batched(v[0], q)
    with pytest.raises(ValueError, match="queries must be"):
        block_attn_res_batched(v, torch.randn(3, 31))
    with pytest.raises(ValueError, match="CUDA"):
        block_attn_res_batched(v, q)


def test_module_initialises_query_to_zero_and_folds_the_gain():
    m = reference.BlockAttnRes(32)
    assert torch.equal(m.w, torch.zeros(32)) and torch.equal(m.g, torch.ones(32))
    v = torch.randn(4, 1, 3, 32)
    torch.testing.assert_close(m(v), v.mean(0), rtol=1e-6, atol=1e-6)
    h = BlockAttnResHIP(32)
    assert torch.equal(h.w, torch.zeros(32)) and torch.equal(h.g, torch.ones(32))
    assert BlockAttnResHIP(32, norm_affine=False).g is None


def test_rmsnorm_gain_is_redundant_with_the_query():
    """reference.py:61-70: <w, g*v_hat> == <w*g, v_hat> (test_reference.py:204-214)."""
    m = reference.BlockAttnRes(16).double()
    with torch.no_grad():
        m.w.copy_(torch.randn(16, **F64))
        m.g.copy_(torch.randn(16, **F64))
    v = torch.randn(4, 2, 3, 16, **F64)
    torch.testing.assert_close(m(v), block_attn_res_reference(v, m.w * m.g, m.eps))


def test_eager_comparators_match_the_oracle():
    v = torch.randn(5, 2, 3, 24, **F64)
    w = torch.randn(24, **F64) * 0.3
    ref = block_attn_res_reference(v, w)
    for name, fn in baselines.FORMULATIONS.items():
        torch.testing.assert_close(fn(v, w), ref, rtol=1e-12, atol=1e-12, msg=name)
    torch.testing.assert_close(baselines.chunked_form(v, w, chunk=2), ref, rtol=1e-12, atol=1e-12)
    q = torch.randn(3, 24, **F64)
    torch.testing.assert_close(baselines.batched_folded_form(v, q),
                               torch.stack([block_attn_res_reference(v, qi) for qi in q]))


def test_byte_model():
    assert reference.attn_res_min_bytes(9, 1, 4096, 2048) == 167_772_160
    assert reference.attn_res_train_bytes(9, 1, 4096, 2048) == 486_539_264
    assert reference.attn_res_batched_bytes(9, 8, 1, 4096, 2048) == 285_245_440
    assert reference.arithmetic_intensity(9, 1, 1, 1) == pytest.approx(54 / 20)
    assert reference.ridge_point(10.0, 4.0) == 2.5
    assert reference.DEFAULT_EPS == 1e-6


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                       cwd=str(__import__("pathlib").Path(__file__).resolve().parents[1]), timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
