"""Pins the CPU oracle (oracle/) before anything is checked against it.

The reference commits no golden vectors, so the oracle is pinned by:
  1. every semantic property of the reference's tests/test_reference.py,
     restated on oracle.reference (float64);
  2. hand-derived closed forms (a two-source antipodal case whose output is a
     tanh, and an axis-aligned case computed with `math`);
  3. the backward derivation (C closed form) against torch.autograd of the
     paper form, central differences and gradcheck/gradgradcheck;
  4. agreement of the two independent restatements (C loops vs torch einsum);
  5. the committed fixtures (tests/golden/attnres_golden.npz).
Section 6 plants plausible mistakes in copies of the oracle (1/sqrt(D)
scaling, normalised values in the sum, softmax over the wrong axis, sum
instead of mean, a sign flip or a dropped term in the backward) and shows each
one fails at least one pin, so the pins have teeth.
"""

from __future__ import annotations

import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import c_oracle
from oracle.reference import (
    DEFAULT_EPS,
    arithmetic_intensity,
    attn_res_flops,
    attn_res_min_bytes,
    attn_with_stats,
    batched_folded_form,
    block_attn_res_oracle,
    block_attn_res_reference,
    check_against,
    dtype_floor,
    folded_form,
    merge_online_softmax,
    oracle_grads,
    paper_form,
    rel_l2,
    rms_norm,
)

F64 = dict(dtype=torch.float64)
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "attnres_golden.npz"


def _inputs(n=5, b=2, t=7, d=16, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, b, t, d, generator=g, **F64)
    w = torch.randn(d, generator=g, **F64)
    return v, w / w.norm() * scale


# --------------------------------------------------------------------------
# 1. Semantics (reference tests/test_reference.py, restated)
# --------------------------------------------------------------------------


def test_rms_norm_matches_torch():  # test_reference.py:34-39
    x = torch.randn(3, 4, 32, **F64)
    torch.testing.assert_close(rms_norm(x), torch.nn.functional.rms_norm(x, (32,), None, DEFAULT_EPS),
                               rtol=1e-12, atol=1e-12)


def test_zero_query_gives_uniform_average():  # :42-48
    v, _ = _inputs()
    torch.testing.assert_close(block_attn_res_reference(v, torch.zeros(v.shape[-1], **F64)), v.mean(0))


def test_single_source_is_identity():  # :51-53
    v, w = _inputs(n=1)
    torch.testing.assert_close(block_attn_res_reference(v, w), v[0])


def test_output_is_convex_combination():  # :56-63
    v, w = _inputs(scale=3.0)
    out = block_attn_res_reference(v, w)
    assert (out <= v.amax(0) + 1e-12).all() and (out >= v.amin(0) - 1e-12).all()


def test_weighted_sum_uses_raw_not_normalized_sources():  # :66-78
    v, w = _inputs()
    v2 = v.clone()
    v2[0] *= 50.0
    assert (block_attn_res_reference(v, w) - block_attn_res_reference(v2, w)).abs().max() > 1.0


def test_normalization_makes_scores_scale_invariant():  # :81-109
    v, w = _inputs()
    v2 = v.clone()
    v2[1] *= 100.0
    torch.testing.assert_close(rms_norm(v)[1], rms_norm(v2)[1], rtol=1e-5, atol=1e-5)
    a1 = torch.einsum("d,nbtd->nbt", w, rms_norm(v)).softmax(0)
    a2 = torch.einsum("d,nbtd->nbt", w, rms_norm(v2)).softmax(0)
    torch.testing.assert_close(a1, a2, rtol=1e-4, atol=1e-4)
    b1 = torch.einsum("d,nbtd->nbt", w, v).softmax(0)
    b2 = torch.einsum("d,nbtd->nbt", w, v2).softmax(0)
    assert (b1 - b2).abs().max() > 0.5


def test_softmax_axis_is_depth_not_sequence():  # :112-122
    v, w = _inputs()
    v2 = v.clone()
    v2[:, 0, 3, :] += 10.0
    changed = (block_attn_res_reference(v, w) - block_attn_res_reference(v2, w)).abs().sum(-1) > 1e-9
    assert changed[0, 3] and changed.sum() == 1


def test_no_sqrt_d_scaling():  # :125-136
    v, w = _inputs(n=2, b=1, t=1, d=8)
    expected = torch.einsum("d,nbtd->nbt", w, rms_norm(v)).softmax(0)
    implied = torch.linalg.lstsq(v[:, 0, 0, :].T, block_attn_res_reference(v, w)[0, 0]).solution
    torch.testing.assert_close(implied, expected[:, 0, 0], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("split", [1, 2, 4])
def test_two_phase_online_softmax_merge_is_exact(split):  # :139-150
    v, w = _inputs(n=8)
    o1, m1, l1 = attn_with_stats(v[:split], w)
    o2, m2, l2 = attn_with_stats(v[split:], w)
    o, _, ell = merge_online_softmax(o1, m1, l1, o2, m2, l2)
    torch.testing.assert_close(o / ell.unsqueeze(-1), block_attn_res_reference(v, w), rtol=1e-12, atol=1e-12)


def test_merge_survives_extreme_logit_separation():  # :153-162
    v, w = _inputs(n=6, scale=200.0)
    o1, m1, l1 = attn_with_stats(v[:3], w)
    o2, m2, l2 = attn_with_stats(v[3:], w)
    o, _, ell = merge_online_softmax(o1, m1, l1, o2, m2, l2)
    got = o / ell.unsqueeze(-1)
    assert torch.isfinite(got).all()
    torch.testing.assert_close(got, block_attn_res_reference(v, w), rtol=1e-9, atol=1e-9)


def test_gradients_match_numerical_jacobian():  # :165-173
    g = torch.Generator().manual_seed(0)
    v = torch.randn(4, 1, 3, 6, generator=g, **F64).requires_grad_(True)
    w = torch.randn(6, generator=g, **F64).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: block_attn_res_reference(a, b), (v, w), eps=1e-6,
                                    atol=1e-8, rtol=1e-6)


def test_second_order_gradients():  # :176-185
    g = torch.Generator().manual_seed(0)
    v = torch.randn(3, 1, 2, 5, generator=g, **F64).requires_grad_(True)
    w = torch.randn(5, generator=g, **F64).requires_grad_(True)
    assert torch.autograd.gradgradcheck(lambda a, b: block_attn_res_reference(a, b), (v, w),
                                        atol=1e-6, rtol=1e-5)


def test_batched_folded_form_matches_individual_queries():  # :196-201
    v, _ = _inputs(n=5, b=2, t=3, d=16)
    q = torch.randn(4, 16, **F64)
    torch.testing.assert_close(batched_folded_form(v, q),
                               torch.stack([block_attn_res_reference(v, qi) for qi in q]),
                               rtol=1e-12, atol=1e-12)


def test_eager_forms_agree_with_the_oracle():
    v, w = _inputs(n=6, b=2, t=5, d=48, scale=2.0)
    ref = block_attn_res_reference(v, w)
    torch.testing.assert_close(paper_form(v, w), ref, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(folded_form(v, w), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("shape", [(1, 1, 1, 1), (2, 1, 1, 3), (17, 1, 2, 63), (3, 4, 5, 129)])
def test_odd_shapes(shape):  # :217-222
    v, w = _inputs(*shape)
    out = block_attn_res_reference(v, w)
    assert out.shape == shape[1:] and torch.isfinite(out).all()


def test_rejections():  # :225-232
    with pytest.raises(ValueError, match=r"\[N, B, T, D\]"):
        block_attn_res_reference(torch.randn(3, 4), torch.randn(4))
    with pytest.raises(ValueError, match="D="):
        block_attn_res_reference(torch.randn(2, 1, 3, 8), torch.randn(7))


def test_byte_and_flop_model():  # reference.py:295 and :236-255
    assert math.isclose(arithmetic_intensity(9, 1, 1, 1), 6 * 9 / (10 * 2))
    assert attn_res_min_bytes(9, 1, 4096, 2048) == 167_772_160
    assert attn_res_flops(9, 1, 4096, 2048) == 452_984_832


def test_metric_reports_the_dtype_floor():
    o = torch.randn(64, **F64)
    rep = check_against(o.to(torch.bfloat16), o, rel_l2_tol=1e-2)
    assert rep["ok"] and math.isclose(rep["err_vs_dtype_floor"], 1.0, rel_tol=1e-12)
    assert math.isclose(rel_l2(o, o), 0.0) and dtype_floor(o, torch.float64) == 0.0


# --------------------------------------------------------------------------
# 2. Hand-derived closed forms
# --------------------------------------------------------------------------


def _antipodal_expected(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """Sources v0 = x, v1 = -x share r = (mean(x^2) + eps)^-1/2, logits are
    +-r<w, x>, so alpha0 - alpha1 = tanh(r<w, x>) and out = tanh(r<w, x>) x."""
    r = 1.0 / math.sqrt(float(np.mean(x * x)) + eps)
    return math.tanh(r * float(w @ x)) * x


def test_closed_form_antipodal_sources():
    rng = np.random.default_rng(7)
    for d in (3, 16, 255):
        x = rng.standard_normal(d)
        w = rng.standard_normal(d) * 0.3
        v = np.stack([x, -x])[:, None, :]  # [N=2, T=1, D]
        want = _antipodal_expected(x, w, DEFAULT_EPS)
        np.testing.assert_allclose(c_oracle.forward(v, w)[0], want, rtol=1e-12, atol=1e-13)
        vt = torch.from_numpy(v)[:, None]  # [2, 1, 1, D]
        np.testing.assert_allclose(block_attn_res_reference(vt, torch.from_numpy(w))[0, 0].numpy(), want,
                                   rtol=1e-12, atol=1e-13)


def test_closed_form_axis_aligned_sources():
    """v0 = (2,0,0,0), v1 = (0,3,0,0), w = (a,b,0,0): mean-square 1 and 9/4,
    so logits are 2a/sqrt(1+eps) and 3b/sqrt(9/4+eps) -- a sum instead of a
    mean, or a 1/sqrt(D), changes them."""
    a, b = 0.7, -0.4
    eps = DEFAULT_EPS
    l0 = 2 * a / math.sqrt(1.0 + eps)
    l1 = 3 * b / math.sqrt(2.25 + eps)
    m = max(l0, l1)
    e0, e1 = math.exp(l0 - m), math.exp(l1 - m)
    want = np.array([2 * e0 / (e0 + e1), 3 * e1 / (e0 + e1), 0.0, 0.0])
    v = np.array([[[2.0, 0, 0, 0]], [[0, 3.0, 0, 0]]])
    w = np.array([a, b, 0.0, 0.0])
    np.testing.assert_allclose(c_oracle.forward(v, w)[0], want, rtol=1e-14, atol=1e-15)
    np.testing.assert_allclose(
        block_attn_res_reference(torch.from_numpy(v)[:, None], torch.from_numpy(w))[0, 0].numpy(), want,
        rtol=1e-14, atol=1e-15)


def test_closed_form_gradient_of_antipodal_case():
    """d out/d w for the antipodal case: out = tanh(r<w,x>) x, so
    <g, d out/d w> = (1 - tanh^2) r <g, x> x."""
    rng = np.random.default_rng(11)
    d = 12
    x = rng.standard_normal(d)
    w = rng.standard_normal(d) * 0.3
    g = rng.standard_normal(d)
    r = 1.0 / math.sqrt(float(np.mean(x * x)) + DEFAULT_EPS)
    th = math.tanh(r * float(w @ x))
    want_dw = (1 - th * th) * r * float(g @ x) * x
    _, dw = c_oracle.backward(np.stack([x, -x])[:, None, :], w, g[None, :])
    np.testing.assert_allclose(dw, want_dw, rtol=1e-12, atol=1e-13)


# --------------------------------------------------------------------------
# 3. Backward: closed form vs autograd and central differences
# --------------------------------------------------------------------------


@pytest.mark.parametrize("shape,scale", [((4, 1, 3, 16), 1.0), ((9, 2, 4, 33), 3.0), ((1, 1, 5, 8), 1.0)])
def test_c_backward_matches_autograd(shape, scale):
    v, w = _inputs(*shape, seed=3, scale=scale)
    g = torch.randn(shape[1], shape[2], shape[3], generator=torch.Generator().manual_seed(4), **F64)
    dv64, dw64 = oracle_grads(v, w, g)
    n, b, t, d = shape
    dv, dw = c_oracle.backward(v.reshape(n, b * t, d).numpy(), w.numpy(), g.reshape(b * t, d).numpy())
    np.testing.assert_allclose(dv.reshape(shape), dv64.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, dw64.numpy(), rtol=1e-10, atol=1e-12)


def test_c_backward_matches_central_differences():
    rng = np.random.default_rng(5)
    n, t, d = 3, 2, 7
    v = rng.standard_normal((n, t, d))
    w = rng.standard_normal(d) * 0.5
    g = rng.standard_normal((t, d))
    dv, dw = c_oracle.backward(v, w, g)
    h = 1e-6

    def loss(vv, ww):
        return float(np.sum(c_oracle.forward(vv, ww) * g))

    for idx in [(0, 0, 0), (1, 1, 3), (2, 0, 6)]:
        vp, vm = v.copy(), v.copy()
        vp[idx] += h
        vm[idx] -= h
        assert abs((loss(vp, w) - loss(vm, w)) / (2 * h) - dv[idx]) < 1e-7
    for k in (0, 4):
        wp, wm = w.copy(), w.copy()
        wp[k] += h
        wm[k] -= h
        assert abs((loss(v, wp) - loss(v, wm)) / (2 * h) - dw[k]) < 1e-7


def test_single_source_has_exactly_zero_query_gradient():
    """N=1: alpha == 1 for any logit, so dw is exactly zero
    (reference tests/test_triton_op.py:174-180)."""
    v, w = _inputs(n=1, b=1, t=6, d=10)
    g = torch.randn(1, 6, 10, **F64)
    _, dw = c_oracle.backward(v.reshape(1, 6, 10).numpy(), w.numpy(), g.reshape(6, 10).numpy())
    assert np.all(dw == 0.0)


# --------------------------------------------------------------------------
# 4. The two restatements agree
# --------------------------------------------------------------------------


@pytest.mark.parametrize("shape,scale", [((5, 2, 7, 16), 1.0), ((9, 1, 8, 256), 0.5 * 16), ((17, 1, 3, 63), 2.0)])
def test_c_and_torch_forward_agree(shape, scale):
    v, w = _inputs(*shape, seed=9, scale=scale)
    n, b, t, d = shape
    got = c_oracle.forward(v.reshape(n, b * t, d).numpy(), w.numpy()).reshape(b, t, d)
    np.testing.assert_allclose(got, block_attn_res_oracle(v, w).numpy(), rtol=1e-12, atol=1e-12)


def test_c_stats_merge_and_batched_agree_with_torch():
    v, w = _inputs(n=8, b=1, t=5, d=24, seed=2)
    vt = v.reshape(8, 5, 24).numpy()
    o1, m1, l1 = c_oracle.attn_with_stats(vt[:3], w.numpy())
    o2, m2, l2 = c_oracle.attn_with_stats(vt[3:], w.numpy())
    o, _, ell = c_oracle.merge(o1, m1, l1, o2, m2, l2)
    np.testing.assert_allclose(o / ell[:, None], block_attn_res_reference(v, w)[0].numpy(), rtol=1e-12, atol=1e-12)
    ot, mt, lt = attn_with_stats(v[:3], w)
    np.testing.assert_allclose(o1, ot[0].numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(m1, mt[0].numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(l1, lt[0].numpy(), rtol=1e-12, atol=1e-12)
    q = torch.randn(3, 24, **F64)
    np.testing.assert_allclose(c_oracle.batched(vt, q.numpy()),
                               batched_folded_form(v, q)[:, 0].numpy(), rtol=1e-12, atol=1e-12)


def _stats_by_definition(v, w, eps=DEFAULT_EPS):
    """``(o, m, l)`` of one token set from the definitions, with plain Python
    loops: m is the largest logit, l the sum of exp(logit - m), o the
    exp(logit - m)-weighted sum of the raw sources."""
    n, t, d = len(v), len(v[0]), len(w)
    o = [[0.0] * d for _ in range(t)]
    m, ell = [0.0] * t, [0.0] * t
    for j in range(t):
        logits = []
        for k in range(n):
            row = v[k][j]
            r = 1.0 / math.sqrt(sum(x * x for x in row) / d + eps)
            logits.append(r * sum(a * b for a, b in zip(w, row)))
        m[j] = max(logits)
        ps = [math.exp(z - m[j]) for z in logits]
        ell[j] = sum(ps)
        for k in range(n):
            for c in range(d):
                o[j][c] += ps[k] * v[k][j][c]
    return np.array(o), np.array(m), np.array(ell)


def test_stats_follow_their_definitions():
    """m, l and o of both restatements against the definitions, on a token
    set where row 2 of token 0 is the query direction scaled by 3, so the
    largest logit is known in closed form: c ||w|| / sqrt(c^2 / D + eps)."""
    v, w = _inputs(n=4, b=1, t=3, d=10, seed=5, scale=2.0)
    v = v[:, 0].clone()
    v[2, 0] = 3.0 * w / w.norm()
    o_def, m_def, l_def = _stats_by_definition(v.tolist(), w.tolist())
    want = 3.0 * w.norm().item() / math.sqrt(9.0 / 10 + DEFAULT_EPS)
    assert math.isclose(m_def[0], want, rel_tol=1e-13)
    oc, mc, lc = c_oracle.attn_with_stats(v.numpy(), w.numpy())
    ot, mt, lt = attn_with_stats(v[:, None], w)
    for got in ((oc, mc, lc), (ot[0].numpy(), mt[0].numpy(), lt[0].numpy())):
        np.testing.assert_allclose(got[0], o_def, rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(got[1], m_def, rtol=1e-13, atol=0)
        np.testing.assert_allclose(got[2], l_def, rtol=1e-12, atol=0)
    assert mc[0] == pytest.approx(want, rel=1e-13)


def test_config1_eager_fp32_is_within_the_reference_tolerance():
    """BASELINE config 1 (the reference's CPU plumbing case): N=4 B=1 T=256
    D=512 fp32, seed 0, v ~ N(0,1), w ~ N(0, 0.5), grad_out ~ N(0,1),
    eps 1e-6. The product's eager ``folded_form`` in fp32, forward and
    backward through torch.autograd, against the float64 oracle: rel-L2 at
    most 1e-5 (the reference's fp32 tolerance, bench/bench_operator.py:289)."""
    from switchyard.baselines import folded_form as eager

    gen = torch.Generator().manual_seed(0)
    v = torch.randn(4, 1, 256, 512, generator=gen)
    w = 0.5 * torch.randn(512, generator=gen)
    g = torch.randn(1, 256, 512, generator=gen)
    vv, ww = v.clone().requires_grad_(True), w.clone().requires_grad_(True)
    out = eager(vv, ww, 1e-6)
    out.backward(g)
    o64 = block_attn_res_oracle(v, w)
    dv64, dw64 = oracle_grads(v, w, g)
    for got, ref in ((out, o64), (vv.grad, dv64), (ww.grad, dw64)):
        assert got.dtype == torch.float32
        assert rel_l2(got, ref) <= 1e-5
    # the C restatement agrees with the torch oracle on this case too
    oc = c_oracle.forward(v[:, 0].double().numpy(), w.double().numpy())
    np.testing.assert_allclose(oc, o64[0].numpy(), rtol=1e-10, atol=1e-12)


# --------------------------------------------------------------------------
# 5. Golden fixtures
# --------------------------------------------------------------------------


def _golden_cases():
    z = np.load(GOLDEN)
    return sorted({k.split("/")[0] for k in z.files}), z


@pytest.mark.parametrize("case", _golden_cases()[0])
def test_oracles_reproduce_the_golden_vectors(case):
    _, z = _golden_cases()
    v, w, g, q = (z[f"{case}/{k}"] for k in ("v", "w", "g", "q"))
    n, b, t, d = v.shape
    out = c_oracle.forward(v.reshape(n, b * t, d), w).reshape(b, t, d)
    np.testing.assert_allclose(out, z[f"{case}/out"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(block_attn_res_reference(torch.from_numpy(v), torch.from_numpy(w)).numpy(),
                               z[f"{case}/out"], rtol=1e-12, atol=1e-13)
    dv, dw = c_oracle.backward(v.reshape(n, b * t, d), w, g.reshape(b * t, d))
    np.testing.assert_allclose(dv.reshape(v.shape), z[f"{case}/dv"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(dw, z[f"{case}/dw"], rtol=1e-13, atol=1e-14)
    np.testing.assert_allclose(c_oracle.batched(v.reshape(n, b * t, d), q).reshape(z[f"{case}/batched"].shape),
                               z[f"{case}/batched"], rtol=1e-13, atol=1e-14)
    # Inputs are bf16-exact, so every dtype sees the same values.
    assert np.array_equal(torch.from_numpy(v).to(torch.bfloat16).double().numpy(), v)


# --------------------------------------------------------------------------
# 6. Planted mistakes: each mutant must fail at least one pin
# --------------------------------------------------------------------------


def _fwd_np(v, w, eps=DEFAULT_EPS, *, sqrt_d=False, norm_values=False, sum_not_mean=False,
            token_softmax=False):
    """A forward with optional planted mistakes. v [N, T, D]."""
    ms = (v * v).sum(-1) if sum_not_mean else (v * v).mean(-1)
    r = 1.0 / np.sqrt(ms + eps)
    logit = np.einsum("d,ntd->nt", w, v) * r
    if sqrt_d:
        logit = logit / math.sqrt(v.shape[-1])
    axis = 1 if token_softmax else 0
    p = np.exp(logit - logit.max(axis=axis, keepdims=True))
    alpha = p / p.sum(axis=axis, keepdims=True)
    vals = v * r[..., None] if norm_values else v
    return np.einsum("nt,ntd->td", alpha, vals)


def _bwd_np(v, w, g, eps=DEFAULT_EPS, *, flip_dssq=False, drop_w_term=False):
    n, t, d = v.shape
    ss = (v * v).sum(-1)
    r = 1.0 / np.sqrt(ss / d + eps)
    a = np.einsum("d,ntd->nt", w, v)
    logit = a * r
    p = np.exp(logit - logit.max(0))
    alpha = p / p.sum(0)
    gdot = np.einsum("td,ntd->nt", g, v)
    s = (alpha * gdot).sum(0)
    dlogit = alpha * (gdot - s)
    da = dlogit * r
    dssq = (1 if flip_dssq else -1) * dlogit * a * r ** 3 / (2 * d)
    dv = alpha[..., None] * g[None] + 2 * dssq[..., None] * v
    if not drop_w_term:
        dv = dv + da[..., None] * w
    dw = np.einsum("nt,ntd->d", da, v)
    return dv, dw


def _failed_pins(fwd, bwd) -> list[str]:
    """Run the closed-form, golden and derivative pins on a candidate oracle."""
    failed = []
    rng = np.random.default_rng(3)
    x = rng.standard_normal(16)
    w = rng.standard_normal(16) * 0.3
    if not np.allclose(fwd(np.stack([x, -x])[:, None, :], w)[0], _antipodal_expected(x, w, DEFAULT_EPS),
                       rtol=1e-9, atol=1e-12):
        failed.append("antipodal")
    v = np.array([[[2.0, 0, 0, 0]], [[0, 3.0, 0, 0]]])
    out = fwd(v, np.array([0.7, -0.4, 0, 0]))[0]
    l0, l1 = 1.4 / math.sqrt(1 + DEFAULT_EPS), -1.2 / math.sqrt(2.25 + DEFAULT_EPS)
    e0, e1 = math.exp(l0), math.exp(l1)
    if not np.allclose(out, [2 * e0 / (e0 + e1), 3 * e1 / (e0 + e1), 0, 0], rtol=1e-9):
        failed.append("axis_aligned")
    z = np.load(GOLDEN)
    for case in ("small", "odd", "deep"):
        vv, ww, gg = z[f"{case}/v"], z[f"{case}/w"], z[f"{case}/g"]
        n, b, t, d = vv.shape
        if not np.allclose(fwd(vv.reshape(n, b * t, d), ww).reshape(b, t, d), z[f"{case}/out"], rtol=1e-9):
            failed.append(f"golden_fwd_{case}")
        dv, dw = bwd(vv.reshape(n, b * t, d), ww, gg.reshape(b * t, d))
        if not (np.allclose(dv.reshape(vv.shape), z[f"{case}/dv"], rtol=1e-9, atol=1e-12)
                and np.allclose(dw, z[f"{case}/dw"], rtol=1e-9, atol=1e-12)):
            failed.append(f"golden_bwd_{case}")
    # central difference of the candidate's own forward vs its backward
    vv = rng.standard_normal((3, 2, 5))
    ww = rng.standard_normal(5) * 0.5
    gg = rng.standard_normal((2, 5))
    dv, dw = bwd(vv, ww, gg)
    h = 1e-6
    vp, vm = vv.copy(), vv.copy()
    vp[1, 0, 2] += h
    vm[1, 0, 2] -= h
    fd = (np.sum(fwd(vp, ww) * gg) - np.sum(fwd(vm, ww) * gg)) / (2 * h)
    if abs(fd - dv[1, 0, 2]) > 1e-6:
        failed.append("central_difference")
    return failed


def test_unmutated_oracle_passes_every_pin():
    assert _failed_pins(_fwd_np, _bwd_np) == []


@pytest.mark.parametrize("mutation", ["sqrt_d", "norm_values", "sum_not_mean", "token_softmax"])
def test_planted_forward_mistakes_are_caught(mutation):
    def fwd(v, w):
        return _fwd_np(v, w, **{mutation: True})

    assert _failed_pins(fwd, _bwd_np), f"{mutation} slipped past every pin"


@pytest.mark.parametrize("mutation", ["flip_dssq", "drop_w_term"])
def test_planted_backward_mistakes_are_caught(mutation):
    def bwd(v, w, g):
        return _bwd_np(v, w, g, **{mutation: True})

    assert _failed_pins(_fwd_np, bwd), f"{mutation} slipped past every pin"


# --------------------------------------------------------------------------
# 6. Merge statistics, the merge and the batched operator: gradients
#    (no reference counterpart; pinned by f64 autograd, gradcheck and central
#    differences of the already-pinned forwards)
# --------------------------------------------------------------------------


def _stats_loss(v, w, go, gm, gl):
    o, m, ell = c_oracle.attn_with_stats(v, w)
    return float(np.sum(o * go) + np.sum(m * gm) + np.sum(ell * gl))


def _stats_case(seed=11, n=5, t=4, d=12, scale=1.5):
    rng = np.random.default_rng(seed)
    v = rng.standard_normal((n, t, d))
    w = rng.standard_normal(d) * scale
    go = rng.standard_normal((t, d))
    gm, gl = rng.standard_normal(t), rng.standard_normal(t)
    return v, w, go, gm, gl


def _stats_bwd_np(v, w, go, gm, gl, drop_gm=False, normalized=False, keep_top=False):
    """numpy restatement of oracle_attn_with_stats_backward with plantable mistakes."""
    n, t, d = v.shape
    ssq = np.einsum("ntd,ntd->nt", v, v)
    r = 1.0 / np.sqrt(ssq / d + DEFAULT_EPS)
    a = np.einsum("d,ntd->nt", w, v)
    logit = a * r
    top = logit.argmax(0)
    p = np.exp(logit - logit.max(0))
    if normalized:
        p = p / p.sum(0)
    dl = p * (np.einsum("td,ntd->nt", go, v) + gl)
    other = dl.sum(0) - (0.0 if keep_top else dl[top, np.arange(t)])
    dl[top, np.arange(t)] = (0.0 if drop_gm else gm) - other
    da = dl * r
    dssq = -dl * a * r**3 / (2 * d)
    dv = p[..., None] * go[None] + da[..., None] * w + 2 * dssq[..., None] * v
    return dv, np.einsum("nt,ntd->d", da, v)


def _stats_pins_fail(bwd) -> list[str]:
    failed = []
    v, w, go, gm, gl = _stats_case()
    dv, dw = bwd(v, w, go, gm, gl)
    h = 1e-6
    for idx in [(0, 0, 0), (2, 1, 5), (4, 3, 11)]:
        vp, vm = v.copy(), v.copy()
        vp[idx] += h
        vm[idx] -= h
        fd = (_stats_loss(vp, w, go, gm, gl) - _stats_loss(vm, w, go, gm, gl)) / (2 * h)
        if abs(fd - dv[idx]) > 1e-6 * max(1.0, abs(fd)):
            failed.append(f"dv{idx}")
    for k in (0, 7):
        wp, wm = w.copy(), w.copy()
        wp[k] += h
        wm[k] -= h
        fd = (_stats_loss(v, wp, go, gm, gl) - _stats_loss(v, wm, go, gm, gl)) / (2 * h)
        if abs(fd - dw[k]) > 1e-6 * max(1.0, abs(fd)):
            failed.append(f"dw{k}")
    return failed


def test_c_stats_backward_passes_central_differences():
    assert _stats_pins_fail(c_oracle.attn_with_stats_backward) == []
    assert _stats_pins_fail(_stats_bwd_np) == []


@pytest.mark.parametrize("mutation", ["drop_gm", "normalized", "keep_top"])
def test_planted_stats_backward_mistakes_are_caught(mutation):
    def bwd(*a):
        return _stats_bwd_np(*a, **{mutation: True})

    assert _stats_pins_fail(bwd), f"{mutation} slipped past every pin"


def test_torch_stats_and_merge_pass_gradcheck():
    torch.manual_seed(5)
    v = torch.randn(4, 1, 3, 6, **F64, requires_grad=True)
    w = torch.randn(6, **F64, requires_grad=True)
    assert torch.autograd.gradcheck(lambda a, b: attn_with_stats(a, b), (v, w), eps=1e-6,
                                    atol=1e-8, rtol=1e-6)
    o1, o2 = (torch.randn(3, 5, **F64, requires_grad=True) for _ in range(2))
    m1 = torch.tensor([0.3, -1.0, 2.0], **F64, requires_grad=True)
    m2 = torch.tensor([-0.4, 0.5, 1.2], **F64, requires_grad=True)
    l1, l2 = (torch.rand(3, **F64).add(0.5).requires_grad_() for _ in range(2))
    assert torch.autograd.gradcheck(merge_online_softmax, (o1, m1, l1, o2, m2, l2), eps=1e-6,
                                    atol=1e-8, rtol=1e-6)


def test_c_stats_backward_matches_autograd():
    v, w, go, gm, gl = _stats_case(seed=21, n=7, t=6, d=20, scale=3.0)
    vt = torch.tensor(v, requires_grad=True)
    wt = torch.tensor(w, requires_grad=True)
    o, m, ell = attn_with_stats(vt[:, None], wt)
    loss = (o[0] * torch.tensor(go)).sum() + (m[0] * torch.tensor(gm)).sum() + (ell[0] * torch.tensor(gl)).sum()
    gv, gw = torch.autograd.grad(loss, (vt, wt))
    dv, dw = c_oracle.attn_with_stats_backward(v, w, go, gm, gl)
    np.testing.assert_allclose(dv, gv.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, gw.numpy(), rtol=1e-10, atol=1e-12)


def test_c_merge_backward_matches_autograd():
    rng = np.random.default_rng(8)
    t, d = 6, 9
    o1, o2, go = (rng.standard_normal((t, d)) for _ in range(3))
    m1 = np.array([0.1, 2.0, -1.0, 0.7, 3.0, -2.0])
    m2 = np.array([1.1, 0.5, -0.5, 0.2, 4.0, -3.0])  # group 2 wins some tokens, group 1 others
    l1, l2 = rng.random(t) + 0.5, rng.random(t) + 0.5
    gm, gl = rng.standard_normal(t), rng.standard_normal(t)
    ins = [torch.tensor(a, requires_grad=True) for a in (o1, m1, l1, o2, m2, l2)]
    o, m, ell = merge_online_softmax(*ins)
    loss = (o * torch.tensor(go)).sum() + (m * torch.tensor(gm)).sum() + (ell * torch.tensor(gl)).sum()
    want = torch.autograd.grad(loss, ins)
    got = c_oracle.merge_backward(o1, m1, l1, o2, m2, l2, go, gm, gl)  # same input order
    for g, ref in zip(got, want):
        np.testing.assert_allclose(g, ref.numpy(), rtol=1e-12, atol=1e-12)


def test_c_batched_backward_matches_autograd_of_the_batched_form():
    v, _ = _inputs(n=5, b=1, t=4, d=16, seed=13)
    q = (torch.randn(3, 16, **F64) * 0.7)
    g = torch.randn(3, 1, 4, 16, **F64)
    vt, qt = v.clone().requires_grad_(), q.clone().requires_grad_()
    out = batched_folded_form(vt, qt)
    gv, gq = torch.autograd.grad((out * g).sum(), (vt, qt))
    dv, dq = c_oracle.batched_backward(v[:, 0].numpy(), q.numpy(), g[:, 0].numpy())
    np.testing.assert_allclose(dv, gv[:, 0].numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, gq.numpy(), rtol=1e-10, atol=1e-12)
