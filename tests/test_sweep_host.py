"""Host side of ``bench.py --sweep`` (CPU): which shapes a run measures, and
the float64 comparator that gates each measured shape, pinned against the C
oracle and the dtype-floor metric."""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import bench
from oracle import c_oracle
from switchyard import harness


def test_every_shape_is_measured_once_with_all_its_sets():
    shapes = dict(bench._sweep_shapes(None))
    listed = {(n, b, t, d) for _, n, b, t, d in bench.SWEEP_SHAPES}
    assert set(shapes) == listed
    assert shapes[(9, 1, 4096, 2048)] == ["n-sweep", "t-sweep", "d-sweep-b1"]
    assert shapes[(9, 1, 2048, 2048)] == ["t-sweep", "batch"]
    # the reference's shape sets (bench/bench_operator.py:65-79) are all here
    for shape in [(9, 1, 4096, d) for d in (1024, 2048, 4096, 8192)] + \
                 [(9, b, 2048, 2048) for b in (1, 2, 4, 8)] + [(9, 1, 128, 1024), (9, 1, 512, 1024), (4, 1, 256, 512)]:
        assert shape in shapes


def test_sweep_only_matches_n_only_in_the_n_sweep():
    assert [s for s, _ in bench._sweep_shapes({"N9"})] == [(9, 1, 4096, 2048)]
    assert [s for s, _ in bench._sweep_shapes({"N4"})] == [(4, 1, 4096, 2048)]
    assert [s for s, _ in bench._sweep_shapes({"small"})] == [(9, 1, 128, 1024), (9, 1, 512, 1024), (4, 1, 256, 512)]


def test_reference_tables_cover_the_shapes_they_name():
    shapes = dict(bench._sweep_shapes(None))
    assert set(bench.REFERENCE_RESULTS) <= set(shapes)
    assert len(bench.BATCHED_SHAPE_CHECKS) == 6


@pytest.mark.parametrize("shape", [(3, 2, 5, 64), (9, 1, 7, 63), (1, 1, 3, 16)])
def test_float64_comparator_equals_the_c_oracle(shape):
    n, b, t, d = shape
    g = torch.Generator().manual_seed(sum(shape))
    v = torch.randn(n, b, t, d, generator=g)
    w = 0.5 * torch.randn(d, generator=g)
    go = torch.randn(b, t, d, generator=g)
    out, dv, dw = harness.float64_operator(v, w, go)
    rdw = np.zeros(d)
    for bi in range(b):
        vb, gb = v[:, bi].double().numpy(), go[bi].double().numpy()
        np.testing.assert_allclose(out[bi].numpy(), c_oracle.forward(vb, w.double().numpy()), rtol=0, atol=1e-12)
        rdv, dwb = c_oracle.backward(vb, w.double().numpy(), gb)
        np.testing.assert_allclose(dv[:, bi].numpy(), rdv, rtol=0, atol=1e-12)
        rdw += dwb
    np.testing.assert_allclose(dw.numpy(), rdw, rtol=1e-12, atol=1e-12)


def test_gate_applies_the_north_star_bars():
    ref = torch.randn(4096, dtype=torch.float64, generator=torch.Generator().manual_seed(0))
    assert bench._gate("bf16", ref.to(torch.bfloat16), ref)["ok"]          # exactly the floor
    noisy = (ref * (1 + 0.02 * torch.randn(4096, dtype=torch.float64))).to(torch.bfloat16)
    assert not bench._gate("bf16", noisy, ref)["ok"]                          # well above it
    assert bench._gate("fp32", ref.float(), ref)["ok"]
    assert not bench._gate("fp32", (ref * (1 + 1e-4)).float(), ref)["ok"]   # 1e-4 > 1e-5
    bad = ref.to(torch.bfloat16).clone()
    bad[0] = float("nan")
    assert not bench._gate("bf16", bad, ref)["ok"]
