"""Pointer-table source input (GPU): ``block_attn_res_sources`` against the
stacked operator and the float64 oracle.

The table entry points run the same kernels on the same rows as the stacked
ones, so outputs and gradients must match the stacked operator bit for bit,
for sources that are separate allocations, views of one buffer, or a mix.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from oracle import c_oracle  # noqa: E402
from oracle.reference import DEFAULT_EPS, dtype_floor, rel_l2  # noqa: E402
from switchyard import _lib  # noqa: E402
from switchyard.table_op import MAX_SOURCES, block_attn_res_sources  # noqa: E402
from switchyard.triton_op import block_attn_res_batched, block_attn_res_triton  # noqa: E402

DEV = "cuda"


def _make(n, b, t, d, dtype, seed=0, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, b, t, d, generator=g).to(dtype)
    w = torch.randn(d, generator=g)
    w = (w / w.norm() * scale).to(dtype)
    gr = torch.randn(b, t, d, generator=g).to(dtype)
    return v.to(DEV), w.to(DEV), gr.to(DEV)


def _separate(v):
    """Each source its own allocation (not a view of v)."""
    return [v[i].clone() for i in range(v.shape[0])]


SHAPES = [(1, 1, 64, 256), (5, 2, 33, 512), (9, 1, 256, 2048), (16, 1, 64, 1024),
          (3, 1, 40, 777), (9, 1, 64, 4096), (16, 1, 64, 2048), (12, 1, 32, 4096)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_table_matches_the_stacked_operator_bit_for_bit(shape, dtype):
    print(f"table fwd/bwd {shape} {dtype}", flush=True)
    v, w, gr = _make(*shape, dtype, seed=3, scale=4.0)
    vs = v.clone().requires_grad_()
    ws = w.clone().requires_grad_()
    ref = block_attn_res_triton(vs, ws)
    ref.backward(gr)

    srcs = [s.requires_grad_() for s in _separate(v)]
    wt = w.clone().requires_grad_()
    got = block_attn_res_sources(srcs, wt)
    got.backward(gr)
    assert torch.equal(got, ref)
    for i, s in enumerate(srcs):
        assert torch.equal(s.grad, vs.grad[i]), f"source {i}"
    assert torch.equal(wt.grad, ws.grad)


def test_table_accepts_views_and_mixed_allocations():
    v, w, _ = _make(6, 2, 48, 1024, torch.bfloat16, seed=5, scale=2.0)
    ref = block_attn_res_triton(v, w)
    mixed = [v[0], v[1].clone(), v[2], v[3].clone(), v[4], v[5]]
    assert torch.equal(block_attn_res_sources(mixed, w), ref)
    # sources in any memory order: the table, not the addresses, fixes the order
    perm = [3, 0, 5, 1, 4, 2]
    assert torch.equal(block_attn_res_sources([v[i] for i in perm], w),
                       block_attn_res_triton(v[perm].contiguous(), w))


def test_table_reaches_the_oracle_floor():
    v, w, gr = _make(9, 1, 128, 2048, torch.bfloat16, seed=7, scale=8.0)
    got = block_attn_res_sources(list(v.unbind(0)), w)
    oracle = c_oracle.forward(v.reshape(9, 128, 2048).double().cpu().numpy(), w.double().cpu().numpy())
    oracle = torch.from_numpy(oracle).reshape(1, 128, 2048)
    err, floor = rel_l2(got, oracle), dtype_floor(oracle, torch.bfloat16)
    assert err <= 1.10 * floor, (err, floor)


def test_table_rejects_what_it_cannot_take():
    v, w, _ = _make(MAX_SOURCES + 1, 1, 8, 64, torch.bfloat16)
    with pytest.raises(ValueError, match="at most 16"):
        block_attn_res_sources(list(v.unbind(0)), w)
    with pytest.raises(ValueError, match="at least one"):
        block_attn_res_sources([], w)
    with pytest.raises(ValueError, match="every source"):
        block_attn_res_sources([v[0], v[1, :, :4]], w)
    with pytest.raises(ValueError, match="same dtype"):
        block_attn_res_sources([v[0], v[1].float()], w)
    with pytest.raises(ValueError, match=r"w must be \[64\]"):
        block_attn_res_sources([v[0]], w[:32])


def test_c_table_entry_points_validate_before_launch():
    lib = _lib.lib()
    v, w, _ = _make(2, 1, 8, 64, torch.bfloat16)
    out = torch.empty(1, 8, 64, device=DEV, dtype=torch.bfloat16)
    rows = _lib.pointer_table(list(v.unbind(0)))
    bad = (ctypes.c_void_p * 2)(v[0].data_ptr(), None)
    p = ctypes.c_void_p
    assert lib.sy_fwd_table(bad, p(w.data_ptr()), p(out.data_ptr()), None, 2, 8, 64, 2, 2, 1e-6, None) == -1
    big = (ctypes.c_void_p * 17)(*([v[0].data_ptr()] * 17))
    assert lib.sy_fwd_table(big, p(w.data_ptr()), p(out.data_ptr()), None, 17, 8, 64, 2, 2, 1e-6, None) == -2
    assert lib.sy_fwd_table(rows, p(w.data_ptr()), p(out.data_ptr()), None, 2, 8, 64, 2, 2, 1e-6,
                            _lib.stream_ptr(v.device)) == 0
    torch.cuda.synchronize()
    assert torch.equal(out, block_attn_res_triton(v, w))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_batched_table_matches_the_stacked_batched_op(dtype):
    v, _, _ = _make(9, 1, 96, 2048, dtype, seed=2)
    q = (torch.randn(5, 2048, generator=torch.Generator().manual_seed(1)) * 0.5).to(dtype).to(DEV)
    ref = block_attn_res_batched(v, q)
    out = torch.empty_like(ref)
    lib = _lib.lib()
    srcs = _separate(v)  # kept alive until the launch has run
    rc = lib.sy_fwd_batched_table(_lib.pointer_table(srcs), ctypes.c_void_p(q.data_ptr()),
                                  ctypes.c_void_p(out.data_ptr()), 9, 5, 96, 2048,
                                  _lib.dtype_code(dtype), DEFAULT_EPS, _lib.stream_ptr(v.device))
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
