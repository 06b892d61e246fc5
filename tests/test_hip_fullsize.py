"""GPU checks at the committed golden vectors and at BASELINE.json's full size.

Full size (N=9, B=1, T=4096, D=2048) is too large for the float64 CPU oracle
to run in seconds, so there the checks are size-independent properties: a
single source is the identity (bitwise), a zero query averages, tokens are
independent (a slice equals the full run bitwise), the backward is linear in
grad_out, dw is bit-reproducible, and the C ABI's staged and fused backward
and its stats / recompute paths agree.
"""

from __future__ import annotations

import ctypes
import pathlib

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from oracle.reference import dtype_floor, rel_l2  # noqa: E402
from switchyard import _lib  # noqa: E402
from switchyard.hip_op import block_attn_res_batched, block_attn_res_hip  # noqa: E402

DEV = torch.device("cuda")
GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "attnres_golden.npz"
FULL = (9, 1, 4096, 2048)


def _bound(floor, dtype, grad=False):
    """bf16/fp16: 1.10x the rounding floor. fp32: 1e-6 for outputs (the
    reference's forward bound) and 1e-5 for gradients (the north-star fp32
    bound; a saturated softmax amplifies fp32 logit rounding into dw)."""
    if dtype == torch.float32:
        return 1e-5 if grad else 1e-6
    return max(1.10 * floor, 1e-6)


def _cases():
    z = np.load(GOLDEN)
    return sorted({k.split("/")[0] for k in z.files})


@pytest.mark.parametrize("case", _cases())
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_golden_vectors(case, dtype):
    z = np.load(GOLDEN)
    v, w, g, q = (torch.from_numpy(z[f"{case}/{k}"]) for k in ("v", "w", "g", "q"))
    vt = v.to(dtype).to(DEV).requires_grad_(True)
    wt = w.to(dtype).to(DEV).requires_grad_(True)
    out = block_attn_res_hip(vt, wt)
    out.backward(g.to(dtype).to(DEV))
    want = {k: torch.from_numpy(z[f"{case}/{k}"]) for k in ("out", "dv", "dw", "batched")}
    for name, got in (("out", out), ("dv", vt.grad), ("dw", wt.grad)):
        if name == "dw" and v.shape[0] == 1:
            assert torch.count_nonzero(got) == 0
            continue
        err = rel_l2(got, want[name])
        bound = _bound(dtype_floor(want[name], dtype), dtype, grad=name != "out")
        assert err <= bound, f"{case} {name}: {err:.3e} > {bound:.3e}"
    with torch.no_grad():
        got = block_attn_res_batched(v.to(dtype).to(DEV), q.to(dtype).to(DEV))
    err = rel_l2(got, want["batched"])
    assert err <= _bound(dtype_floor(want["batched"], dtype), dtype)


def _full(dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    n, b, t, d = FULL
    v = torch.randn(n, b, t, d, generator=g).to(dtype).to(DEV)
    w = (0.5 * torch.randn(d, generator=g)).to(dtype).to(DEV)
    gr = torch.randn(b, t, d, generator=g).to(dtype).to(DEV)
    return v, w, gr


def test_single_source_is_the_identity_bitwise():
    v, w, _ = _full()
    assert torch.equal(block_attn_res_hip(v[:1], w), v[0])


def test_zero_query_averages_at_full_size():
    v, _, _ = _full(torch.float32)
    out = block_attn_res_hip(v, torch.zeros(v.shape[-1], device=DEV))
    torch.testing.assert_close(out, v.mean(0), rtol=2e-6, atol=2e-6)


def test_tokens_are_independent_bitwise():
    """A token's output depends only on its own rows and on whether it is its
    wave's final token (the persistent forward folds a final token's rows in
    as they land, a rounding apart from the two-pass form of earlier tokens):
    a slice of the full run's final round equals a run of that slice, where
    every token is final, bit for bit; earlier-round tokens agree within the
    bf16 rounding."""
    v, w, _ = _full()
    n, b, t, d = FULL
    info = (ctypes.c_int32 * 4)()
    assert _lib.lib().sy_kernel_info(0, n, b * t, d, 2, 2, info) == 0
    slots = info[3] * 4  # one-wave tokens, four per 256-thread workgroup
    assert t <= 2 * slots, "the full run holds at most two tokens a wave"
    full = block_attn_res_hip(v, w)
    lo = max(slots, t - 600)  # inside the final round
    part = block_attn_res_hip(v[:, :, lo:lo + 517].contiguous(), w)
    assert torch.equal(full[:, lo:lo + 517], part)
    early = block_attn_res_hip(v[:, :, 1000:1517].contiguous(), w)
    torch.testing.assert_close(full[:, 1000:1517].float(), early.float(), rtol=2**-7, atol=2**-7)
    assert rel_l2(early, full[:, 1000:1517].double()) <= 2**-8


def _fwd_bwd(v, w, g):
    vt, wt = v.clone().requires_grad_(True), w.clone().requires_grad_(True)
    block_attn_res_hip(vt, wt).backward(g)
    return vt.grad, wt.grad


def test_backward_is_linear_in_grad_out():
    v, w, g1 = _full(torch.float32, seed=1)
    g2 = torch.randn_like(g1)
    dv1, dw1 = _fwd_bwd(v, w, g1)
    dv2, dw2 = _fwd_bwd(v, w, g2)
    dv3, dw3 = _fwd_bwd(v, w, g1 + 2.0 * g2)
    assert rel_l2(dv3, dv1 + 2.0 * dv2) < 1e-6
    assert rel_l2(dw3, dw1 + 2.0 * dw2) < 1e-5


def test_full_size_dw_is_bit_reproducible():
    v, w, g = _full()
    a = _fwd_bwd(v, w, g)
    b = _fwd_bwd(v, w, g)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def test_abi_stats_and_recompute_paths_and_staged_backward_agree():
    lib = _lib.lib()
    v, w, g = _full(seed=3)
    n, b, t, d = FULL
    nt = b * t
    stream = _lib.stream_ptr(DEV)
    out = torch.empty(b, t, d, device=DEV, dtype=v.dtype)
    stats = torch.empty(2, n, nt, device=DEV)
    assert lib.sy_fwd(_ptr(v), _ptr(w), _ptr(out), _ptr(stats), n, nt, d, nt * d, 2, 2, 1e-6, stream) == 0
    ws_bytes = lib.sy_bwd_workspace_bytes(n, nt, d, 2, 2)
    assert 0 < ws_bytes <= 8 << 20
    ws = torch.empty(ws_bytes // 4, device=DEV)
    res = {}
    for name, st in (("stats", stats), ("recompute", None)):
        dv = torch.empty_like(v)
        dw = torch.empty(d, device=DEV, dtype=w.dtype)
        assert lib.sy_bwd(_ptr(v), _ptr(w), _ptr(g), _ptr(st), _ptr(dv), _ptr(dw), _ptr(ws), ws_bytes,
                          n, nt, d, nt * d, 2, 2, 1e-6, stream) == 0
        res[name] = (dv, dw)
    assert rel_l2(res["stats"][0], res["recompute"][0].double()) < 2e-3
    assert rel_l2(res["stats"][1], res["recompute"][1].double()) < 2e-3
    # staged == fused, bitwise
    dv = torch.empty_like(v)
    dw = torch.empty(d, device=DEV, dtype=w.dtype)
    rows = lib.sy_bwd_partial_rows(n, nt, d, 2, 2, 1, 1)
    assert rows > 0 and rows * d * 4 <= ws_bytes
    assert lib.sy_bwd_main(_ptr(v), _ptr(w), _ptr(g), _ptr(stats), _ptr(dv), _ptr(ws), ws_bytes,
                           n, nt, d, nt * d, 2, 2, 1e-6, stream) == 0
    assert lib.sy_dw_reduce(_ptr(ws), rows, d, _ptr(dw), 2, stream) == 0
    assert torch.equal(dv, res["stats"][0]) and torch.equal(dw, res["stats"][1])
    # a short workspace is refused before any launch
    assert lib.sy_bwd(_ptr(v), _ptr(w), _ptr(g), _ptr(stats), _ptr(dv), _ptr(dw), _ptr(ws), 1024,
                      n, nt, d, nt * d, 2, 2, 1e-6, stream) == -4


def test_kernel_info_reports_the_persistent_grids():
    lib = _lib.lib()
    info = (ctypes.c_int32 * 4)()
    n, b, t, d = FULL
    assert lib.sy_kernel_info(0, n, b * t, d, 2, 2, info) == 0
    vgpr, lds, per_cu, grid = list(info)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert 0 < vgpr <= 256 and per_cu >= 1 and grid == min(cus * per_cu, b * t // 4)
    assert lib.sy_kernel_info(1, n, b * t, d, 2, 2, info) == 0
    vgpr, lds, per_cu, grid = list(info)
    # The backward's (1, 4, 9) tile runs one wave per SIMD in 256-thread
    # workgroups: up to 512 registers (VGPRs + AGPRs), one workgroup per CU.
    bplan = _lib.plan(_lib.OP_BWD, n, d, torch.bfloat16)
    waves_per_block = bplan["block_threads"] // 64
    waves_per_simd = min(8, 512 // (-(-vgpr // 8) * 8))
    assert 0 < vgpr <= 512 and lds > 0 and grid == cus * per_cu
    assert per_cu == max(1, waves_per_simd * 4 // waves_per_block)


def test_speed_of_light_and_probes():
    from switchyard.hip_op import bandwidth_probe, probe_grid, speed_of_light

    v, _, _ = _full(torch.float32)
    torch.testing.assert_close(speed_of_light(v), v.sum(0), rtol=1e-5, atol=1e-5)
    src = torch.arange(1 << 20, device=DEV, dtype=torch.int32)
    dst = torch.empty_like(src)
    bandwidth_probe("copy", src, dst)
    assert torch.equal(src, dst)
    bandwidth_probe("write", None, dst)
    assert torch.all(dst.view(torch.float32) == 1.0)
    out = torch.zeros(probe_grid(src.numel() * 4), device=DEV)
    bandwidth_probe("read", src, out)
    torch.cuda.synchronize()
    # the 9:1 mix probe: 36 KiB steps in, 4 KiB steps out (one step ragged at the end)
    steps = 37
    mix_src = torch.randint(-1000, 1000, (steps * 9 * 1024 - 9 * 4 * 37,), device=DEV, dtype=torch.int32)
    mix_dst = torch.zeros(mix_src.numel() // 9, device=DEV, dtype=torch.int32)
    bandwidth_probe("mix", mix_src, mix_dst)
    full = (steps - 1) * 9 * 1024
    want = mix_src[:full].view(steps - 1, 9, 256, 4).sum(1).flatten()
    assert torch.equal(mix_dst[: (steps - 1) * 1024], want)
