"""The tiles the shape sweeps time, checked at the shapes that select them (GPU).

Which register tile a launch runs depends on N, D and (below three tokens per
CU) the token count, so a test at a small T can exercise a different kernel
from the one a sweep times. These cases run the sweep shapes themselves -- or,
for the D sweep, the same tile at a token count above four per CU -- assert
through ``sy_plan_for_tokens`` which tile the launch takes, and compare the
forward output, dv and dw with the float64 C oracle at the 1.10x dtype-floor
bar. If a future planner change moves a shape onto another tile, the tile
assertion fails before the numbers are compared.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from oracle import c_oracle  # noqa: E402
from oracle.reference import dtype_floor, rel_l2  # noqa: E402
from switchyard import _lib  # noqa: E402
from switchyard.hip_op import block_attn_res_hip  # noqa: E402

DEV = "cuda"
CUS = torch.cuda.get_device_properties(0).multi_processor_count


def _tile(op, n, d, dtype, n_tok):
    p = _lib.plan(op, n, d, dtype, n_tok=n_tok)
    return p["family_name"], (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"])


def _check(n, b, t, d, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    v = torch.randn(n, b, t, d, generator=gen).to(dtype)
    w = (0.5 * torch.randn(d, generator=gen)).to(dtype)
    g = torch.randn(b, t, d, generator=gen).to(dtype)
    vv = v.to(DEV).requires_grad_(True)
    ww = w.to(DEV).requires_grad_(True)
    out = block_attn_res_hip(vv, ww)
    out.backward(g.to(DEV))
    torch.cuda.synchronize()
    n_tok = b * t
    v64 = v.double().reshape(n, n_tok, d).numpy()
    ro = torch.from_numpy(c_oracle.forward(v64, w.double().numpy()))
    rdv, rdw = c_oracle.backward(v64, w.double().numpy(), g.double().reshape(n_tok, d).numpy())
    res = {}
    for name, got, ref in (("out", out.detach().reshape(n_tok, d), ro),
                           ("dv", vv.grad.reshape(n, n_tok, d), torch.from_numpy(rdv)),
                           ("dw", ww.grad, torch.from_numpy(rdw))):
        err, floor = rel_l2(got.cpu(), ref), dtype_floor(ref, dtype)
        res[name] = err / floor
        assert err <= 1.10 * floor, f"{name}: rel_l2 {err:.4e} vs floor {floor:.4e}"
    return res


# (n, b, t, d): expected (forward family, tile), (backward tile)
SWEEP_CASES = [
    # N sweep, B=1 T=4096 D=2048 (config 4)
    ((2, 1, 4096, 2048), ("resident", (1, 4, 4)), (1, 4, 4)),
    ((4, 1, 4096, 2048), ("resident", (1, 4, 4)), (1, 4, 4)),
    ((16, 1, 4096, 2048), ("chunked", (1, 4, 4)), (1, 4, 16)),
    # 2 <= N <= 4 in 16 bits: the four-chunk 4-row backward at every width,
    # with a partly filled tile at N=3; the 9-row four-wave tile at D=8192
    ((3, 1, 1024, 2048), ("resident", (1, 4, 4)), (1, 4, 4)),
    ((2, 1, 1024, 4096), ("resident", (2, 4, 4)), (2, 4, 4)),
    ((4, 1, 768, 8192), ("resident", (4, 4, 4)), (4, 4, 4)),
    ((9, 1, 768, 8192), ("resident", (4, 4, 9)), (4, 4, 9)),
    # N between the sweep points: the 16-row backward with a partly filled tile
    # (four tokens per CU: the forward's four-row chunks on two waves)
    ((12, 1, 4 * 256, 2048), ("chunked", (2, 2, 4)), (1, 4, 16)),
    # D sweep tiles (config 4 uses B=4 T=4096; the tile depends only on the
    # token count being above two per CU, four for the D=1024 backward)
    ((9, 4, 512, 1024), ("resident", (1, 2, 9)), (1, 2, 9)),
    ((9, 4, 256, 4096), ("resident", (2, 4, 9)), (2, 4, 9)),
    # 16 < N <= 32: the 32-row backward tile (the reference's n-sweep has N=32)
    ((32, 1, 4096, 2048), ("chunked", (1, 4, 4)), (2, 2, 32)),
    ((17, 1, 4 * 256, 2048), ("chunked", (1, 4, 4)), (2, 2, 32)),
    ((24, 4, 256, 1024), ("chunked", (1, 2, 16)), (2, 1, 32)),
    ((32, 1, 1024, 4096), ("chunked", (2, 4, 4)), (4, 2, 32)),
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape,fwd,bwd", SWEEP_CASES, ids=[f"N{s[0]}B{s[1]}T{s[2]}D{s[3]}" for s, _, _ in SWEEP_CASES])
def test_sweep_shape_runs_its_tile_at_the_oracle_floor(shape, fwd, bwd, dtype):
    n, b, t, d = shape
    if shape in ((12, 1, 4 * 256, 2048), (17, 1, 4 * 256, 2048)):
        t = 4 * CUS  # four tokens per CU on any device
    n_tok = b * t
    assert n_tok > 2 * CUS, "the token-count rule would pick another tile"
    print(f"sweep tile N={n} B={b} T={t} D={d} {dtype}: expect fwd {fwd} bwd {bwd}", flush=True)
    assert _tile(_lib.OP_FWD, n, d, dtype, n_tok) == fwd
    assert _tile(_lib.OP_BWD, n, d, dtype, n_tok) == ("resident", bwd)
    res = _check(n, b, t, d, dtype, seed=100 + n + d // 512)
    print(f"  ratios to the floor: {res}", flush=True)


@pytest.mark.parametrize("n,t,d", [(32, 1024, 2048), (19, 600, 1024)])
def test_32_row_tile_in_fp32(n, t, d):
    """fp32 rows take the four-wave 32-row tile at D=2048 (512 chunks) and the
    two-wave one at D=1024; bar: the reference's fp32 tolerance."""
    tile = (4, 2, 32) if d == 2048 else (2, 2, 32)
    assert _tile(_lib.OP_BWD, n, d, torch.float32, t) == ("resident", tile)
    gen = torch.Generator().manual_seed(n)
    v = torch.randn(n, 1, t, d, generator=gen)
    w = 0.5 * torch.randn(d, generator=gen)
    g = torch.randn(1, t, d, generator=gen)
    vv, ww = v.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    out = block_attn_res_hip(vv, ww)
    out.backward(g.to(DEV))
    v64 = v.double()[:, 0].numpy()
    ro = torch.from_numpy(c_oracle.forward(v64, w.double().numpy()))
    rdv, rdw = c_oracle.backward(v64, w.double().numpy(), g.double()[0].numpy())
    assert rel_l2(out.detach()[0].cpu(), ro) <= 1e-6
    assert rel_l2(vv.grad[:, 0].cpu(), torch.from_numpy(rdv)) <= 1e-5
    assert rel_l2(ww.grad.cpu(), torch.from_numpy(rdw)) <= 1e-5


TALLER_CASES = [
    # 32 < N <= 64: the 64-row backward tile (a per-layer AttnRes model's
    # readout sees n_blocks + 1 sources), in each dtype, partly filled at N=33
    ((33, 600, 2048), torch.bfloat16, (4, 1, 64)),
    ((64, 300, 1024), torch.float16, (2, 1, 64)),
    ((48, 256, 1024), torch.float32, (4, 1, 64)),
]


@pytest.mark.parametrize("shape,dtype,tile", TALLER_CASES, ids=lambda x: str(x))
def test_64_row_backward_tile(shape, dtype, tile):
    """The 64-row tile against the float64 C oracle (16-bit at the 1.10x floor,
    fp32 at 1e-6 / 1e-5), and bit for bit the same on a second run."""
    n, t, d = shape
    print(f"64-row tile N={n} T={t} D={d} {dtype}: expect bwd {tile}", flush=True)
    assert _tile(_lib.OP_BWD, n, d, dtype, t) == ("resident", tile)
    gen = torch.Generator().manual_seed(n + t)
    v = torch.randn(n, 1, t, d, generator=gen).to(dtype)
    w = (0.5 * torch.randn(d, generator=gen)).to(dtype)
    g = torch.randn(1, t, d, generator=gen).to(dtype)
    runs = []
    for _ in range(2):
        vv, ww = v.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
        out = block_attn_res_hip(vv, ww)
        out.backward(g.to(DEV))
        runs.append((out.detach().cpu(), vv.grad.cpu(), ww.grad.cpu()))
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    out, dv, dw = runs[0]
    v64 = v.double()[:, 0].numpy()
    ro = torch.from_numpy(c_oracle.forward(v64, w.double().numpy()))
    rdv, rdw = c_oracle.backward(v64, w.double().numpy(), g.double()[0].numpy())
    for name, got, ref, bar in (("out", out[0], ro, 1e-6), ("dv", dv[:, 0], torch.from_numpy(rdv), 1e-5),
                                ("dw", dw, torch.from_numpy(rdw), 1e-5)):
        err = rel_l2(got, ref)
        if dtype != torch.float32:
            bar = 1.10 * dtype_floor(ref, dtype)
        assert err <= bar, f"{name}: rel_l2 {err:.4e} vs {bar:.4e}"


EIGHT_WAVE_CASES = [
    # rows of 2048 chunks, covered only by eight waves of four chunks: fp32
    # D=8192 (the d-sweep's B=1 shape, 9 rows; and 4 rows) and 16-bit D=16384
    ((9, 768, 8192), torch.float32, (8, 4, 9)),
    ((4, 600, 8192), torch.float32, (8, 4, 4)),
    ((3, 600, 16384), torch.bfloat16, (8, 4, 4)),
    # 16-bit rows with 9 rows: w and grad_out kept packed (spills remain)
    ((9, 560, 16384), torch.bfloat16, (8, 4, 9)),
    ((6, 600, 16384), torch.float16, (8, 4, 9)),
]


@pytest.mark.parametrize("shape,dtype,tile", EIGHT_WAVE_CASES, ids=lambda x: str(x))
def test_eight_wave_backward_tiles(shape, dtype, tile):
    """The eight-wave four-chunk backward (two waves a SIMD) against the
    float64 C oracle: fp32 at the reference's fp32 bars (1e-6 forward, 1e-5
    gradients), 16-bit at the 1.10x floor."""
    n, t, d = shape
    print(f"eight-wave tile N={n} T={t} D={d} {dtype}: expect bwd {tile}", flush=True)
    assert _tile(_lib.OP_BWD, n, d, dtype, t) == ("resident", tile)
    if dtype != torch.float32:
        _check(n, 1, t, d, dtype, seed=7)
        return
    gen = torch.Generator().manual_seed(n + d)
    v = torch.randn(n, 1, t, d, generator=gen)
    w = 0.5 * torch.randn(d, generator=gen)
    g = torch.randn(1, t, d, generator=gen)
    vv, ww = v.to(DEV).requires_grad_(True), w.to(DEV).requires_grad_(True)
    out = block_attn_res_hip(vv, ww)
    out.backward(g.to(DEV))
    v64 = v.double()[:, 0].numpy()
    ro = torch.from_numpy(c_oracle.forward(v64, w.double().numpy()))
    rdv, rdw = c_oracle.backward(v64, w.double().numpy(), g.double()[0].numpy())
    assert rel_l2(out.detach()[0].cpu(), ro) <= 1e-6
    assert rel_l2(vv.grad[:, 0].cpu(), torch.from_numpy(rdv)) <= 1e-5
    assert rel_l2(ww.grad.cpu(), torch.from_numpy(rdw)) <= 1e-5


def test_fp32_d8192_backward_without_stats_stays_generic():
    """Without the forward's stats the 9-row eight-wave tile would spill over
    100 VGPRs, so that call runs the generic kernel, inside the workspace the
    query sizes (its grid and the tile's), at the fp32 bar."""
    import ctypes

    n, t, d = 9, 600, 8192
    gen = torch.Generator().manual_seed(11)
    v = torch.randn(n, 1, t, d, generator=gen)
    w = 0.5 * torch.randn(d, generator=gen)
    g = torch.randn(1, t, d, generator=gen)
    lib, code = _lib.lib(), _lib.dtype_code(torch.float32)
    vd, wd, gd = v.to(DEV), w.to(DEV), g.to(DEV)
    ws_bytes = lib.sy_bwd_workspace_bytes(n, t, d, code, code)
    assert ws_bytes >= lib.sy_bwd_partial_rows(n, t, d, code, code, 1, 0) * d * 4
    assert ws_bytes >= lib.sy_bwd_partial_rows(n, t, d, code, code, 1, 1) * d * 4
    ws = torch.empty(ws_bytes // 4, device=DEV)
    dv, dw = torch.empty_like(vd), torch.empty(d, device=DEV)
    P = ctypes.c_void_p
    rc = lib.sy_bwd(P(vd.data_ptr()), P(wd.data_ptr()), P(gd.data_ptr()), None, P(dv.data_ptr()),
                    P(dw.data_ptr()), P(ws.data_ptr()), ws_bytes, n, t, d, t * d, code, code, 1e-6,
                    _lib.stream_ptr(vd.device))
    assert rc == 0
    torch.cuda.synchronize()
    v64 = v.double()[:, 0].numpy()
    rdv, rdw = c_oracle.backward(v64, w.double().numpy(), g.double()[0].numpy())
    assert rel_l2(dv[:, 0].cpu(), torch.from_numpy(rdv)) <= 1e-5
    assert rel_l2(dw.cpu(), torch.from_numpy(rdw)) <= 1e-5


def test_32_row_tile_is_bitwise_deterministic_and_other_callers_fall_back():
    """Two runs give the same bits; without the forward's stats the backward
    at N > 16 runs the generic kernel and still matches."""
    import ctypes

    n, t, d = 24, 3 * CUS, 2048
    gen = torch.Generator().manual_seed(3)
    v = torch.randn(n, 1, t, d, generator=gen).to(torch.bfloat16).to(DEV)
    w = (0.5 * torch.randn(d, generator=gen)).to(torch.bfloat16).to(DEV)
    g = torch.randn(1, t, d, generator=gen).to(torch.bfloat16).to(DEV)
    grads = []
    for _ in range(2):
        vv, ww = v.clone().requires_grad_(True), w.clone().requires_grad_(True)
        block_attn_res_hip(vv, ww).backward(g)
        grads.append((vv.grad, ww.grad))
    assert torch.equal(grads[0][0], grads[1][0]) and torch.equal(grads[0][1], grads[1][1])
    lib, code = _lib.lib(), _lib.dtype_code(torch.bfloat16)
    ws_bytes = lib.sy_bwd_workspace_bytes(n, t, d, code, code)
    ws = torch.empty(ws_bytes // 4, device=DEV)
    dv, dw = torch.empty_like(v), torch.empty(d, device=DEV, dtype=torch.bfloat16)
    P = ctypes.c_void_p
    rc = lib.sy_bwd(P(v.data_ptr()), P(w.data_ptr()), P(g.data_ptr()), None, P(dv.data_ptr()), P(dw.data_ptr()),
                    P(ws.data_ptr()), ws_bytes, n, t, d, t * d, code, code, 1e-6, _lib.stream_ptr(v.device))
    assert rc == 0
    torch.cuda.synchronize()
    for got, ref in ((dv, grads[0][0]), (dw, grads[0][1])):
        assert rel_l2(got.cpu(), ref.cpu()) <= 1e-2  # two bf16 roundings of the same values
    v64 = v.double()[:, 0].cpu().numpy()
    rdv, rdw = c_oracle.backward(v64, w.double().cpu().numpy(), g.double()[0].cpu().numpy())
    for got, ref in ((dv[:, 0], torch.from_numpy(rdv)), (dw, torch.from_numpy(rdw))):
        assert rel_l2(got.cpu(), ref) <= 1.10 * dtype_floor(ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("n_q,family", [(1, "resident"), (2, "resident"), (4, "matrix"), (16, "matrix")])
def test_query_sweep_shapes_at_the_oracle_floor(n_q, family, dtype):
    """The batched forward at the query-sweep counts (the config-3 sweep's
    Q = 1, 2, 4, 16 next to Q = 8) on the plan the sweep times, against the
    float64 C oracle at the 1.10x floor."""
    from switchyard.triton_op import block_attn_res_batched

    n, t, d = 9, 4 * CUS, 2048
    assert _lib.plan(_lib.OP_BATCHED, n, d, dtype, n_q=n_q)["family_name"] == family
    gen = torch.Generator().manual_seed(40 + n_q)
    v = torch.randn(n, 1, t, d, generator=gen).to(dtype)
    q = (0.5 * torch.randn(n_q, d, generator=gen)).to(dtype)
    got = block_attn_res_batched(v.to(DEV), q.to(DEV)).reshape(n_q, t, d).cpu()
    ref = torch.from_numpy(c_oracle.batched(v.double()[:, 0].numpy(), q.double().numpy()))
    for i in range(n_q):
        err, floor = rel_l2(got[i], ref[i]), dtype_floor(ref[i], dtype)
        assert err <= 1.10 * floor, f"query {i}: rel_l2 {err:.4e} vs floor {floor:.4e}"


#: The reference's eight-query shape checks of the batched forward
#: (docs/batched_queries.md:27-34) as (N, B, T, D) and the family each
#: launches on MI355X: the matrix cores everywhere, with eight waves of 512
#: columns per token at D = 4096.
EIGHT_QUERY_SHAPES = [((2, 1, 4096, 2048), "matrix"), ((16, 1, 4096, 2048), "matrix"),
                      ((9, 1, 4096, 1024), "matrix"), ((9, 1, 128, 1024), "matrix"),
                      ((9, 4, 2048, 2048), "matrix"), ((9, 1, 4096, 4096), "matrix")]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("shape,family", EIGHT_QUERY_SHAPES, ids=lambda x: str(x))
def test_eight_query_shape_checks_at_the_oracle_floor(shape, family, dtype):
    """Eight queries at each of the reference's shape checks, on the family the
    sweep times, against the float64 C oracle at the 1.10x floor. Tokens are
    independent, so the oracle runs on a slice of 256 tokens (the first and
    last 128) of the full-size launch."""
    from switchyard.triton_op import block_attn_res_batched

    n, b, t, d = shape
    n_q = 8
    print(f"eight-query shape N{n} B{b} T{t} D{d} {dtype}", flush=True)
    assert _lib.plan(_lib.OP_BATCHED, n, d, dtype, n_q=n_q)["family_name"] == family
    gen = torch.Generator().manual_seed(n + t + d)
    v = torch.randn(n, b, t, d, generator=gen).to(dtype)
    q = (0.5 * torch.randn(n_q, d, generator=gen)).to(dtype)
    got = block_attn_res_batched(v.to(DEV), q.to(DEV)).reshape(n_q, b * t, d).cpu()
    flat = v.reshape(n, b * t, d)
    pick = torch.cat([torch.arange(0, min(128, b * t)), torch.arange(max(128, b * t - 128), b * t)])
    ref = torch.from_numpy(c_oracle.batched(flat[:, pick].double().numpy(), q.double().numpy()))
    for i in range(n_q):
        err, floor = rel_l2(got[i, pick], ref[i]), dtype_floor(ref[i], dtype)
        assert err <= 1.10 * floor, f"query {i}: rel_l2 {err:.4e} vs floor {floor:.4e}"


@pytest.mark.parametrize("t", [1, 3, 4 * CUS + 5])
@pytest.mark.parametrize("n_q", [4, 16])
def test_matrix_batched_forward_at_d4096_ragged(t, n_q):
    """The eight-wave D = 4096 matrix-core tile at token counts below, at and
    past the grid (an idle workgroup, a ragged last round), with 4 and 16
    queries and 1-9 sources, including the statistics outputs."""
    from switchyard.stats_op import block_attn_res_batched_with_stats
    from switchyard.triton_op import block_attn_res_batched

    d = 4096
    for n in (1, 5, 9):
        print(f"D=4096 matrix N{n} T{t} Q{n_q}", flush=True)
        assert _lib.plan(_lib.OP_BATCHED, n, d, torch.bfloat16, n_q=n_q)["family_name"] == "matrix"
        gen = torch.Generator().manual_seed(7 * n + t)
        v = torch.randn(n, 1, t, d, generator=gen).to(torch.bfloat16)
        q = (0.5 * torch.randn(n_q, d, generator=gen)).to(torch.bfloat16)
        got = block_attn_res_batched(v.to(DEV), q.to(DEV)).reshape(n_q, t, d).cpu()
        o, m, ell = block_attn_res_batched_with_stats(v.to(DEV), q.to(DEV))
        ref = torch.from_numpy(c_oracle.batched(v.double()[:, 0].numpy(), q.double().numpy()))
        v64 = v.double()[:, 0].numpy()
        r = 1.0 / np.sqrt((v64**2).mean(-1) + 1e-6)  # [n, t]
        for i in range(n_q):
            assert rel_l2(got[i], ref[i]) <= 1.10 * dtype_floor(ref[i], torch.bfloat16), (n, i)
            ro, rm, rl = c_oracle.attn_with_stats(v64, q[i].double().numpy())
            assert rel_l2(o[i].reshape(t, d).cpu(), torch.from_numpy(ro)) <= 1.10 * dtype_floor(
                torch.from_numpy(ro), torch.bfloat16), (n, i)
            # m is a logit, a dot product over D that may cancel to far below
            # its terms: 1e-5 relative plus 2**-20 of the terms' absolute sum
            terms = ((np.abs(v64) @ np.abs(q[i].double().numpy())) * r).max(0)
            dm = np.linalg.norm(m[i].reshape(t).cpu().double().numpy() - rm)
            assert dm <= 1e-5 * np.linalg.norm(rm) + 2.0**-20 * np.linalg.norm(terms), (n, i)
            assert rel_l2(ell[i].reshape(t).cpu(), torch.from_numpy(rl)) <= 1e-5
