"""Robustness of ``sy_bwd`` (GPU): its workspace may hold arbitrary bytes, one
workspace may serve back-to-back calls, the persistent grid may be smaller
than the reduction's 16 row groups, and a captured HIP graph of the backward
(main kernel + dw reduction) must replay correctly on fresh inputs, with eager
work between replays. In every case dv and dw must equal, bit for bit, the
staged path (``sy_bwd_main`` + ``sy_dw_reduce``) and dw must match the float64
oracle.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from oracle import c_oracle  # noqa: E402
from oracle.reference import dtype_floor, rel_l2  # noqa: E402
from switchyard import _lib  # noqa: E402

DEV = "cuda"
P = ctypes.c_void_p


def _inputs(n, t, d, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, 1, t, d, generator=g).to(dtype).to(DEV)
    w = (torch.randn(d, generator=g) * 0.5).to(dtype).to(DEV)
    go = torch.randn(1, t, d, generator=g).to(dtype).to(DEV)
    return v, w, go


def _bwd(v, w, go, ws, stats=None):
    lib = _lib.lib()
    n, _, t, d = v.shape
    code = _lib.dtype_code(v.dtype)
    dv = torch.empty_like(v)
    dw = torch.empty(d, device=DEV, dtype=w.dtype)
    rc = lib.sy_bwd(P(v.data_ptr()), P(w.data_ptr()), P(go.data_ptr()),
                    None if stats is None else P(stats.data_ptr()), P(dv.data_ptr()), P(dw.data_ptr()),
                    P(ws.data_ptr()), ws.numel() * ws.element_size(), n, t, d, t * d, code, code, 1e-6,
                    _lib.stream_ptr(v.device))
    assert rc == 0
    return dv, dw


def _staged(v, w, go, stats=None):
    lib = _lib.lib()
    n, _, t, d = v.shape
    code = _lib.dtype_code(v.dtype)
    ws_bytes = lib.sy_bwd_workspace_bytes(n, t, d, code, code)
    ws = torch.empty(ws_bytes // 4, device=DEV)
    dv = torch.empty_like(v)
    dw = torch.empty(d, device=DEV, dtype=w.dtype)
    st = _lib.stream_ptr(v.device)
    rc = lib.sy_bwd_main(P(v.data_ptr()), P(w.data_ptr()), P(go.data_ptr()),
                         None if stats is None else P(stats.data_ptr()), P(dv.data_ptr()), P(ws.data_ptr()),
                         ws_bytes, n, t, d, t * d, code, code, 1e-6, st)
    assert rc == 0
    rows = lib.sy_bwd_partial_rows(n, t, d, code, code, 1, int(stats is not None))
    assert lib.sy_dw_reduce(P(ws.data_ptr()), rows, d, P(dw.data_ptr()), code, st) == 0
    return dv, dw


def _workspace(n, t, d, dtype, fill=None):
    code = _lib.dtype_code(dtype)
    nbytes = _lib.lib().sy_bwd_workspace_bytes(n, t, d, code, code)
    ws = torch.empty(nbytes // 4, device=DEV)
    if fill == "garbage":  # arbitrary bytes
        ws.view(torch.int32).copy_(torch.randint(-2**31, 2**31 - 1, (ws.numel(),), dtype=torch.int32))
    elif fill == "ones":
        ws.fill_(1.0)
    return ws


@pytest.mark.parametrize("fill", [None, "garbage", "ones"])
@pytest.mark.parametrize("shape", [(9, 4096, 2048), (9, 1000, 2048), (4, 333, 1024), (9, 37, 2048),
                                   (2, 5, 512), (9, 1, 2048), (3, 1000, 2048), (2, 777, 4096)])
def test_backward_equals_the_staged_path_whatever_the_workspace_holds(shape, fill):
    n, t, d = shape
    print(f"sy_bwd {shape} workspace {fill}", flush=True)
    v, w, go = _inputs(n, t, d, seed=t)
    ws = _workspace(n, t, d, v.dtype, fill)
    dv, dw = _bwd(v, w, go, ws)
    sdv, sdw = _staged(v, w, go)
    assert torch.equal(dv, sdv)
    assert torch.equal(dw, sdw)
    rdv, rdw = c_oracle.backward(v[:, 0].double().cpu().numpy(), w.double().cpu().numpy(),
                                 go[0].double().cpu().numpy())
    rdw = torch.from_numpy(rdw)
    assert rel_l2(dw.cpu(), rdw) <= 1.10 * dtype_floor(rdw, torch.bfloat16)


def test_back_to_back_calls_on_one_workspace():
    v, w, go = _inputs(9, 2048, 2048, seed=1)
    ws = _workspace(9, 2048, 2048, v.dtype, "garbage")
    ref = _staged(v, w, go)[1]
    dws = [_bwd(v, w, go, ws)[1] for _ in range(8)]
    torch.cuda.synchronize()
    for dw in dws:
        assert torch.equal(dw, ref)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_graph_replays_match_eager(dtype):
    """Capture one backward into a HIP graph and replay it on fresh inputs, with
    eager work and a synchronisation between replays; every replay must equal
    the eager result."""
    n, t, d = 9, 1024, 2048
    v, w, go = _inputs(n, t, d, dtype, seed=5)
    ws = _workspace(n, t, d, dtype, "garbage")
    sv, sw, sg = v.clone(), w.clone(), go.clone()
    dv = torch.empty_like(v)
    dw = torch.empty(d, device=DEV, dtype=dtype)
    code = _lib.dtype_code(dtype)
    lib = _lib.lib()

    def launch():
        rc = lib.sy_bwd(P(sv.data_ptr()), P(sw.data_ptr()), P(sg.data_ptr()), None, P(dv.data_ptr()),
                        P(dw.data_ptr()), P(ws.data_ptr()), ws.numel() * 4, n, t, d, t * d, code, code,
                        1e-6, _lib.stream_ptr(sv.device))
        assert rc == 0

    launch()  # warm up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for rep in range(4):
        nv, nw, ng = _inputs(n, t, d, dtype, seed=100 + rep)
        sv.copy_(nv)
        sw.copy_(nw)
        sg.copy_(ng)
        graph.replay()
        torch.cuda.synchronize()
        edv, edw = _staged(nv, nw, ng)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(dv, edv), f"replay {rep}: dv"
        assert torch.equal(dw, edw), f"replay {rep}: dw"


def test_misaligned_buffers_fit_the_queried_workspace():
    """v and dv one element past 16-byte alignment run the generic backward,
    whose grid is capped to the partial rows sy_bwd_workspace_bytes sizes for
    the vector plans; dv and dw still match the float64 oracle."""
    n, t, d = 9, 1000, 2048
    lib = _lib.lib()
    v, w, go = _inputs(n, t, d, seed=11)
    vbuf = torch.empty(v.numel() + 1, device=DEV, dtype=v.dtype)
    vm = vbuf[1:].view(v.shape)
    vm.copy_(v)
    dvbuf = torch.empty_like(vbuf)
    dv = dvbuf[1:].view(v.shape)
    dw = torch.empty(d, device=DEV, dtype=w.dtype)
    code = _lib.dtype_code(v.dtype)
    ws = _workspace(n, t, d, v.dtype)
    rows_vec = lib.sy_bwd_partial_rows(n, t, d, code, code, 1, 0)
    rows_generic = lib.sy_bwd_partial_rows(n, t, d, code, code, 0, 0)
    assert 1 <= rows_generic <= ws.numel() // d and rows_vec <= ws.numel() // d
    rc = lib.sy_bwd(P(vm.data_ptr()), P(w.data_ptr()), P(go.data_ptr()), None, P(dv.data_ptr()),
                    P(dw.data_ptr()), P(ws.data_ptr()), ws.numel() * 4, n, t, d, t * d, code, code, 1e-6,
                    _lib.stream_ptr(v.device))
    assert rc == 0
    torch.cuda.synchronize()
    rdv, rdw = c_oracle.backward(v[:, 0].double().cpu().numpy(), w.double().cpu().numpy(),
                                 go[0].double().cpu().numpy())
    for got, ref, what in ((dv[:, 0].cpu(), rdv, "dv"), (dw.cpu(), rdw, "dw")):
        ref = torch.as_tensor(ref)
        err = rel_l2(got, ref)
        assert err <= 1.10 * dtype_floor(ref, torch.bfloat16), f"{what}: rel_l2 {err:.3e}"
