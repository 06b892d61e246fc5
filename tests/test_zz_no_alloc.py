"""sy_bwd_static, the backward that allocates nothing (GPU).

It runs the same kernels on the same grid as sy_bwd, with the dw partial rows
in the library's static per-GPU array instead of a caller workspace, so its dv
and dw must equal sy_bwd's bit for bit -- on two calls in a row, the second
with a smaller input (the array keeps the first call's rows), and on replays
of a HIP graph that captured it. Calls after the first allocate no device
memory, and a shape whose partial rows do not fit the array is refused.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from switchyard import _lib  # noqa: E402

DEV = "cuda"
P = ctypes.c_void_p
WORKSPACE = -4
STATIC_BYTES = 8 << 20


def _case(n, t, d, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, 1, t, d, generator=g).to(dtype).to(DEV)
    w = (0.5 * torch.randn(d, generator=g)).to(dtype).to(DEV)
    go = torch.randn(1, t, d, generator=g).to(dtype).to(DEV)
    stats = torch.empty(2, n, t, device=DEV, dtype=torch.float32)
    out = torch.empty(1, t, d, device=DEV, dtype=dtype)
    code = _lib.dtype_code(dtype)
    rc = _lib.lib().sy_fwd(P(v.data_ptr()), P(w.data_ptr()), P(out.data_ptr()), P(stats.data_ptr()), n, t, d,
                           t * d, code, code, 1e-6, _lib.stream_ptr(v.device))
    assert rc == 0
    return v, w, go, stats


def _with_workspace(v, w, go, stats):
    n, _, t, d = v.shape
    code = _lib.dtype_code(v.dtype)
    lib = _lib.lib()
    nbytes = lib.sy_bwd_workspace_bytes(n, t, d, code, code)
    ws = torch.empty(max(1, nbytes // 4), device=DEV, dtype=torch.float32)
    dv, dw = torch.empty_like(v), torch.empty(d, device=DEV, dtype=w.dtype)
    rc = lib.sy_bwd(P(v.data_ptr()), P(w.data_ptr()), P(go.data_ptr()), P(stats.data_ptr()), P(dv.data_ptr()),
                    P(dw.data_ptr()), P(ws.data_ptr()), nbytes, n, t, d, t * d, code, code, 1e-6,
                    _lib.stream_ptr(v.device))
    assert rc == 0
    return dv, dw


def _static(v, w, go, stats):
    n, _, t, d = v.shape
    code = _lib.dtype_code(v.dtype)
    dv, dw = torch.empty_like(v), torch.empty(d, device=DEV, dtype=w.dtype)
    rc = _lib.lib().sy_bwd_static(P(v.data_ptr()), P(w.data_ptr()), P(go.data_ptr()), P(stats.data_ptr()),
                                  P(dv.data_ptr()), P(dw.data_ptr()), n, t, d, t * d, code, code, 1e-6,
                                  _lib.stream_ptr(v.device))
    return rc, dv, dw


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_static_backward_equals_the_workspace_backward_on_two_calls(dtype):
    for n, t, d, seed in ((9, 4096, 2048, 1), (4, 333, 1024, 2)):  # the second call is smaller
        print(f"sy_bwd_static N={n} T={t} D={d} {dtype}", flush=True)
        ins = _case(n, t, d, dtype, seed)
        rc, dv, dw = _static(*ins)
        assert rc == 0
        rdv, rdw = _with_workspace(*ins)
        torch.cuda.synchronize()
        assert torch.equal(dv, rdv)
        assert torch.equal(dw, rdw)


def test_static_backward_refuses_a_shape_beyond_its_array():
    n, t, d = 9, 4096, 16384  # the generic kernel: 1024 partial rows of 64 KiB
    code = _lib.dtype_code(torch.bfloat16)
    need = _lib.lib().sy_bwd_workspace_bytes(n, t, d, code, code)
    print(f"sy_bwd_static refusal: needs {need} bytes", flush=True)
    if need <= STATIC_BYTES:
        pytest.skip(f"this device's grid needs only {need} bytes at D={d}")
    # The size check comes before any device work. Real buffers of the full
    # shape all the same (2.5 GB), so that a check moved after a launch would
    # read and write valid memory and show up as a wrong return code here.
    v = torch.zeros(n, 1, t, d, device=DEV, dtype=torch.bfloat16)
    w = torch.zeros(d, device=DEV, dtype=torch.bfloat16)
    go = torch.zeros(1, t, d, device=DEV, dtype=torch.bfloat16)
    dv, dw = torch.empty_like(v), torch.full((d,), 7.0, device=DEV, dtype=torch.bfloat16)
    rc = _lib.lib().sy_bwd_static(P(v.data_ptr()), P(w.data_ptr()), P(go.data_ptr()), None, P(dv.data_ptr()),
                                  P(dw.data_ptr()), n, t, d, t * d, code, code, 1e-6,
                                  _lib.stream_ptr(torch.device(DEV)))
    assert rc == WORKSPACE
    torch.cuda.synchronize()
    assert bool((dw == 7.0).all())  # nothing ran


def test_static_backward_allocates_nothing_and_replays_in_a_graph():
    """After a first call (which resolves the array's address), further calls
    leave torch's allocator and the device's free memory where they were; one
    call captured into a HIP graph replays to sy_bwd's bits on fresh inputs,
    with eager work between replays."""
    n, t, d, dtype = 9, 2048, 2048, torch.bfloat16
    v, w, go, stats = _case(n, t, d, dtype, 7)
    sv, sw, sg, sst = v.clone(), w.clone(), go.clone(), stats.clone()
    dv, dw = torch.empty_like(v), torch.empty(d, device=DEV, dtype=dtype)
    code = _lib.dtype_code(dtype)
    lib = _lib.lib()

    def launch():
        rc = lib.sy_bwd_static(P(sv.data_ptr()), P(sw.data_ptr()), P(sg.data_ptr()), P(sst.data_ptr()),
                               P(dv.data_ptr()), P(dw.data_ptr()), n, t, d, t * d, code, code, 1e-6,
                               _lib.stream_ptr(sv.device))
        assert rc == 0

    launch()
    torch.cuda.synchronize()
    before = (torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0])
    for _ in range(3):
        launch()
    torch.cuda.synchronize()
    assert (torch.cuda.memory_allocated(), torch.cuda.mem_get_info()[0]) == before
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for rep in range(3):
        nv, nw, ng, nst = _case(n, t, d, dtype, 50 + rep)
        sv.copy_(nv)
        sw.copy_(nw)
        sg.copy_(ng)
        sst.copy_(nst)
        graph.replay()
        torch.cuda.synchronize()
        rdv, rdw = _with_workspace(nv, nw, ng, nst)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(dv, rdv), f"replay {rep}: dv"
        assert torch.equal(dw, rdw), f"replay {rep}: dw"
