"""The forward + backward step captured into a HIP graph (GPU), as the sweeps'
device-only times capture it (`switchyard.harness.time_graph`): `sy_fwd` with
statistics, then `sy_bwd` from them, on a side stream. Each replay runs on
fresh inputs copied into the captured buffers, with eager work of the same
operator between replays, and must equal an eager step bit for bit (out, dv,
dw). Shapes: config 2's tile at 4 tokens per CU and a token-count-rule tile
(two tokens per CU, D=1024), plus the batched forward's two-slot kernel.
"""

from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from switchyard import _lib  # noqa: E402

DEV = torch.device("cuda")
CUS = torch.cuda.get_device_properties(0).multi_processor_count
P = ctypes.c_void_p


def _inputs(n, t, d, seed):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, 1, t, d, generator=g).to(torch.bfloat16).to(DEV)
    w = (0.5 * torch.randn(d, generator=g)).to(torch.bfloat16).to(DEV)
    go = torch.randn(1, t, d, generator=g).to(torch.bfloat16).to(DEV)
    return v, w, go


class _Step:
    """Buffers and the two C-ABI calls of one step on a given stream."""

    def __init__(self, n, t, d):
        lib = _lib.lib()
        self.n, self.t, self.d, self.lib = n, t, d, lib
        self.v, self.w, self.go = _inputs(n, t, d, 0)
        self.out = torch.empty(1, t, d, device=DEV, dtype=torch.bfloat16)
        self.stats = torch.empty(2, n, t, device=DEV)
        self.dv = torch.empty_like(self.v)
        self.dw = torch.empty(d, device=DEV, dtype=torch.bfloat16)
        self.ws_bytes = int(lib.sy_bwd_workspace_bytes(n, t, d, _lib.SY_BF16, _lib.SY_BF16))
        self.ws = torch.empty(max(1, self.ws_bytes // 4), device=DEV)

    def run(self, stream):
        n, t, d, lib, bf = self.n, self.t, self.d, self.lib, _lib.SY_BF16
        s = P(stream.cuda_stream)
        assert lib.sy_fwd(P(self.v.data_ptr()), P(self.w.data_ptr()), P(self.out.data_ptr()),
                          P(self.stats.data_ptr()), n, t, d, t * d, bf, bf, 1e-6, s) == 0
        assert lib.sy_bwd(P(self.v.data_ptr()), P(self.w.data_ptr()), P(self.go.data_ptr()),
                          P(self.stats.data_ptr()), P(self.dv.data_ptr()), P(self.dw.data_ptr()),
                          P(self.ws.data_ptr()), self.ws_bytes, n, t, d, t * d, bf, bf, 1e-6, s) == 0

    def results(self):
        return self.out.clone(), self.dv.clone(), self.dw.clone()


@pytest.mark.parametrize("n,t,d", [(9, 4 * CUS, 2048), (9, 2 * CUS, 1024), (4, 333, 2048)])
def test_step_replays_from_a_graph_bit_for_bit(n, t, d):
    print(f"graph step N={n} T={t} D={d}", flush=True)
    side = torch.cuda.Stream()
    cap = _Step(n, t, d)
    eager = _Step(n, t, d)
    with torch.cuda.stream(side):
        cap.run(side)  # warm-up outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        cap.run(side)
    for rep in range(3):
        v, w, go = _inputs(n, t, d, 10 + rep)
        cap.v.copy_(v), cap.w.copy_(w), cap.go.copy_(go)
        eager.v.copy_(v), eager.w.copy_(w), eager.go.copy_(go)
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            graph.replay()
        torch.cuda.synchronize()
        eager.run(torch.cuda.current_stream())  # eager work between replays
        torch.cuda.synchronize()
        for a, b, what in zip(cap.results(), eager.results(), ("out", "dv", "dw")):
            assert torch.equal(a, b), f"replay {rep}: {what}"


def test_batched_forward_replays_from_a_graph_bit_for_bit():
    """The two-slot matrix-core batched forward (config 3's kernel) in a graph."""
    n, q, t, d = 9, 8, 4 * CUS + 1, 2048  # an odd token count: the last group's second slot is empty
    lib = _lib.lib()
    side = torch.cuda.Stream()
    g = torch.Generator().manual_seed(3)
    qs = (0.5 * torch.randn(q, d, generator=g)).to(torch.bfloat16).to(DEV)
    v_cap = torch.empty(n, 1, t, d, device=DEV, dtype=torch.bfloat16)
    out_cap = torch.empty(q, 1, t, d, device=DEV, dtype=torch.bfloat16)
    out_eager = torch.empty_like(out_cap)
    assert _lib.plan(_lib.OP_BATCHED, n, d, torch.bfloat16, n_q=q)["family_name"] == "matrix"

    def call(v, out, stream):
        assert lib.sy_fwd_batched(P(v.data_ptr()), P(qs.data_ptr()), P(out.data_ptr()), n, q, t, d, t * d,
                                  _lib.SY_BF16, 1e-6, P(stream.cuda_stream)) == 0

    v_cap.copy_(torch.randn(n, 1, t, d, generator=g).to(torch.bfloat16))
    with torch.cuda.stream(side):
        call(v_cap, out_cap, side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        call(v_cap, out_cap, side)
    for rep in range(3):
        v_cap.copy_(torch.randn(n, 1, t, d, generator=g).to(torch.bfloat16))
        torch.cuda.synchronize()
        with torch.cuda.stream(side):
            graph.replay()
        torch.cuda.synchronize()
        call(v_cap, out_eager, torch.cuda.current_stream())
        torch.cuda.synchronize()
        assert torch.equal(out_cap, out_eager), f"replay {rep}"
