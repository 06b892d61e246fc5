"""The token-count tile rule (GPU). At D = 2048 with at most two tokens per CU
the forward runs (4,1,NR) up to one token per CU and (2,2,NR) up to two
(3 <= N <= 9), the backward (4,1,NR) (N >= 2); the forward over 10-16 rows
keeps four-row chunks on four waves up to three tokens per CU and on two up
to six. fp32 forwards take four waves a token up to one token per CU (10-16
rows: four-row chunks up to two); 16-bit D = 4096 up to one token per CU runs
the forward on four waves of two chunks and the backward on eight of one. Where a wave's row slice is two
chunks a lane (16-bit D = 1024, fp32 D = 512) the backward runs (4,1,NR) up to
two tokens per CU and (2,1,NR) up to four; fp32 rows of four chunks
(D = 1024) take the backward's (4,1,NR) up to two tokens per CU. Above that
the plan's tiles. Each case checks, bit for bit, that the default launch
equals the launch forced onto the expected tile with the measurement override
of sy_tuning_set, and that the result matches the float64 oracle. Token
counts are derived from the device's CU count.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

if not torch.cuda.is_available():  # pragma: no cover
    pytest.skip("needs a HIP device", allow_module_level=True)

from oracle import c_oracle  # noqa: E402
from oracle.reference import dtype_floor, rel_l2  # noqa: E402
from switchyard.hip_op import block_attn_res_hip  # noqa: E402

DEV = "cuda"
CUS = torch.cuda.get_device_properties(0).multi_processor_count


def _run(n, t, d, seed, dtype=torch.bfloat16):
    g = torch.Generator().manual_seed(seed)
    v = torch.randn(n, 1, t, d, generator=g).to(dtype).to(DEV)
    w = (torch.randn(d, generator=g) * 0.5).to(dtype).to(DEV)
    go = torch.randn(1, t, d, generator=g).to(dtype).to(DEV)
    vv, ww = v.clone().requires_grad_(), w.clone().requires_grad_()
    out = block_attn_res_hip(vv, ww)
    out.backward(go)
    torch.cuda.synchronize()
    return (v, w, go), (out.detach(), vv.grad, ww.grad)


@pytest.mark.parametrize("n,per_cu,d,fwd_tile,bwd_tile,dtype", [
    (9, 1, 2048, "4,1,9", "4,1,9", torch.bfloat16),
    (9, 2, 2048, "2,2,9", "4,1,9", torch.bfloat16),
    (9, 2, 2048, "2,2,9", "4,1,9", torch.float16),
    (4, 2, 2048, "2,2,4", "4,1,4", torch.bfloat16),
    (16, 2, 2048, "4,1,4", "4,1,16", torch.bfloat16),
    (12, 3, 2048, "4,1,4", "1,4,16", torch.float16),
    (16, 5, 2048, "2,2,4", "1,4,16", torch.bfloat16),
    (10, 6, 2048, "2,2,4", "1,4,16", torch.bfloat16),
    (16, 8, 2048, "1,4,4", "1,4,16", torch.bfloat16),
    (9, 4, 2048, "1,4,9", "1,4,9", torch.bfloat16),
    (2, 1, 2048, "1,4,4", "4,1,4", torch.bfloat16),
    (2, 4, 2048, "1,4,4", "1,4,4", torch.bfloat16),
    (9, 1, 1024, "1,2,9", "4,1,9", torch.bfloat16),
    (9, 2, 1024, "1,2,9", "4,1,9", torch.float16),
    (16, 2, 1024, "1,2,16", "4,1,16", torch.bfloat16),
    (2, 2, 1024, "1,2,4", "4,1,4", torch.bfloat16),
    (9, 4, 1024, "1,2,9", "2,1,9", torch.bfloat16),
    (4, 4, 1024, "1,2,4", "2,1,4", torch.bfloat16),
    (9, 8, 1024, "1,2,9", "1,2,9", torch.bfloat16),
    (9, 1, 4096, "4,2,9", "8,1,9", torch.bfloat16),
    (4, 1, 4096, "4,2,4", "8,1,4", torch.float16),
    (9, 2, 4096, "2,4,9", "2,4,9", torch.bfloat16),
    (9, 1, 1024, "4,1,9", "4,1,9", torch.float32),
    (9, 1, 2048, "4,2,9", "2,4,9", torch.float32),
    (9, 2, 2048, "2,4,9", "2,4,9", torch.float32),
    (16, 2, 2048, "4,2,4", "2,4,16", torch.float32),
    (4, 2, 1024, "1,4,4", "4,1,4", torch.float32),
    (9, 4, 1024, "1,4,9", "1,4,9", torch.float32),
    (9, 1, 512, "1,2,9", "4,1,9", torch.float32),
    (9, 4, 512, "1,2,9", "2,1,9", torch.float32),
])
def test_default_launch_takes_the_rule_tile(n, per_cu, d, fwd_tile, bwd_tile, dtype):
    from switchyard import _lib

    t = CUS * per_cu
    print(f"token rule N={n} T={t} D={d} {dtype} expect fwd {fwd_tile} bwd {bwd_tile}", flush=True)
    for op, want in ((_lib.OP_FWD, fwd_tile), (_lib.OP_BWD, bwd_tile)):
        p = _lib.plan(op, n, d, dtype, n_tok=t)
        assert (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == tuple(map(int, want.split(",")))
    ins, got = _run(n, t, d, seed=n + per_cu, dtype=dtype)
    with _lib.tuning(fwd_tile=map(int, fwd_tile.split(",")), bwd_tile=map(int, bwd_tile.split(","))):
        _, forced = _run(n, t, d, seed=n + per_cu, dtype=dtype)
    for a, b, what in zip(got, forced, ("out", "dv", "dw")):
        assert torch.equal(a, b), what
    v, w, go = ins
    ro = torch.as_tensor(c_oracle.forward(v[:, 0].double().cpu().numpy(), w.double().cpu().numpy()))
    rdv, rdw = c_oracle.backward(v[:, 0].double().cpu().numpy(), w.double().cpu().numpy(),
                                 go[0].double().cpu().numpy())
    for x, ref, what in ((got[0][0].cpu(), ro, "out"), (got[1][:, 0].cpu(), torch.as_tensor(rdv), "dv"),
                         (got[2].cpu(), torch.as_tensor(rdw), "dw")):
        # fp32: the reference's forward bound and the north-star gradient bound
        bar = (1e-6 if what == "out" else 1e-5) if dtype == torch.float32 else 1.10 * dtype_floor(ref, dtype)
        assert rel_l2(x, ref) <= bar, what


@pytest.mark.parametrize("per_cu,d,fwd_tile,bwd_tile", [
    (1, 2048, (4, 1, 9), (4, 1, 9)), (2, 2048, (2, 2, 9), (4, 1, 9)), (16, 2048, (1, 4, 9), (1, 4, 9)),
    (2, 1024, (1, 2, 9), (4, 1, 9)), (4, 1024, (1, 2, 9), (2, 1, 9)), (16, 1024, (1, 2, 9), (1, 2, 9))])
def test_plan_for_tokens_reports_the_launched_tile(per_cu, d, fwd_tile, bwd_tile):
    from switchyard import _lib

    for op, want in ((_lib.OP_FWD, fwd_tile), (_lib.OP_BWD, bwd_tile)):
        p = _lib.plan(op, 9, d, torch.bfloat16, n_tok=CUS * per_cu)
        assert (p["waves_per_token"], p["chunks_per_lane"], p["rows_per_tile"]) == want
