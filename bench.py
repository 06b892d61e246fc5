#!/usr/bin/env python3
"""Block AttnRes on one MI355X: fwd and fwd+bwd time and HBM roofline fraction.

Workload (the one its metric is quoted on): N=9
sources, B=1, T=4096, D=2048, bf16; v ~ N(0,1), w ~ N(0, 0.5) (std 0.5),
grad_out ~ N(0,1), eps 1e-6. Inputs are generated on the CPU (seed 0),
rounded to bf16 and copied to HBM before anything is timed.

A *step* is one forward + backward of the operator on one batch: sy_fwd
(1 kernel) then sy_bwd (2 kernels: the persistent backward and the dw
reduction), called through the C ABI on torch's current stream. The timed
region is exactly ``--steps`` steps between two synchronizes, cycling through
``--rotations`` independent input/output sets (6 x 330 MiB, far beyond the
256 MiB Infinity Cache) so no step finds its operands cached.

``value`` = algorithmic fwd+bwd bytes ((3N+2) slabs of B*T*D*2 bytes) per
second over the timed region, whole job (one GPU). ``roofline`` is for the
dominant kernel (the backward: (2N+1) slabs per launch), timed live over
``--steps`` back-to-back launches with HIP events on the launch stream.
``cpu_baseline`` times the oracle's eager fp32 formulation (forward +
backward through torch.autograd) on the host cores.

Modes:
  python bench.py [--steps K --warmup W]        the JSON line (stdout)
  python bench.py --kernel {fwd,bwd,reduce,sol,copy} --iters K
                                                run one kernel K times (for rocprofv3)
  python bench.py --summarize DIR --title T     rocprofv3 CSV -> markdown summary
  python bench.py --sweep                       BASELINE configs 3-4: batched Q=8 and the
                                                N / T / D sweeps (fwd, fwd+bwd), JSON lines
  python bench.py --model [--model-scale S]     config 5: decoder training step, standard vs
                                                AttnRes (framework) vs AttnRes (HIP), JSON line
  python bench.py --traffic FETCH_DIR WRITE_DIR --json-out F
                                                rocprofv3 --pmc runs of --kernel all ->
                                                calibrated HBM bytes per launch (JSON)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
for _p in (ROOT / "blackwell-switchyard_amd", ROOT):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

METRIC = "fwd & fwd+bwd ms + % HBM roofline, N=9 B=1 T=4096 D=2048 bf16"
HBM_PEAK_GBPS = 8000.0
TRAFFIC_FILE = ROOT / "profiles" / "traffic_N9_B1_T4096_D2048_bf16.json"


def log(*a) -> None:
    print(*a, file=sys.stderr, flush=True)


def parse_args() -> argparse.Namespace:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--n", type=int, default=9)
    ap.add_argument("--b", type=int, default=1)
    ap.add_argument("--t", type=int, default=4096)
    ap.add_argument("--d", type=int, default=2048)
    ap.add_argument("--dtype", default="bfloat16", choices=["bfloat16", "float16", "float32"])
    ap.add_argument("--w-std", type=float, default=0.5, help="w ~ N(0, w_std); BASELINE.json uses 0.5")
    ap.add_argument("--rotations", type=int, default=6)
    ap.add_argument("--flushed-reps", type=int, default=50, help="reference-style per-rep flushed latency reps")
    ap.add_argument("--cpu-budget-s", type=float, default=15.0)
    ap.add_argument("--check-tokens", type=int, default=512,
                    help="tokens of out/dv the correctness check compares (dw: all tokens)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-extras", action="store_true", help="skip flushed latency, kernel count, memory")
    ap.add_argument("--kernel", choices=["fwd", "bwd", "reduce", "sol", "copy", "all"], default=None)
    ap.add_argument("--iters", type=int, default=20)
    ap.add_argument("--summarize", type=pathlib.Path, default=None)
    ap.add_argument("--title", default="")
    ap.add_argument("--json-out", type=pathlib.Path, default=None)
    ap.add_argument("--quick", action="store_true",
                    help="--schedule / --sweep: a few launches per row and a copy-probe calibration "
                         "launch at the end (a rocprofv3 --pmc target)")
    ap.add_argument("--traffic-set", default="config2",
                    choices=["config2", "schedule", "n32", "n4", "n16", "d8192f32"],
                    help="--traffic: which kernels and workload the counter runs covered (nN: "
                         "bench.py --sweep --sweep-only NN --quick; d8192f32: bench.py --sweep "
                         "--dtype float32 --sweep-only d-sweep-b1 --quick)")
    ap.add_argument("--sweep", action="store_true")
    ap.add_argument("--sweep-only", default=None,
                    help="comma list of sweep names (n-sweep, t-sweep, d-sweep, d-sweep-b1, batch, small, "
                         "batched) or N<n> for that n-sweep shape")
    ap.add_argument("--schedule", action="store_true")
    ap.add_argument("--model", action="store_true")
    ap.add_argument("--model-scale", default="1.3B", choices=["1.3B", "small"])
    ap.add_argument("--model-batch", type=int, default=4)
    ap.add_argument("--model-seq", type=int, default=2048)
    ap.add_argument("--model-reps", type=int, default=10)
    ap.add_argument("--traffic", nargs=2, type=pathlib.Path, default=None, metavar=("FETCH_DIR", "WRITE_DIR"))
    return ap.parse_args()


# ---------------------------------------------------------------------------
# Workload
# ---------------------------------------------------------------------------


class Workload:
    """Rotating HBM-resident input/output sets and C-ABI step closures."""

    def __init__(self, args, torch, device):
        from switchyard import _lib

        self.torch, self.dev, self.lib, self._lib = torch, device, _lib.lib(), _lib
        self.n, self.b, self.t, self.d = args.n, args.b, args.t, args.d
        self.dtype = getattr(torch, args.dtype)
        self.n_tok = self.b * self.t
        self.item = torch.finfo(self.dtype).bits // 8
        self.slab = self.n_tok * self.d * self.item
        gen = torch.Generator().manual_seed(0)
        v = torch.randn(self.n, self.b, self.t, self.d, generator=gen).to(self.dtype)
        w = (args.w_std * torch.randn(self.d, generator=gen)).to(self.dtype)
        g = torch.randn(self.b, self.t, self.d, generator=gen).to(self.dtype)
        self.cpu = (v, w, g)
        self.w = w.to(device)
        vt, gt = v.to(device), g.to(device)
        self.code = _lib.dtype_code(self.dtype)
        self.ws_bytes = int(self.lib.sy_bwd_workspace_bytes(self.n, self.n_tok, self.d, self.code, self.code))
        self.rows = int(self.lib.sy_bwd_partial_rows(self.n, self.n_tok, self.d, self.code, self.code, 1, 1))
        self.sets = []
        for k in range(max(1, args.rotations)):
            s = {
                "v": vt if k == 0 else vt.clone(),
                "g": gt if k == 0 else gt.clone(),
                "out": torch.empty(self.b, self.t, self.d, device=device, dtype=self.dtype),
                "stats": torch.empty(2, self.n, self.n_tok, device=device, dtype=torch.float32),
                "dv": torch.empty(self.n, self.b, self.t, self.d, device=device, dtype=self.dtype),
                "dw": torch.empty(self.d, device=device, dtype=self.dtype),
                "ws": torch.empty(max(1, self.ws_bytes // 4), device=device, dtype=torch.float32),
                "sol": torch.empty(self.b, self.t, self.d, device=device, dtype=self.dtype),
            }
            self.sets.append(s)
        self.stream = _lib.stream_ptr(device)

    @staticmethod
    def _p(t):
        return ctypes.c_void_p(t.data_ptr())

    def _check(self, rc, what):
        self._lib.check(rc, what)

    def fwd(self, s):
        self._check(self.lib.sy_fwd(self._p(s["v"]), self._p(self.w), self._p(s["out"]), self._p(s["stats"]),
                                    self.n, self.n_tok, self.d, self.n_tok * self.d, self.code, self.code,
                                    1e-6, self.stream), "sy_fwd")

    def bwd(self, s):
        self._check(self.lib.sy_bwd(self._p(s["v"]), self._p(self.w), self._p(s["g"]), self._p(s["stats"]),
                                    self._p(s["dv"]), self._p(s["dw"]), self._p(s["ws"]), self.ws_bytes,
                                    self.n, self.n_tok, self.d, self.n_tok * self.d, self.code, self.code,
                                    1e-6, self.stream), "sy_bwd")

    def bwd_main(self, s):
        self._check(self.lib.sy_bwd_main(self._p(s["v"]), self._p(self.w), self._p(s["g"]), self._p(s["stats"]),
                                         self._p(s["dv"]), self._p(s["ws"]), self.ws_bytes, self.n, self.n_tok,
                                         self.d, self.n_tok * self.d, self.code, self.code, 1e-6, self.stream),
                    "sy_bwd_main")

    def reduce(self, s):
        self._check(self.lib.sy_dw_reduce(self._p(s["ws"]), self.rows, self.d, self._p(s["dw"]), self.code,
                                          self.stream), "sy_dw_reduce")

    def sol(self, s):
        self._check(self.lib.sy_sol(self._p(s["v"]), self._p(s["sol"]), self.n, self.n_tok, self.d,
                                    self.n_tok * self.d, self.code, self.stream), "sy_sol")

    def step(self, s):
        self.fwd(s)
        self.bwd(s)

    def closures(self, name):
        f = getattr(self, name)
        return [(lambda s=s: f(s)) for s in self.sets]


# ---------------------------------------------------------------------------
# Reference-style extras (flushed per-rep latency, kernel counts, workspace)
# ---------------------------------------------------------------------------


def api_extras(wl, args, torch, harness):
    from switchyard.hip_op import block_attn_res_hip, speed_of_light

    dev = wl.dev
    v = wl.sets[0]["v"]
    vg = v.detach().clone().requires_grad_(True)
    wg = wl.w.detach().clone().requires_grad_(True)
    g = wl.sets[0]["g"]

    def fwd():
        return block_attn_res_hip(v, wl.w)

    def fwd_bwd():
        vg.grad = None
        wg.grad = None
        block_attn_res_hip(vg, wg).backward(g)

    reps = args.flushed_reps
    out = {
        "method": "autograd API, caches flushed (1 GiB write) before every rep, HIP events, median",
        "fwd": harness.measure_latency(fwd, device=dev, warmup=10, reps=reps).as_dict(),
        "fwd_bwd": harness.measure_latency(fwd_bwd, device=dev, warmup=10, reps=reps).as_dict(),
        "sol": harness.measure_latency(lambda: speed_of_light(v), device=dev, warmup=10, reps=reps).as_dict(),
    }
    try:
        out["fwd_kernels"] = harness.count_kernels(fwd, device=dev).as_dict()
        out["fwd_bwd_kernels"] = harness.count_kernels(fwd_bwd, device=dev).as_dict()
    except Exception as exc:  # noqa: BLE001
        out["kernel_count_error"] = str(exc)[:200]
    resident = v.numel() * v.element_size() + wl.w.numel() * wl.w.element_size() + wl.slab
    out["fwd_memory"] = harness.measure_memory(fwd, device=dev, resident_bytes=resident).as_dict()
    out["fwd_bwd_memory"] = harness.measure_memory(fwd_bwd, device=dev, resident_bytes=resident,
                                                    output_bytes=wl.slab).as_dict()
    return out


# ---------------------------------------------------------------------------
# CPU baseline leg: the only part of bench.py that touches oracle/
# ---------------------------------------------------------------------------


def cpu_baseline_leg(wl, args, torch):
    """Check the timed kernels' own full-size outputs against the float64 C
    oracle, then time the oracle's eager fp32 formulation on the host.

    The checker reruns the timed C-ABI step (``sy_fwd`` + ``sy_bwd`` on
    rotating set 0, the same launch as every timed step) once with
    BASELINE.json's query and once with the reference's unit-norm query
    (bench/bench_operator.py:326-336), and compares the first ``--check-tokens``
    tokens of ``out`` and ``dv`` (tokens are independent, so the oracle on
    those tokens is exact for them) and the full-shape ``dw`` (a sum over every
    token) with the oracle. Bar: 1.10x the dtype rounding floor."""
    import numpy as np

    from oracle import c_oracle
    from oracle import reference as oref
    from switchyard import _lib

    v, w, g = wl.cpu
    ts = min(args.check_tokens, wl.n_tok)
    v64 = v.double().reshape(wl.n, wl.n_tok, wl.d).numpy()
    g64 = g.double().reshape(wl.n_tok, wl.d).numpy()
    s = wl.sets[0]
    oracle_s = []

    def check(wq):
        wl.w = wq.to(wl.dev)
        wl.step(s)  # the timed launch, full size
        torch.cuda.synchronize(wl.dev)
        out = s["out"].reshape(wl.n_tok, wl.d)[:ts].cpu()
        dv = s["dv"].reshape(wl.n, wl.n_tok, wl.d)[:, :ts].cpu()
        dw = s["dw"].cpu()
        t0 = time.perf_counter()
        w64 = wq.double().numpy()
        o_ref = torch.from_numpy(c_oracle.forward(np.ascontiguousarray(v64[:, :ts]), w64))
        _, dw_ref = c_oracle.backward(v64, w64, g64)
        dv_ref, _ = c_oracle.backward(np.ascontiguousarray(v64[:, :ts]), w64, np.ascontiguousarray(g64[:ts]))
        oracle_s.append(time.perf_counter() - t0)
        res = {}
        for name, got, ref in (("out", out, o_ref), ("dv", dv, torch.from_numpy(dv_ref)),
                               ("dw", dw, torch.from_numpy(dw_ref))):
            err, floor = oref.rel_l2(got, ref), oref.dtype_floor(ref, wl.dtype)
            res[name] = {"rel_l2": err, "floor": floor, "ratio": err / floor if floor else None}
        return res

    w_timed = wl.w
    try:
        result = {"what": (f"outputs of the timed sy_fwd + sy_bwd launch at full size (N={wl.n} "
                           f"n_tok={wl.n_tok} D={wl.d}): out and dv on the first {ts} tokens, dw over "
                           "all tokens, against the float64 C oracle"),
                  "tiles": {k: {kk: vv for kk, vv in _lib.plan(op, wl.n, wl.d, wl.dtype, n_tok=wl.n_tok).items()
                                if kk in ("family_name", "waves_per_token", "chunks_per_lane", "rows_per_tile")}
                            for k, op in (("fwd", _lib.OP_FWD), ("bwd", _lib.OP_BWD))},
                  "baseline_query": check(w)}
        wu = torch.randn(wl.d, generator=torch.Generator().manual_seed(1))
        result["unit_norm_query"] = check((wu / wu.norm()).to(wl.dtype))
    finally:
        wl.w = w_timed
    result["ok"] = all(r[k]["ratio"] is not None and r[k]["ratio"] <= 1.10
                       for r in (result["baseline_query"], result["unit_norm_query"])
                       for k in ("out", "dv", "dw"))
    result["oracle_s"] = round(sum(oracle_s), 2)
    check_result = result

    # -- timed CPU baseline ---------------------------------------------------
    threads = torch.get_num_threads()
    v32 = v.float().requires_grad_(True)
    w32 = w.float().requires_grad_(True)
    g32 = g.float()

    def once():
        v32.grad = None
        w32.grad = None
        oref.folded_form(v32, w32, oref.DEFAULT_EPS).backward(g32)

    t0 = time.perf_counter()
    once()  # warmup, also sizes the rep count
    first = time.perf_counter() - t0
    reps = max(1, min(5, int(args.cpu_budget_s / max(first, 1e-3))))
    samples = []
    for _ in range(reps):
        t0 = time.perf_counter()
        once()
        samples.append(time.perf_counter() - t0)
    samples.sort()
    med = samples[len(samples) // 2]
    nbytes = (3 * wl.n + 2) * wl.slab
    cpu = {
        "value": nbytes / med / 1e9,
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"full workload (N={wl.n} B={wl.b} T={wl.t} D={wl.d}), fp32 copies of the bf16 inputs; "
                   f"oracle.reference.folded_form forward + torch.autograd backward; median of {reps} reps "
                   f"after 1 warmup; {med * 1e3:.1f} ms per fwd+bwd"),
        "ms_per_step": med * 1e3,
        "host_cpu": None,
        "host_logical_cpus": os.cpu_count(),
    }
    return check_result, cpu


# ---------------------------------------------------------------------------
# Modes
# ---------------------------------------------------------------------------


def run_kernel_mode(args):
    """Launch kernels --iters times over the rotating sets (rocprofv3 target).
    ``all`` runs fwd, bwd, reduce, sol and the 1 GiB copy probe in turn."""
    import torch

    from switchyard import harness
    from switchyard.hip_op import bandwidth_probe

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    kinds = ["fwd", "bwd", "reduce", "sol", "copy"] if args.kernel == "all" else [args.kernel]
    wl = None
    if any(k != "copy" for k in kinds):
        wl = Workload(args, torch, dev)
        for s in wl.sets:  # stats and partials must exist for bwd / reduce
            wl.fwd(s)
            wl.bwd_main(s)
        torch.cuda.synchronize(dev)
    for kind in kinds:
        if kind == "copy":
            nbytes = 1 << 30
            src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
            dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            ms = harness.time_loop([lambda: bandwidth_probe("copy", src, dst)], device=dev, iters=args.iters)
            log(f"copy: {args.iters} x {nbytes} bytes, {ms * 1e3:.2f} us average")
            del src, dst
            continue
        name = {"fwd": "fwd", "bwd": "bwd_main", "reduce": "reduce", "sol": "sol"}[kind]
        ms = harness.time_loop(wl.closures(name), device=dev, iters=args.iters)
        log(f"{kind}: {args.iters} launches, {ms * 1e3:.2f} us average (HIP events)")


def summarize(args):
    """Condense rocprofv3 CSV output under DIR into a short markdown table."""
    import csv

    d = args.summarize
    stats = sorted(d.rglob("*kernel_stats.csv"))
    counters = sorted(d.rglob("*counter_collection.csv"))
    lines = [f"### {args.title or d.name}", ""]
    for f in stats:
        lines += ["| kernel | calls | avg us | min us | max us |", "|---|---:|---:|---:|---:|"]
        with open(f) as fh:
            for row in csv.DictReader(fh):
                name = row.get("Name") or row.get("KernelName") or "?"
                lines.append(f"| `{name[:90]}` | {row.get('Calls')} | {float(row.get('AverageNs', 0)) / 1e3:.2f} | "
                             f"{float(row.get('MinNs', 0)) / 1e3:.2f} | {float(row.get('MaxNs', 0)) / 1e3:.2f} |")
        lines.append("")
    for f in counters:
        agg: dict[tuple[str, str], list[float]] = {}
        with open(f) as fh:
            for row in csv.DictReader(fh):
                key = ((row.get("Kernel_Name") or "?")[:90], row.get("Counter_Name") or "?")
                agg.setdefault(key, []).append(float(row.get("Counter_Value") or 0))
        lines += ["| kernel | counter | dispatches | mean per dispatch |", "|---|---|---:|---:|"]
        for (k, c), vals in sorted(agg.items()):
            lines.append(f"| `{k}` | {c} | {len(vals)} | {sum(vals) / len(vals):.1f} |")
        lines.append("")
    print("\n".join(lines))


def _counter_means(d: pathlib.Path, counter: str) -> dict[str, float]:
    import csv

    agg: dict[str, list[float]] = {}
    for f in sorted(d.rglob("*counter_collection.csv")):
        with open(f) as fh:
            for row in csv.DictReader(fh):
                if row.get("Counter_Name") == counter:
                    agg.setdefault(row.get("Kernel_Name") or "?", []).append(float(row.get("Counter_Value") or 0))
    return {k: sum(v) / len(v) for k, v in agg.items()}


def _copy_probe_calibration(torch, dev) -> None:
    """Three launches of the 1 GiB copy probe: the known-size kernel that
    calibrates FETCH_SIZE and WRITE_SIZE in a counter run."""
    from switchyard.hip_op import bandwidth_probe

    nbytes = 1 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    for _ in range(3):
        bandwidth_probe("copy", src, dst)
    torch.cuda.synchronize(dev)


def _launch_floor_and_copy_rate(torch, dev, loop, side) -> tuple[float, float]:
    """The two floors a small shape's step is reported against: microseconds
    per kernel of back-to-back launches of a kernel that does next to nothing
    (the write probe on 16 bytes, one workgroup), replayed from a HIP graph so
    that no host time is in it, and the 1 GiB copy probe's read+write rate in
    GB/s."""
    from switchyard import harness
    from switchyard.hip_op import bandwidth_probe

    tiny = torch.empty(4, dtype=torch.int32, device=dev)
    floor_ms = harness.time_graph([lambda: bandwidth_probe("write", None, tiny)], stream=side, per_graph=200)
    nbytes = 1 << 30
    src = torch.empty(nbytes, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    copy_ms = loop([lambda: bandwidth_probe("copy", src, dst)], device=dev, iters=20)
    del src, dst
    return floor_ms * 1e3, 2 * nbytes / copy_ms / 1e6


def _traffic_kernels(args):
    """(label, name substring, excluded substring, algorithmic bytes per launch,
    workload) of the kernels a counter run of --traffic-set covered."""
    slab = args.b * args.t * args.d * 2
    if args.traffic_set == "config2":
        n = args.n
        wl = f"N={n} B={args.b} T={args.t} D={args.d} bf16"
        return [("fwd", "k_fwd_res", None, (n + 1) * slab, wl),
                ("bwd_main", "k_bwd<", None, (2 * n + 1) * slab, wl),
                ("sol", "k_sol_res", None, (n + 1) * slab, wl)]
    if args.traffic_set == "schedule":  # bench.py --schedule --quick
        n, s, d = 9, 8, 2048
        slab = 4096 * d * 2
        wl = f"N={n} B=1 T=4096 D={d} bf16, S={s} queries"
        return [("batched_fwd", "k_batched_mx", None, (n + s) * slab + s * d * 2, wl),
                ("batched_bwd", "k_bwd_batched_mx", None, (2 * n + s) * slab + s * d * 2, wl),
                ("merge_fwd", "k_merge", "k_merge_bwd", 3 * slab + 6 * 4096 * 4, wl),
                ("merge_bwd", "k_merge_bwd", None, 5 * slab + 10 * 4096 * 4, wl),
                # the fused phase 2 (5 sources + the prior's o1 in, out written)
                ("phase2_fused", "4, 9, true, false>", None, 7 * slab + 4 * 4096 * 4, wl),
                ("table_bwd", "true, 1>", None, (2 * n + 1) * slab, wl)]
    if args.traffic_set in ("n4", "n16"):  # bench.py --sweep --sweep-only N4 (N16) --quick
        n, d = int(args.traffic_set[1:]), 2048
        slab = 4096 * d * 2
        wl = f"N={n} B=1 T=4096 D={d} bf16"
        fwd = ("fwd", "k_fwd_res", None) if n <= 9 else ("fwd_chunked", "k_fwd<", None)
        return [(*fwd, (n + 1) * slab, wl), ("bwd_main", "k_bwd<", None, (2 * n + 1) * slab, wl)]
    if args.traffic_set == "d8192f32":  # bench.py --sweep --dtype float32 --sweep-only d-sweep-b1 --quick
        n, d = 9, 8192
        slab = 4096 * d * 4
        wl = f"N={n} B=1 T=4096 D={d} fp32"
        # the eight-wave tiles run only at D=8192 in that set
        return [("fwd", "k_fwd_res<sy::F32, 8, 4, 9", None, (n + 1) * slab, wl),
                ("bwd_main", "k_bwd<sy::F32, 8, 4, 9, true, 0>", None, (2 * n + 1) * slab, wl)]
    n, d = 32, 2048  # bench.py --sweep --sweep-only N32 --quick
    slab = 4096 * d * 2
    wl = f"N={n} B=1 T=4096 D={d} bf16"
    return [("fwd_chunked", "k_fwd<", None, (n + 1) * slab, wl),
            ("bwd_tall", "k_bwd_tall", None, (2 * n + 1) * slab, wl)]


def traffic_mode(args):
    """HBM bytes per launch from FETCH_SIZE / WRITE_SIZE (KiB per dispatch),
    each scaled so the 1 GiB copy probe reads and writes exactly 1 GiB."""
    fetch = _counter_means(args.traffic[0], "FETCH_SIZE")
    write = _counter_means(args.traffic[1], "WRITE_SIZE")

    def pick(table, needle):
        hits = [v for k, v in table.items() if needle in k]
        if not hits:
            raise SystemExit(f"no dispatch of {needle} in the counter data")
        return hits[0]

    gib_kib = float(1 << 20)
    fscale = gib_kib / pick(fetch, "k_probe_copy")
    wscale = gib_kib / pick(write, "k_probe_copy")
    kernels = _traffic_kernels(args)
    rec = {"workload": kernels[0][4], "fetch_scale": fscale, "write_scale": wscale,
           "method": "rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE (KiB per dispatch), each scaled by what the "
                     "counter reads for the 1 GiB copy probe"}
    for key, needle, exclude, nbytes, _ in kernels:
        def hit(table):
            vals = [v for k, v in table.items() if needle in k and (exclude is None or exclude not in k)]
            if not vals:
                raise SystemExit(f"no dispatch of {needle} in the counter data")
            return sum(vals) / len(vals)

        f_kib, w_kib = hit(fetch), hit(write)
        tot = (f_kib * fscale + w_kib * wscale) * 1024
        rec[f"{key}_bytes_per_launch"] = round(tot)
        rec[f"{key}_fetch_kib"] = f_kib
        rec[f"{key}_write_kib"] = w_kib
        rec[f"{key}_algorithmic_bytes"] = nbytes
        rec[f"{key}_traffic_over_algorithmic"] = tot / nbytes
    line = json.dumps(rec, indent=1)
    if args.json_out:
        args.json_out.write_text(line + "\n")
    print(line)


SWEEP_SHAPES = (
    [("n-sweep", n, 1, 4096, 2048) for n in (2, 4, 8, 9, 16, 32)]
    + [("t-sweep", 9, 1, t, 2048) for t in (512, 1024, 2048, 4096, 8192, 16384)]
    # BASELINE.json configs[3] puts the D sweep at B=4 ...
    + [("d-sweep", 9, 4, 4096, d) for d in (1024, 2048, 4096)]
    # ... the reference's own shape sets (bench/bench_operator.py:65-79) at B=1,
    # with its batch and small sets
    + [("d-sweep-b1", 9, 1, 4096, d) for d in (1024, 2048, 4096, 8192)]
    + [("batch", 9, b, 2048, 2048) for b in (1, 2, 4, 8)]
    + [("small", 9, 1, 128, 1024), ("small", 9, 1, 512, 1024), ("small", 4, 1, 256, 512)]
)

#: The reference's published numbers on its RTX PRO 6000 (docs/results.md:20-60):
#: (N, B, T, D) -> (forward ms, fwd+bwd ms, forward % of its speed-of-light kernel).
REFERENCE_RESULTS = {
    (9, 1, 2048, 2048): (0.070, 0.181, 91), (9, 2, 2048, 2048): (0.125, 0.365, 97),
    (9, 4, 2048, 2048): (0.229, 0.688, 98), (9, 8, 2048, 2048): (0.440, 1.337, 100),
    (9, 1, 4096, 1024): (0.068, 0.191, 100), (9, 1, 4096, 2048): (0.123, 0.365, 97),
    (9, 1, 4096, 4096): (0.242, 0.924, 93), (9, 1, 4096, 8192): (0.522, 1.997, 85),
    (2, 1, 4096, 2048): (0.037, 0.177, 106), (4, 1, 4096, 2048): (0.066, 0.170, 97),
    (8, 1, 4096, 2048): (0.106, 0.309, 102), (16, 1, 4096, 2048): (0.197, 0.608, 101),
    (32, 1, 4096, 2048): (0.379, 1.552, 98), (9, 1, 128, 1024): (0.010, 0.169, 80),
    (9, 1, 512, 1024): (0.014, 0.112, 86), (4, 1, 256, 512): (0.008, 0.163, 100),
    (9, 1, 512, 2048): (0.025, 0.175, 75), (9, 1, 8192, 2048): (0.227, 0.686, 98),
    (9, 1, 16384, 2048): (0.442, 1.335, 99),
}

#: The reference's eight-query shape checks of the batched forward
#: (docs/batched_queries.md:27-34): (N, B, T, D) -> its ms on the RTX PRO 6000.
BATCHED_SHAPE_CHECKS = {
    (2, 1, 4096, 2048): 0.117, (16, 1, 4096, 2048): 0.344, (9, 1, 4096, 1024): 0.109,
    (9, 1, 128, 1024): 0.016, (9, 4, 2048, 2048): 0.393, (9, 1, 4096, 4096): 2.241,
}


def _sweep_shapes(only):
    """Distinct (N, B, T, D) of SWEEP_SHAPES in order, each with the sets that
    list it. ``only`` keeps a shape when one of its sets is named, or, for
    n-sweep shapes, when ``N<n>`` is."""
    shapes: dict[tuple, list[str]] = {}
    for name, n, b, t, d in SWEEP_SHAPES:
        shapes.setdefault((n, b, t, d), []).append(name)
    for shape, names in shapes.items():
        if only is None or any(x in only for x in names) or ("n-sweep" in names and f"N{shape[0]}" in only):
            yield shape, names


def _gate(tag, got, ref):
    """Per-tensor float64 check: 16-bit results within 1.10x the dtype floor,
    fp32 within 1e-5 relative L2 (the north star's bars)."""
    from switchyard import harness

    rep = harness.check_against(got, ref, rel_l2_tol=1e-5 if tag == "fp32" else float("inf"))
    if tag != "fp32":
        ratio = rep["err_vs_dtype_floor"]
        rep["ok"] = bool(ratio is not None and ratio <= 1.10 and not rep["nan_or_inf"])
        rep["rel_l2_tol"] = "1.10 x dtype floor"
    return {k: (round(v, 7) if isinstance(v, float) else v) for k, v in rep.items()}


DTYPE_TAG = {"bfloat16": "bf16", "float16": "fp16", "float32": "fp32"}


def sweep_mode(args):
    """Configs 3 and 4 of BASELINE.json in ``--dtype``: one JSON line per shape.
    With --json-out the run is also written as a results file for the
    regression gate (python -m switchyard.regression)."""
    import torch

    from switchyard import _lib, harness
    from switchyard.reference import attn_res_batched_bytes, attn_res_min_bytes, attn_res_train_bytes

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib, st = _lib.lib(), _lib.stream_ptr(dev)
    P = Workload._p
    dt = getattr(torch, args.dtype)
    code, tag = _lib.dtype_code(dt), DTYPE_TAG[args.dtype]
    item = torch.finfo(dt).bits // 8
    gen = torch.Generator(device=dev).manual_seed(0)
    results = []
    failed = []
    only = set(args.sweep_only.split(",")) if args.sweep_only else None
    loop = harness.time_loop if args.quick else harness.time_loop_median
    side = torch.cuda.Stream(dev)  # graph captures (device-only times)
    side_ptr = ctypes.c_void_p(side.cuda_stream)
    floor_us = copy_gbps = None  # --quick runs are counter targets: no extra probe launches
    if not args.quick:
        floor_us, copy_gbps = _launch_floor_and_copy_rate(torch, dev, loop, side)
        log(f"launch floor {floor_us:.2f} us a kernel, copy probe {copy_gbps:.0f} GB/s")
    for (n, b, t, d), names in _sweep_shapes(only):
        name = names[0]
        nt = b * t
        slab = nt * d * item
        rot = max(2, min(6, int((3 << 30) // ((2 * n + 3) * slab))))
        sets = []
        for _ in range(rot):
            v = torch.randn(n, b, t, d, device=dev, generator=gen).to(dt)
            sets.append(dict(v=v, g=torch.randn(b, t, d, device=dev, generator=gen).to(dt),
                             out=torch.empty(b, t, d, device=dev, dtype=dt),
                             stats=torch.empty(2, n, nt, device=dev), dv=torch.empty_like(v),
                             dw=torch.empty(d, device=dev, dtype=dt)))
        w = (0.5 * torch.randn(d, device=dev, generator=gen)).to(dt)
        ws_bytes = int(lib.sy_bwd_workspace_bytes(n, nt, d, code, code))
        ws = torch.empty(max(1, ws_bytes // 4), device=dev)

        def fwd(s, stream=st):
            _lib.check(lib.sy_fwd(P(s["v"]), P(w), P(s["out"]), P(s["stats"]), n, nt, d, nt * d, code, code,
                                  1e-6, stream), "sy_fwd")

        def bwd(s, stream=st):
            _lib.check(lib.sy_bwd(P(s["v"]), P(w), P(s["g"]), P(s["stats"]), P(s["dv"]), P(s["dw"]), P(ws),
                                  ws_bytes, n, nt, d, nt * d, code, code, 1e-6, stream), "sy_bwd")

        def sol(s):  # the ceiling: same bytes and launch shape, out = sum_n v_n
            _lib.check(lib.sy_sol(P(s["v"]), P(s["out"]), n, nt, d, nt * d, code, st), "sy_sol")

        iters = max(20, min(200, int(2e5 / (n * t * b * d / 1e4))))
        rows = int(lib.sy_bwd_partial_rows(n, nt, d, code, code, 1, 1))

        def bwd_main(s, stream=st):  # sy_bwd's first kernel: dv and the dw partial rows
            _lib.check(lib.sy_bwd_main(P(s["v"]), P(w), P(s["g"]), P(s["stats"]), P(s["dv"]), P(ws), ws_bytes,
                                       n, nt, d, nt * d, code, code, 1e-6, stream), "sy_bwd_main")

        def reduce(s, stream=st):  # its second: the partial rows summed into dw
            _lib.check(lib.sy_dw_reduce(P(ws), rows, d, P(s["dw"]), code, stream), "sy_dw_reduce")

        for s in sets:  # warm-up: a shape's first launches query kernel attributes
            fwd(s)
            bwd(s)
        if args.quick:
            iters = 3
        f_ms = loop([lambda s=s: fwd(s) for s in sets], device=dev, iters=iters)
        fb_ms = loop([lambda s=s: (fwd(s), bwd(s)) for s in sets], device=dev, iters=iters)
        fbg_ms = fg_ms = bm_ms = red_ms = None
        if not args.quick:  # replayed from HIP graphs: device time only
            fbg_ms = harness.time_graph([lambda s=s: (fwd(s, side_ptr), bwd(s, side_ptr)) for s in sets],
                                        stream=side)
            torch.cuda.synchronize(dev)
            replayed = [sets[0][k].clone() for k in ("out", "dv", "dw")]
            fwd(sets[0])
            bwd(sets[0])
            torch.cuda.synchronize(dev)
            if not all(torch.equal(a, sets[0][k]) for a, k in zip(replayed, ("out", "dv", "dw"))):
                failed.append(f"N{n} B{b} T{t} D{d} (graph replay differs from the eager step)")
            # The split (dw is then the last set's: the partial rows are shared;
            # the float64 gate below recomputes set 0 first).
            fg_ms = harness.time_graph([lambda s=s: fwd(s, side_ptr) for s in sets], stream=side)
            bm_ms = harness.time_graph([lambda s=s: bwd_main(s, side_ptr) for s in sets], stream=side)
            red_ms = harness.time_graph([lambda s=s: reduce(s, side_ptr) for s in sets], stream=side)
        for s in sets:
            sol(s)
        sol_ms = loop([lambda s=s: sol(s) for s in sets], device=dev, iters=iters)
        fb = attn_res_train_bytes(n, b, t, d, item)
        fw = attn_res_min_bytes(n, b, t, d, item)
        fplan = _lib.plan(_lib.OP_FWD, n, d, dt, n_tok=nt)
        bplan = _lib.plan(_lib.OP_BWD, n, d, dt, n_tok=nt)
        # Float64 gate of the timed launches' own outputs (set 0; same inputs,
        # same bits as every timed call on it), as the reference's harness
        # checks every shape before timing it (bench/harness.py:295-358).
        s0 = sets[0]
        fwd(s0)
        bwd(s0)
        ref_out, ref_dv, ref_dw = harness.float64_operator(s0["v"], w, s0["g"])
        check = {"out": _gate(tag, s0["out"], ref_out), "dv": _gate(tag, s0["dv"], ref_dv),
                 "dw": _gate(tag, s0["dw"], ref_dw)}
        check["ok"] = all(c["ok"] for c in check.values())
        del ref_out, ref_dv, ref_dw
        rec = {"sweep": name, "sweeps": names, "impl": "switchyard_hip", "N": n, "B": b, "T": t, "D": d,
               "dtype": tag, "rotating_sets": rot,
               "fwd_us": round(f_ms * 1e3, 2), "fwd_gbps": round(fw / f_ms / 1e6, 1),
               "fwd_frac_hbm_peak": round(fw / f_ms / 1e6 / HBM_PEAK_GBPS, 4),
               "sol_us": round(sol_ms * 1e3, 2),
               "fwd_pct_of_ceiling": round(100 * sol_ms / f_ms, 1),
               "fwd_bwd_us": round(fb_ms * 1e3, 2), "fwd_bwd_gbps": round(fb / fb_ms / 1e6, 1),
               "fwd_bwd_frac_hbm_peak": round(fb / fb_ms / 1e6 / HBM_PEAK_GBPS, 4),
               "bwd_main_graph_us": None if bm_ms is None else round(bm_ms * 1e3, 2),
               "reduce_graph_us": None if red_ms is None else round(red_ms * 1e3, 2),
               # fwd+bwd's floor: its three kernels' launches plus its bytes at the copy rate
               "fwd_graph_us": None if fg_ms is None else round(fg_ms * 1e3, 2),
               "fwd_bwd_graph_us": None if fbg_ms is None else round(fbg_ms * 1e3, 2),
               "launch_floor_us": None if floor_us is None else round(floor_us, 2),
               "fwd_bwd_floor_us": None if floor_us is None else round(3 * floor_us + fb / copy_gbps / 1e3, 2),
               "workspace_bytes": ws_bytes + 2 * n * nt * 4,
               "fwd_tile": [fplan["family_name"], fplan["waves_per_token"], fplan["chunks_per_lane"],
                            fplan["rows_per_tile"]],
               "bwd_tile": [bplan["family_name"], bplan["waves_per_token"], bplan["chunks_per_lane"],
                            bplan["rows_per_tile"]],
               "check": check}
        ref = REFERENCE_RESULTS.get((n, b, t, d))
        if ref is not None and tag == "bf16":
            rec["reference_rtx_pro_6000"] = {"fwd_us": 1e3 * ref[0], "fwd_bwd_us": 1e3 * ref[1],
                                             "fwd_pct_of_ceiling": ref[2]}
        print(json.dumps(rec), flush=True)
        results.append(rec)
        if not check["ok"]:
            failed.append(f"N{n} B{b} T{t} D{d}")
        del sets, ws
        torch.cuda.empty_cache()
    # Config 3: batched, Q=8 queries sharing one read of v.
    if only is None or "batched" in only:
        batched_sweep(args, results, failed)
    elif args.quick:
        _copy_probe_calibration(torch, dev)
    if args.json_out:
        args.json_out.parent.mkdir(parents=True, exist_ok=True)
        args.json_out.write_text(json.dumps({"environment": harness.environment(), "dtype": tag,
                                             "results": results}, indent=1))
    if failed:
        log(f"bench.py --sweep: float64 gate failed at {', '.join(failed)}")
        sys.exit(1)


def batched_sweep(args, results, failed):
    """Config 3 (Q=8 at N=9 B=1 T=4096 D=2048), the reference's query-count
    sweep around it (Q = 1, 2, 4, 16; docs/batched_queries.md:16-22) and its
    eight-query shape checks (:27-34), each gated against float64."""
    import torch

    from switchyard import _lib, harness
    from switchyard.reference import attn_res_batched_bytes

    dev = torch.device("cuda:0")
    lib, st = _lib.lib(), _lib.stream_ptr(dev)
    side = torch.cuda.Stream(dev)  # graph captures (device-only times)
    side_ptr = ctypes.c_void_p(side.cuda_stream)
    P = Workload._p
    dt = getattr(torch, args.dtype)
    code, tag = _lib.dtype_code(dt), DTYPE_TAG[args.dtype]
    item = torch.finfo(dt).bits // 8
    gen = torch.Generator(device=dev).manual_seed(0)
    gq = torch.Generator().manual_seed(1)  # the reference's query seed (bench/harness.py:68-69)
    qmax = 16
    all_queries = (0.5 * torch.randn(qmax, 8192, generator=gq)).to(dt).to(dev)
    ref_q_us = {1: 121.0, 2: 133.0, 4: 152.0, 8: 198.7, 16: 369.0}
    cases = [((9, 1, 4096, 2048), q) for q in (8, 1, 2, 4, 16)]
    cases += [(shape, 8) for shape in BATCHED_SHAPE_CHECKS if shape != (9, 1, 4096, 2048)]
    prev = None
    for (n, b, t, d), q in cases:
        nt = b * t
        if prev != (n, b, t, d):
            sets = None
            torch.cuda.empty_cache()
            slab = nt * d * item
            rot = max(2, min(6, int((3 << 30) // ((n + qmax) * slab))))
            sets = [dict(v=torch.randn(n, b, t, d, device=dev, generator=gen).to(dt),
                         out=torch.empty(qmax, b, t, d, device=dev, dtype=dt)) for _ in range(rot)]
            prev = (n, b, t, d)
        queries = all_queries[:q, :d].contiguous()

        def batched(s, q=q, queries=queries, n=n, nt=nt, d=d, stream=st):
            _lib.check(lib.sy_fwd_batched(P(s["v"]), P(queries), P(s["out"]), n, q, nt, d, nt * d, code, 1e-6,
                                          stream), "sy_fwd_batched")

        for s in sets:  # warm-up: first launches load code objects and query attributes
            batched(s)
        # 100-call loops, as the config-3 line always used: 20-call loops of the
        # batched forward read 5-8% slower (clocks still ramping between loops)
        iters = 3 if args.quick else 100
        loop = harness.time_loop if args.quick else harness.time_loop_median
        ms = loop([lambda s=s: batched(s) for s in sets], device=dev, iters=iters)
        gms = None if args.quick else harness.time_graph([lambda s=s: batched(s, stream=side_ptr) for s in sets],
                                                         stream=side)
        nbytes = attn_res_batched_bytes(n, q, b, t, d, item)
        s0 = sets[0]
        batched(s0)
        check = {}
        for k in range(q):
            ref, _, _ = harness.float64_operator(s0["v"], queries[k])
            check[f"out[{k}]"] = _gate(tag, s0["out"][k], ref)
        worst = max(check.values(), key=lambda c: c["rel_l2"])
        check = {"queries": q, "ok": all(c["ok"] for c in check.values()), "worst": worst}
        plan = _lib.plan(_lib.OP_BATCHED, n, d, dt, n_q=q)
        config3 = (n, b, t, d) == (9, 1, 4096, 2048)
        rec = {"sweep": ("batched" if q == 8 else "batched-q") if config3 else "batched-shape",
               "impl": "switchyard_hip", "N": n, "B": b, "T": t, "D": d, "Q": q, "dtype": tag,
               "fwd_us": round(ms * 1e3, 2), "fwd_gbps": round(nbytes / ms / 1e6, 1),
               "fwd_frac_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4),
               "fwd_graph_us": None if gms is None else round(gms * 1e3, 2),
               "family": plan["family_name"], "check": check}
        if tag == "bf16":
            rec["reference_rtx_pro_6000_us"] = ref_q_us[q] if config3 else 1e3 * BATCHED_SHAPE_CHECKS[(n, b, t, d)]
        print(json.dumps(rec), flush=True)
        results.append(rec)
        if not check["ok"]:
            failed.append(f"batched N{n} B{b} T{t} D{d} Q{q}")
    del sets
    torch.cuda.empty_cache()


def schedule_mode(args):
    """The widened rows at config 2/3 shapes (bf16): pointer-table input vs the
    stacked operator, attn_with_stats / merge / two-phase, batched statistics,
    and the batched backward. One JSON line per measurement."""
    import torch

    from switchyard import _lib, harness

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib, st = _lib.lib(), _lib.stream_ptr(dev)
    P = Workload._p
    dt, code, item = torch.bfloat16, _lib.SY_BF16, 2
    n, b, t, d, nq = 9, 1, 4096, 2048, 8
    nt = b * t
    slab = nt * d * item
    gen = torch.Generator(device=dev).manual_seed(0)
    w = (0.5 * torch.randn(d, device=dev, generator=gen)).to(dt)
    rot = 6
    results = []

    def emit(name, ms, nbytes, **extra):
        rec = {"row": name, "N": n, "B": b, "T": t, "D": d, "dtype": "bf16", "us": round(ms * 1e3, 2),
               "algorithmic_bytes": nbytes, "gbps": round(nbytes / ms / 1e6, 1),
               "frac_hbm_peak": round(nbytes / ms / 1e6 / HBM_PEAK_GBPS, 4), **extra}
        print(json.dumps(rec), flush=True)
        results.append(rec)

    def timed(fns, iters=100):
        for f in fns:
            f()
        if args.quick:
            return harness.time_loop(fns, device=dev, iters=3)
        return harness.time_loop_median(fns, device=dev, iters=iters)

    # --- pointer table vs stacked (config 2) ---------------------------------
    ws_bytes = int(lib.sy_bwd_workspace_bytes(n, nt, d, code, code))
    sets = []
    for _ in range(rot):
        v = torch.randn(n, b, t, d, device=dev, generator=gen).to(dt)
        srcs = [torch.randn(b, t, d, device=dev, generator=gen).to(dt) for _ in range(n)]  # separate allocations
        dvs = [torch.empty(b, t, d, device=dev, dtype=dt) for _ in range(n)]
        sets.append(dict(v=v, srcs=srcs, tab=_lib.pointer_table(srcs), dvs=dvs, dtab=_lib.pointer_table(dvs),
                         g=torch.randn(b, t, d, device=dev, generator=gen).to(dt),
                         out=torch.empty(b, t, d, device=dev, dtype=dt), stats=torch.empty(2, n, nt, device=dev),
                         dv=torch.empty_like(v), dw=torch.empty(d, device=dev, dtype=dt),
                         ws=torch.empty(max(1, ws_bytes // 4), device=dev)))

    def fwd_stacked(s):
        _lib.check(lib.sy_fwd(P(s["v"]), P(w), P(s["out"]), P(s["stats"]), n, nt, d, nt * d, code, code, 1e-6,
                              st), "sy_fwd")

    def bwd_stacked(s):
        _lib.check(lib.sy_bwd(P(s["v"]), P(w), P(s["g"]), P(s["stats"]), P(s["dv"]), P(s["dw"]), P(s["ws"]),
                              ws_bytes, n, nt, d, nt * d, code, code, 1e-6, st), "sy_bwd")

    def fwd_table(s):
        _lib.check(lib.sy_fwd_table(s["tab"], P(w), P(s["out"]), P(s["stats"]), n, nt, d, code, code, 1e-6, st),
                   "sy_fwd_table")

    def bwd_table(s):
        _lib.check(lib.sy_bwd_table(s["tab"], P(w), P(s["g"]), P(s["stats"]), s["dtab"], P(s["dw"]), P(s["ws"]),
                                    ws_bytes, n, nt, d, code, code, 1e-6, st), "sy_bwd_table")

    def stack_then_fwd(s):  # what a caller with separate sources pays without the table
        torch.stack(s["srcs"], out=s["v"])
        fwd_stacked(s)

    fw, fb = (n + 1) * slab, (3 * n + 2) * slab
    emit("stacked_fwd", timed([lambda s=s: fwd_stacked(s) for s in sets]), fw)
    emit("table_fwd", timed([lambda s=s: fwd_table(s) for s in sets]), fw)
    emit("stack_copy_then_fwd", timed([lambda s=s: stack_then_fwd(s) for s in sets]), fw,
         note="torch.stack of the sources into v, then the stacked forward")
    emit("stacked_fwd_bwd", timed([lambda s=s: (fwd_stacked(s), bwd_stacked(s)) for s in sets]), fb)
    emit("table_fwd_bwd", timed([lambda s=s: (fwd_table(s), bwd_table(s)) for s in sets]), fb)

    # --- attn_with_stats, merge, two-phase (config 2) ------------------------
    for s in sets:
        s.update(o1=torch.empty(b, t, d, device=dev, dtype=dt), o2=torch.empty(b, t, d, device=dev, dtype=dt),
                 m1=torch.empty(nt, device=dev), l1=torch.empty(nt, device=dev), m2=torch.empty(nt, device=dev),
                 l2=torch.empty(nt, device=dev), mo=torch.empty(nt, device=dev), lo=torch.empty(nt, device=dev),
                 do1=torch.empty(b, t, d, device=dev, dtype=dt), do2=torch.empty(b, t, d, device=dev, dtype=dt),
                 gm=torch.randn(nt, device=dev, generator=gen), gl=torch.randn(nt, device=dev, generator=gen),
                 dm1=torch.empty(nt, device=dev), dl1=torch.empty(nt, device=dev),
                 dm2=torch.empty(nt, device=dev), dl2=torch.empty(nt, device=dev))
    split = 4

    def stats_fwd(s, lo_, hi_, o, m, ell):
        v = s["v"][lo_:hi_]
        _lib.check(lib.sy_attn_with_stats(P(v), P(w), P(o), P(m), P(ell), None, hi_ - lo_, nt, d, nt * d, code,
                                          code, 1e-6, st), "sy_attn_with_stats")

    def merge(s):
        _lib.check(lib.sy_merge_stats(P(s["o1"]), P(s["m1"]), P(s["l1"]), P(s["o2"]), P(s["m2"]), P(s["l2"]),
                                      P(s["out"]), P(s["mo"]), P(s["lo"]), nt, d, code, st), "sy_merge_stats")

    def merge_bwd(s):
        _lib.check(lib.sy_merge_stats_bwd(P(s["o1"]), P(s["m1"]), P(s["l1"]), P(s["o2"]), P(s["m2"]), P(s["l2"]),
                                          P(s["g"]), P(s["gm"]), P(s["gl"]), P(s["do1"]), P(s["dm1"]), P(s["dl1"]),
                                          P(s["do2"]), P(s["dm2"]), P(s["dl2"]), nt, d, code, st),
                   "sy_merge_stats_bwd")

    emit("attn_with_stats_fwd", timed([lambda s=s: stats_fwd(s, 0, n, s["o1"], s["m1"], s["l1"]) for s in sets]),
         fw + 2 * nt * 4)
    for s in sets:
        stats_fwd(s, 0, split, s["o1"], s["m1"], s["l1"])
        stats_fwd(s, split, n, s["o2"], s["m2"], s["l2"])
    emit("merge_fwd", timed([lambda s=s: merge(s) for s in sets]), 3 * slab + 6 * nt * 4)
    emit("merge_bwd", timed([lambda s=s: merge_bwd(s) for s in sets]), 5 * slab + 10 * nt * 4)
    def phase2_fused(s):  # this group's sources merged with (o1, m1, l1) and normalised in one pass
        v = s["v"][split:n]
        _lib.check(lib.sy_attn_with_stats_merge(P(v), P(w), P(s["o1"]), P(s["m1"]), P(s["l1"]), P(s["out"]),
                                                P(s["mo"]), P(s["lo"]), n - split, nt, d, nt * d, code, code, 1e-6,
                                                1, st), "sy_attn_with_stats_merge")

    emit("two_phase_fwd", timed([lambda s=s: (stats_fwd(s, 0, split, s["o1"], s["m1"], s["l1"]), phase2_fused(s))
                                 for s in sets]), fw,
         note=f"group [0,{split}) with statistics, then group [{split},{n}) merged with it and normalised in "
              "one pass (2 kernels); bytes counted as the single pass's",
         actual_bytes=(n + 3) * slab + 4 * nt * 4)
    emit("two_phase_fwd_unfused", timed([lambda s=s: (stats_fwd(s, 0, split, s["o1"], s["m1"], s["l1"]),
                                                      stats_fwd(s, split, n, s["o2"], s["m2"], s["l2"]), merge(s))
                                         for s in sets]), fw,
         note=f"groups [0,{split}) and [{split},{n}) then the merge kernel (3 kernels, o unnormalised); bytes "
              "counted as the single pass's")
    del sets
    torch.cuda.empty_cache()

    # --- batched with statistics and batched backward (config 3) ------------
    q = (0.5 * torch.randn(nq, d, generator=torch.Generator().manual_seed(1))).to(dt).to(dev)
    bw_bytes = int(lib.sy_bwd_batched_workspace_bytes(n, nq, nt, d, code))
    sets = []
    for _ in range(rot):
        v = torch.randn(n, b, t, d, device=dev, generator=gen).to(dt)
        sets.append(dict(v=v, g=torch.randn(nq, b, t, d, device=dev, generator=gen).to(dt),
                         o=torch.empty(nq, b, t, d, device=dev, dtype=dt), m=torch.empty(nq, nt, device=dev),
                         ell=torch.empty(nq, nt, device=dev), dv=torch.empty_like(v),
                         dq=torch.empty(nq, d, device=dev, dtype=dt), ws=torch.empty(max(1, bw_bytes // 4), device=dev)))

    def batched_fwd(s):
        _lib.check(lib.sy_fwd_batched(P(s["v"]), P(q), P(s["o"]), n, nq, nt, d, nt * d, code, 1e-6, st),
                   "sy_fwd_batched")

    def batched_stats(s):
        _lib.check(lib.sy_batched_with_stats(P(s["v"]), P(q), P(s["o"]), P(s["m"]), P(s["ell"]), n, nq, nt, d,
                                             nt * d, code, 1e-6, st), "sy_batched_with_stats")

    def batched_bwd(s):
        _lib.check(lib.sy_bwd_batched(P(s["v"]), P(q), P(s["g"]), P(s["dv"]), P(s["dq"]), P(s["ws"]), bw_bytes, n,
                                      nq, nt, d, nt * d, code, 1e-6, st), "sy_bwd_batched")

    bf = (n + nq) * slab + nq * d * item
    emit("batched_fwd", timed([lambda s=s: batched_fwd(s) for s in sets]), bf, Q=nq)
    emit("batched_with_stats_fwd", timed([lambda s=s: batched_stats(s) for s in sets]), bf + 2 * nq * nt * 4, Q=nq)
    emit("batched_bwd", timed([lambda s=s: batched_bwd(s) for s in sets]), (2 * n + nq) * slab + 2 * nq * d * item,
         Q=nq, workspace_bytes=bw_bytes,
         note="reads v and the Q output gradients once, writes dv once; S separate backward calls would move "
              f"{nq * (2 * n + 1)} slabs instead of {2 * n + nq}")
    if args.quick:
        _copy_probe_calibration(torch, dev)
    if args.json_out:
        args.json_out.parent.mkdir(parents=True, exist_ok=True)
        args.json_out.write_text(json.dumps({"environment": harness.environment(), "results": results}, indent=1))


MODEL_SCALES = {
    "1.3B": dict(vocab_size=32000, d_model=2048, n_layers=24, n_heads=16, d_ff=5632, n_blocks=8, max_seq_len=4096),
    "small": dict(vocab_size=4096, d_model=512, n_layers=8, n_heads=8, d_ff=1408, n_blocks=4, max_seq_len=512),
}


def profile_step(model, step, dev, iters: int = 3) -> dict:
    """Device time of the residual mechanism inside training steps, from a
    torch.profiler trace: the HIP operator's kernels are found by name (every
    one lives in the ``sy::`` namespace: forward, backward, dw reduction), the
    source staging (arena slot copies, ``torch.stack``) by its
    ``attnres_stage`` region, and for the eager mechanism, whose kernels are
    generic, the forward by its ``attnres_op`` region (its backward cannot be
    told apart and is reported as None). Reference: bench/bench_model.py:211-255
    attributes by region and autograd-node name."""
    import torch
    from torch.profiler import ProfilerActivity, profile

    regions = ("attnres_stage", "attnres_op")
    model.profile_regions = True
    try:
        for _ in range(2):
            step()
        torch.cuda.synchronize(dev)
        with profile(activities=[ProfilerActivity.CPU, ProfilerActivity.CUDA]) as prof:
            for _ in range(iters):
                step()
            torch.cuda.synchronize(dev)
    finally:
        model.profile_regions = False
    total = op_kernels = 0.0
    region_dev: dict[str, float] = {}
    for e in prof.key_averages():
        if e.device_type == torch.autograd.DeviceType.CUDA:
            if e.key in regions or e.key.startswith(("Memcpy", "Memset")):
                continue
            total += e.self_device_time_total
            if "sy::" in e.key:
                op_kernels += e.self_device_time_total
        elif e.key in regions:
            region_dev[e.key] = region_dev.get(e.key, 0.0) + e.device_time_total
    out = {"iters": iters, "total_device_us": round(total / iters, 1),
           "staging_us": round(region_dev.get("attnres_stage", 0.0) / iters, 1)}
    hip = model.cfg.residual == "switchyard"
    if model.cfg.residual == "standard":
        return out
    if hip:
        out["operator_kernels_us"] = round(op_kernels / iters, 1)
        out["attnres_share_of_device_time"] = round((op_kernels / iters + out["staging_us"]) / out["total_device_us"], 4)
    else:
        out["operator_forward_us"] = round(region_dev.get("attnres_op", 0.0) / iters, 1)
        out["operator_backward_us"] = None
        out["attnres_share_of_device_time"] = None
    return out


def model_mode(args):
    """Config 5: tokens/s of a bf16 AdamW training step (reference bench/bench_model.py)."""
    import torch

    from switchyard import harness
    from switchyard.model import ModelConfig, Transformer

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    bsz, seq = args.model_batch, args.model_seq
    variants = [("standard", "arena"), ("attnres", "arena"), ("switchyard", "arena"), ("switchyard", "stack"),
                ("switchyard", "table")]
    out = {"metric": "decoder training step tokens/s (config 5)", "scale": args.model_scale,
           "config": MODEL_SCALES[args.model_scale], "batch": bsz, "seq": seq, "dtype": "bf16",
           "data": "uniform-random token ids, random-init weights (seed 0)", "variants": []}
    for residual, sources in variants:
        torch.manual_seed(0)
        cfg = ModelConfig(**MODEL_SCALES[args.model_scale], residual=residual, sources=sources)
        with dev:  # initialise on the device
            model = Transformer(cfg)
        model = model.to(dtype=torch.bfloat16)
        opt = torch.optim.AdamW(model.parameters(), lr=1e-6)
        idx = torch.randint(0, cfg.vocab_size, (bsz, seq), device=dev)
        tgt = torch.randint(0, cfg.vocab_size, (bsz, seq), device=dev)

        def step():
            model.zero_grad(set_to_none=True)
            model(idx, tgt)[1].backward()
            opt.step()

        def fwd():
            with torch.no_grad():
                return model(idx, tgt)[1]

        t_step = harness.measure_latency(step, device=dev, warmup=3, reps=args.model_reps, flush=False)
        t_fwd = harness.measure_latency(fwd, device=dev, warmup=2, reps=args.model_reps, flush=False)
        torch.cuda.reset_peak_memory_stats(dev)
        step()
        torch.cuda.synchronize(dev)
        rec = {"variant": residual if residual == "standard" else f"{residual}/{sources}",
               "params": model.param_counts()["total"], "step_ms": round(t_step.median_ms, 3),
               "forward_nograd_ms": round(t_fwd.median_ms, 3),
               "tokens_per_s": round(bsz * seq / (t_step.median_ms * 1e-3), 1),
               "peak_memory_gib": round(torch.cuda.max_memory_allocated(dev) / 2**30, 2)}
        if residual != "standard":
            rec["source_counts"] = sum(model.last_source_counts)
        rec["profile"] = profile_step(model, step, dev)
        out["variants"].append(rec)
        log(json.dumps(rec))
        del model, opt
        torch.cuda.empty_cache()
    base = out["variants"][0]["step_ms"]
    for r in out["variants"][1:]:
        r["share_of_step_vs_control"] = round(1 - base / r["step_ms"], 4)
        prof = r.get("profile", {})
        base_dev = out["variants"][0].get("profile", {}).get("total_device_us")
        if base_dev and prof.get("total_device_us"):
            # device-time difference against the control, as a share of this
            # variant's device time: what the mechanism adds on the GPU
            r["device_share_vs_control"] = round(1 - base_dev / prof["total_device_us"], 4)
        if prof.get("attnres_share_of_device_time") is not None:
            # The two measures of the mechanism's cost should agree: the
            # control difference (whole steps) and the profiler's device time.
            r["share_agreement"] = round(prof["attnres_share_of_device_time"] - r["share_of_step_vs_control"], 4)
    out["reference_rtx_pro_6000"] = {"standard_tok_s": 19101, "switchyard_arena_tok_s": 16918,
                                     "note": "reference README.md:82-84, vocab 32768"}
    print(json.dumps(out), flush=True)


def main() -> None:
    args = parse_args()
    if args.sweep:
        sweep_mode(args)
        return
    if args.schedule:
        schedule_mode(args)
        return
    if args.model:
        model_mode(args)
        return
    if args.traffic is not None:
        traffic_mode(args)
        return
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus > 1 or world > 1:
        print("bench.py: this build measures one GPU only. Tokens are independent, so the operator "
              "shards over B*T with no communication in the forward and one 4*D-byte all-reduce of "
              "dw in the backward; one GPU's share is the number measured here. Run with --gpus 1.",
              file=sys.stderr)
        sys.exit(2)
    if args.summarize is not None:
        summarize(args)
        return
    if args.kernel is not None:
        run_kernel_mode(args)
        return

    import torch

    from switchyard import harness
    from switchyard.reference import attn_res_min_bytes, attn_res_train_bytes

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    wl = Workload(args, torch, dev)
    n, b, t, d, item = wl.n, wl.b, wl.t, wl.d, wl.item
    fwd_bytes = attn_res_min_bytes(n, b, t, d, item)
    step_bytes = attn_res_train_bytes(n, b, t, d, item)
    bwd_bytes = (2 * n + 1) * wl.slab
    sol_bytes = fwd_bytes

    # ---- per-kernel averages, live, HIP events on the launch stream --------
    # Measured before the timed steps: the device then enters the timed region
    # at its sustained clocks, as a training loop's step would (after only a
    # few warm-up steps the same K steps read 2% slower: 90.1-90.5 against
    # 88.4 us at config 2 with 200 or 1000 warm-up steps).
    k_iters = max(args.steps, 200)
    per = {}
    for name in ("fwd", "bwd_main", "bwd", "sol"):  # median of three loops after an untimed one
        per[name] = harness.time_loop_median(wl.closures(name), device=dev, iters=k_iters)
    # The 4 us reduction alone is launch-bound in a host loop (each launch
    # costs the host more than the kernel takes): its share of the step is
    # timed as sy_bwd (main + reduction) minus the main kernel.
    per["reduce"] = per.pop("bwd") - per["bwd_main"]

    steps = [(lambda s=s: wl.step(s)) for s in wl.sets]
    for i in range(args.warmup):
        steps[i % len(steps)]()
    torch.cuda.synchronize(dev)

    # ---- timed region: exactly --steps steps ------------------------------
    t0 = time.perf_counter()
    ms_step = harness.time_loop(steps, device=dev, iters=args.steps)
    wall_ms = (time.perf_counter() - t0) * 1e3 / args.steps
    log(f"step (fwd+bwd): {ms_step * 1e3:.2f} us  [{step_bytes / ms_step / 1e6:.0f} GB/s]  wall {wall_ms * 1e3:.2f} us")

    nbytes_copy = 1 << 30
    src = torch.empty(nbytes_copy, dtype=torch.uint8, device=dev).fill_(3)
    dst = torch.empty(nbytes_copy, dtype=torch.uint8, device=dev)
    from switchyard.hip_op import bandwidth_probe

    copy_ms = harness.time_loop([lambda: bandwidth_probe("copy", src, dst)], device=dev, iters=20)
    copy_gbps = 2 * nbytes_copy / copy_ms / 1e6
    del src, dst
    for k, ms in per.items():
        log(f"  {k:9s} {ms * 1e3:8.2f} us")
    log(f"  copy probe {copy_gbps:.0f} GB/s (read+write)")

    fwd_gbps = fwd_bytes / per["fwd"] / 1e6
    bwd_gbps = bwd_bytes / per["bwd_main"] / 1e6
    traffic = None
    if TRAFFIC_FILE.exists() and (n, b, t, d, args.dtype) == (9, 1, 4096, 2048, "bfloat16"):
        try:
            traffic = json.loads(TRAFFIC_FILE.read_text()).get("bwd_main_bytes_per_launch")
        except (OSError, ValueError):
            traffic = None

    rec = {
        "metric": METRIC,
        "value": round(step_bytes / ms_step / 1e6, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bfloat16": "bf16", "float16": "f16", "float32": "f32"}[args.dtype],
        "data": f"synthetic, CPU seed 0: v~N(0,1), w~N(0,{args.w_std}), grad_out~N(0,1), rounded to {args.dtype}",
        "config": {"workload": "Block AttnRes fwd+bwd (sy_fwd + sy_bwd via the C ABI)", "n_src": n, "batch": b,
                   "seq_len": t, "d_model": d, "eps": 1e-6, "parallelism": "none (1 GPU)",
                   "rotating_sets": len(wl.sets)},
        "roofline": {
            "kernel": "k_bwd (persistent backward: reads v and grad_out, writes dv)",
            "bound": "hbm",
            "achieved": round(bwd_gbps, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(bwd_gbps / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "traffic_source": ("stored: profiles/traffic_N9_B1_T4096_D2048_bf16.json (rocprofv3 --pmc "
                               "FETCH_SIZE and WRITE_SIZE of this kernel, calibrated on a copy kernel); "
                               "not measured in this run") if traffic is not None else None,
            "algorithmic_bytes_per_launch": bwd_bytes,
            "avg_launch_us": round(per["bwd_main"] * 1e3, 3),
        },
        "fwd": {"kernel": "k_fwd_res", "avg_launch_us": round(per["fwd"] * 1e3, 3), "bytes": fwd_bytes,
                "achieved_gbps": round(fwd_gbps, 1), "frac_hbm_peak": round(fwd_gbps / HBM_PEAK_GBPS, 4),
                "frac_of_sol_kernel": round(per["sol"] / per["fwd"], 4),
                "frac_of_copy_probe": round(fwd_gbps / copy_gbps, 4)},
        "fwd_bwd": {"ms": round(ms_step, 5), "bytes": step_bytes, "achieved_gbps": round(step_bytes / ms_step / 1e6, 1),
                    "frac_hbm_peak": round(step_bytes / ms_step / 1e6 / HBM_PEAK_GBPS, 4),
                    "kernels_per_step": 3, "wall_ms_per_step": round(wall_ms, 5)},
        "kernels_us": {k: round(v * 1e3, 3) for k, v in per.items()},
        "sol_gbps": round(sol_bytes / per["sol"] / 1e6, 1),
        "copy_probe_gbps": round(copy_gbps, 1),
        "bwd_workspace_bytes": wl.ws_bytes,
        "stats_bytes": 2 * n * wl.n_tok * 4,
    }
    if not args.no_extras:
        try:
            rec["reference_method"] = api_extras(wl, args, torch, harness)
        except Exception as exc:  # noqa: BLE001
            rec["reference_method"] = {"error": f"{type(exc).__name__}: {exc}"[:300]}
    rec["cpu_baseline"] = None
    failed = None
    if not args.no_cpu_baseline:
        try:
            check, cpu = cpu_baseline_leg(wl, args, torch)
            cpu["host_cpu"] = harness.cpu_model()
            rec["cpu_baseline"] = cpu
            rec["correctness"] = check
            if not check["ok"]:
                failed = "the timed kernels' outputs are off the 1.10x dtype-floor bar"
        except Exception as exc:  # noqa: BLE001
            rec["cpu_baseline_error"] = f"{type(exc).__name__}: {exc}"[:300]
            failed = "the correctness check raised"
    rec["environment"] = harness.environment()
    rec["provenance"] = harness.provenance(ROOT, argv=sys.argv, seeds={"inputs": 0, "unit_norm_query": 1})
    rec["commit"] = rec["provenance"]["commit"]
    line = json.dumps(rec)
    if args.json_out:
        args.json_out.parent.mkdir(parents=True, exist_ok=True)
        args.json_out.write_text(line + "\n")
    print(line, flush=True)
    if failed:
        log(f"bench.py: {failed}")
        sys.exit(1)


if __name__ == "__main__":
    main()
