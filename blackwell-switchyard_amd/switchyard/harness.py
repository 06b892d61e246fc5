"""Measurement primitives for the Block AttnRes operator on MI355X.

Mirrors the reference's bench/harness.py (timing with order statistics, cache
flush between timed reps, workspace accounting, kernel counting, environment
record) with two MI355X-specific changes:

* **Flush size.** MI355X has a 4 MiB L2 per XCD and a 256 MiB memory-side
  Infinity Cache (MALL). The reference's 384 MiB flush (harness.py:37-38) is
  sized for a 128 MiB L2; here 1 GiB is written between reps so a timed rep
  starts from HBM.
* **Rotating inputs.** Back-to-back timing (bench.py's K-step loop) cycles
  through several independent input/output sets whose total is many times the
  MALL, so consecutive steps never find their operands cached.

Timing uses HIP events recorded on the stream the kernels run on (torch's
current stream, which is also where ``switchyard.hip_op`` launches).
"""

from __future__ import annotations

import gc
import os
import platform
import statistics
import subprocess
import time
from collections.abc import Callable
from dataclasses import dataclass, field

import torch

#: Bytes written between timed reps: 4x the 256 MiB Infinity Cache.
FLUSH_BYTES = 1 << 30
#: MI355X published peaks.
HBM_PEAK_BYTES_PER_S = 8.0e12
_flush: dict[torch.device, torch.Tensor] = {}


def flush_caches(device: torch.device) -> None:
    """Evict L2 and the Infinity Cache by writing FLUSH_BYTES."""
    buf = _flush.get(device)
    if buf is None:
        buf = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=device)
        _flush[device] = buf
    buf.fill_(1)


@dataclass
class Timing:
    median_ms: float
    p10_ms: float
    p90_ms: float
    min_ms: float
    mean_ms: float
    cv: float
    reps: int
    warmup: int
    flushed: bool

    def as_dict(self) -> dict:
        return dict(self.__dict__)


def _stats(samples: list[float], warmup: int, flushed: bool) -> Timing:
    samples = sorted(samples)
    n = len(samples)
    mean = statistics.fmean(samples)
    return Timing(
        median_ms=samples[n // 2],
        p10_ms=samples[max(0, int(0.10 * n))],
        p90_ms=samples[min(n - 1, int(0.90 * n))],
        min_ms=samples[0],
        mean_ms=mean,
        cv=(statistics.pstdev(samples) / mean) if mean > 0 else 0.0,
        reps=n,
        warmup=warmup,
        flushed=flushed,
    )


def measure_latency(fn: Callable[[], object], *, device: torch.device, warmup: int = 25,
                    reps: int = 100, flush: bool = True) -> Timing:
    """Per-call latency, one HIP event pair per rep, caches flushed before
    each rep (reference harness.py:96-138)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize(device)
    samples = []
    for _ in range(reps):
        if flush:
            flush_caches(device)
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        fn()
        end.record()
        torch.cuda.synchronize(device)
        samples.append(start.elapsed_time(end))
    return _stats(samples, warmup, flush)


def time_loop(fns: list[Callable[[], object]], *, device: torch.device, iters: int) -> float:
    """Average ms per call of ``iters`` back-to-back calls, cycling through
    ``fns`` (each bound to its own rotating buffers), bracketed by one event
    pair after a synchronize."""
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(iters):
        fns[i % len(fns)]()
    end.record()
    torch.cuda.synchronize(device)
    return start.elapsed_time(end) / iters


def time_loop_median(fns: list[Callable[[], object]], *, device: torch.device, iters: int, reps: int = 3) -> float:
    """Median over ``reps`` of :func:`time_loop`, after one untimed loop of
    the same length: a few launches do not bring the device to its
    sustained clocks (a batched forward's first 50-call loop reads ~6% slower
    than its later ones)."""
    time_loop(fns, device=device, iters=iters)
    runs = sorted(time_loop(fns, device=device, iters=iters) for _ in range(reps))
    return runs[len(runs) // 2]


def time_graph(fns: list[Callable[[], object]], *, stream: torch.cuda.Stream, per_graph: int = 40,
               replays: int = 10, reps: int = 3) -> float:
    """Device-only ms per call: ``per_graph`` calls (cycling through ``fns``)
    captured into one HIP graph on ``stream`` and replayed ``replays`` times
    between two events, the median over ``reps`` such loops. The calls must
    launch on ``stream``. A Python loop of small launches measures the host's
    enqueue time instead (a ctypes call of the C ABI costs ~3.5-5.5 us of host
    time), which hides what the device takes for shapes below that."""
    device = stream.device
    with torch.cuda.stream(stream):
        for f in fns:
            f()
    torch.cuda.synchronize(device)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for i in range(per_graph):
            fns[i % len(fns)]()
    torch.cuda.synchronize(device)
    graph.replay()
    torch.cuda.synchronize(device)
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    runs = []
    with torch.cuda.stream(stream):
        for _ in range(reps):
            start.record()
            for _ in range(replays):
                graph.replay()
            end.record()
            torch.cuda.synchronize(device)
            runs.append(start.elapsed_time(end) / (replays * per_graph))
    del graph
    return sorted(runs)[len(runs) // 2]


@dataclass
class MemoryReport:
    peak_allocated_bytes: int
    workspace_bytes: int
    resident_bytes: int
    incremental_peak_bytes: int
    returned_bytes: int
    allocation_count: int

    def as_dict(self) -> dict:
        return dict(self.__dict__)


def measure_memory(fn: Callable[[], object], *, device: torch.device, resident_bytes: int,
                   output_bytes: int | None = None) -> MemoryReport:
    """Allocator high-water mark of one call minus what it returns: the
    workspace on top of the caller's data (reference harness.py:158-211)."""
    fn()
    torch.cuda.synchronize(device)
    gc.collect()
    torch.cuda.empty_cache()
    base = torch.cuda.memory_allocated(device)
    torch.cuda.reset_peak_memory_stats(device)
    before = torch.cuda.memory_stats(device).get("allocation.all.allocated", 0)
    out = fn()
    torch.cuda.synchronize(device)
    peak = torch.cuda.max_memory_allocated(device)
    after = torch.cuda.memory_stats(device).get("allocation.all.allocated", 0)

    def nbytes(obj) -> int:
        if isinstance(obj, torch.Tensor):
            return obj.numel() * obj.element_size()
        if isinstance(obj, (list, tuple)):
            return sum(nbytes(x) for x in obj)
        return 0

    returned = nbytes(out)
    accounted = returned if output_bytes is None else output_bytes
    inc = max(0, peak - base)
    ws = max(0, inc - accounted)
    del out
    return MemoryReport(resident_bytes + ws, ws, resident_bytes, inc, returned, after - before)


@dataclass
class KernelReport:
    total_kernels: int | None
    total_device_us: float | None
    by_name: dict = field(default_factory=dict)

    def as_dict(self) -> dict:
        return {"total_kernels": self.total_kernels, "total_device_us": self.total_device_us,
                "by_name": self.by_name}


def count_kernels(fn: Callable[[], object], *, device: torch.device, iters: int = 3) -> KernelReport:
    """Device kernels per call, from torch.profiler (reference harness.py:228-292):
    memcpy/memset excluded, an unstable or empty count reported as unavailable."""
    from torch.profiler import ProfilerActivity, profile

    for _ in range(3):
        fn()
    torch.cuda.synchronize(device)
    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        for _ in range(iters):
            fn()
        torch.cuda.synchronize(device)
    by_name: dict[str, dict] = {}
    total, total_us = 0, 0.0
    for evt in prof.key_averages():
        if evt.device_type != torch.autograd.DeviceType.CUDA or evt.count == 0:
            continue
        if evt.key.startswith(("Memcpy", "Memset", "cuda", "hip")):
            continue
        by_name[evt.key] = {"launches_per_call": evt.count / iters,
                            "device_us_per_call": evt.self_device_time_total / iters}
        total += evt.count
        total_us += evt.self_device_time_total
    if total == 0 or total % iters:
        return KernelReport(None, None, {"_unavailable": f"profiler counted {total} kernels over {iters} calls"})
    return KernelReport(total // iters, total_us / iters, by_name)


def achieved_bandwidth_gbps(nbytes: int, ms: float) -> float:
    return nbytes / (ms * 1e-3) / 1e9


# ---------------------------------------------------------------------------
# Per-shape correctness gate of the sweeps
# ---------------------------------------------------------------------------


def float64_operator(v: torch.Tensor, w: torch.Tensor, grad_out: torch.Tensor | None = None,
                     eps: float = 1e-6):
    """out (and dv, dw for ``grad_out``) of the operator in float64 on v's
    device: ``r_n = rsqrt(mean_d v_n^2 + eps)``, ``alpha = softmax_n(r_n <w, v_n>)``,
    ``out = sum_n alpha_n v_n`` (reference src/switchyard/reference.py:130-133),
    gradients by autograd. Written with elementwise products and sums only (no
    batched matrix products), so that it runs on the GPU in float64 at full
    sweep sizes within seconds. The benchmark's comparator, as the reference's
    harness compares every shape with its float64 oracle; the test suite's
    oracle is separate."""
    v64 = v.detach().to(torch.float64).requires_grad_(grad_out is not None)
    w64 = w.detach().to(torch.float64).requires_grad_(grad_out is not None)
    with torch.enable_grad():
        logit = (v64 * w64).sum(-1) * torch.rsqrt(v64.pow(2).mean(-1) + eps)
        alpha = torch.softmax(logit, dim=0)
        out = (alpha.unsqueeze(-1) * v64).sum(0)
        if grad_out is None:
            return out.detach(), None, None
        dv, dw = torch.autograd.grad(out, (v64, w64), grad_out.detach().to(torch.float64))
    return out.detach(), dv, dw


def check_against(got: torch.Tensor, ref: torch.Tensor, *, rel_l2_tol: float) -> dict:
    """Relative L2 error of ``got`` against a float64 ``ref`` and the error the
    float64 values themselves take on when rounded to ``got``'s dtype (the
    dtype floor); the reference's metric (bench/harness.py:295-358)."""
    o = ref.to(torch.float64)
    g = got.to(torch.float64)
    o_norm = o.norm().item()
    rel = (g - o).norm().item() / o_norm if o_norm > 0 else float("inf")
    floor = (o.to(got.dtype).to(torch.float64) - o).norm().item() / o_norm if o_norm > 0 else 0.0
    bad = bool(torch.isnan(got).any().item() or torch.isinf(got).any().item())
    return {"ok": rel <= rel_l2_tol and not bad, "rel_l2": rel, "rel_l2_tol": rel_l2_tol,
            "dtype_floor_rel_l2": floor, "err_vs_dtype_floor": rel / floor if floor > 0 else None,
            "nan_or_inf": bad}


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def environment() -> dict:
    """What produced a number (reference harness.py:365-383), for ROCm."""
    dev = torch.cuda.current_device()
    p = torch.cuda.get_device_properties(dev)
    return {
        "torch": torch.__version__,
        "hip": torch.version.hip,
        "python": platform.python_version(),
        "device_name": p.name,
        "gcn_arch": getattr(p, "gcnArchName", None),
        "cu_count": p.multi_processor_count,
        "device_memory_bytes": p.total_memory,
        "host_cpu": cpu_model(),
        "host_cores": os.cpu_count(),
        "timestamp_utc": time.strftime("%Y-%m-%dT%H:%M:%SZ", time.gmtime()),
    }


#: Files whose content identifies a build of this repository.
_SOURCE_GLOBS = ("blackwell-switchyard_amd/csrc/*.cpp", "blackwell-switchyard_amd/csrc/*.hip",
                 "blackwell-switchyard_amd/csrc/*.hpp", "blackwell-switchyard_amd/csrc/Makefile",
                 "blackwell-switchyard_amd/switchyard/*.py", "include/*.h", "bench.py",
                 "__graft_entry__.py")
BUILD_INFO = "blackwell-switchyard_amd/switchyard/_build_info.json"


def source_fingerprint(root) -> str:
    """SHA-256 over the sources that make the library and the bench (sorted
    relative paths and contents): identifies the code a number came from on
    a machine where no git history exists."""
    import hashlib
    import pathlib

    root = pathlib.Path(root)
    h = hashlib.sha256()
    for pattern in _SOURCE_GLOBS:
        for f in sorted(root.glob(pattern)):
            h.update(str(f.relative_to(root)).encode())
            h.update(b"\0")
            h.update(f.read_bytes())
    return h.hexdigest()


def provenance(root, *, argv, seeds) -> dict:
    """What produced a record (reference bench/harness.py:42-70): the git
    commit and dirty flag recorded when the library was built (the GPU box
    carries no git history), the source fingerprint then and now, argv and
    seeds."""
    import json
    import pathlib

    root = pathlib.Path(root)
    live = source_fingerprint(root)
    info = {}
    try:
        info = json.loads((root / BUILD_INFO).read_text())
    except (OSError, ValueError):
        pass
    commit = repository_commit(str(root)) or info.get("commit")
    return {"commit": commit, "dirty_at_build": info.get("dirty"), "built_at": info.get("built_at"),
            "build_fingerprint": info.get("fingerprint"), "source_fingerprint": live,
            "sources_match_build": info.get("fingerprint") == live if info else None,
            "argv": list(argv), "seeds": seeds}


def repository_commit(path: str) -> str | None:
    try:
        r = subprocess.run(["git", "-C", path, "rev-parse", "HEAD"], capture_output=True, text=True,
                           check=False)
        return r.stdout.strip() or None
    except OSError:
        return None
