"""Performance regression gate over stored sweep results.

Mirrors the reference's ``scripts/check_regression.py``: a local gate (CI has
no MI355X) that compares a benchmark run against a stored baseline and exits
non-zero if any tracked measurement regressed by more than a threshold
(default 7%, outside the run-to-run noise of these kernels and well inside
the 2x a mis-dispatched shape costs). Intended use on the GPU box::

    python bench.py --sweep --dtype bfloat16 --json-out results/sweep_bf16.json
    python bench.py --sweep --dtype float16  --json-out results/sweep_fp16.json
    python bench.py --sweep --dtype float32  --json-out results/sweep_fp32.json
    python -m switchyard.regression            # compare with results/baseline/
    python -m switchyard.regression --accept   # bless the current run

Each results file is ``{"environment": {...}, "dtype": ..., "results": [...]}``
as ``bench.py --sweep`` writes it; a record is keyed by implementation, shape
and dtype. Only the tracked numbers are kept in the baseline.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

REPO = Path(__file__).resolve().parents[2]
RESULTS = REPO / "results"
BASELINE_FILE = RESULTS / "baseline" / "sweep_baseline.json"

#: (record field, human name, lower is better)
TRACKED = [
    ("fwd_us", "forward us", True),
    ("fwd_bwd_us", "fwd+bwd us", True),
    ("fwd_graph_us", "forward us (device)", True),
    ("fwd_bwd_graph_us", "fwd+bwd us (device)", True),
    ("workspace_bytes", "workspace bytes", True),
]

#: Event-timed numbers and their device-only twins (the same calls replayed
#: from a HIP graph). Where both runs carry the twin, it is gated instead: for
#: shapes whose kernels take less than the host's ~4-5 us a call, the
#: event-timed loop measures the host.
DEVICE_TWIN = {"forward us": "forward us (device)", "fwd+bwd us": "fwd+bwd us (device)"}

#: Only these implementations gate; others are information.
GATED = {"switchyard_hip"}

#: Environment fields whose change makes a comparison doubtful.
ENV_FIELDS = ("device_name", "gcn_arch", "torch", "hip")


def record_key(rec: dict, dtype: str | None) -> str:
    q = f"|Q{rec['Q']}" if rec.get("Q") else ""
    return f"{rec.get('impl', 'switchyard_hip')}|N{rec['N']}|B{rec['B']}|T{rec['T']}|D{rec['D']}{q}|{dtype}"


def load_results(results_dir: Path) -> tuple[dict, dict]:
    """All records of ``sweep_*.json`` under ``results_dir`` and the first
    file's environment."""
    out: dict[str, dict] = {}
    env: dict = {}
    for path in sorted(results_dir.glob("sweep_*.json")):
        data = json.loads(path.read_text())
        env = env or data.get("environment", {})
        for r in data.get("results", []):
            if r.get("skipped"):
                continue
            out[record_key(r, data.get("dtype", r.get("dtype")))] = r
    return out, env


def compact(records: dict) -> dict:
    """Keep only the tracked numbers of each record."""
    out = {}
    for key, rec in records.items():
        entry = {name: rec[field] for field, name, _ in TRACKED if rec.get(field) is not None}
        if entry:
            out[key] = entry
    return out


def compare(base: dict, cur: dict, threshold: float, gated: set | None):
    """(regressions, improvements, missing) of a compact current run against
    a compact baseline. A row is (shape, impl, metric, baseline, current, delta),
    delta > 0 meaning worse."""
    regressions, improvements, missing = [], [], []
    for key, b_entry in base.items():
        impl = key.split("|")[0]
        if gated is not None and impl not in gated:
            continue
        c_entry = cur.get(key)
        if c_entry is None:
            missing.append(key)
            continue
        for _, name, lower_better in TRACKED:
            twin = DEVICE_TWIN.get(name)
            if twin is not None and b_entry.get(twin) is not None and c_entry.get(twin) is not None:
                continue
            b, c = b_entry.get(name), c_entry.get(name)
            if b is None or c is None or b == 0:
                continue
            delta = (c - b) / b
            if not lower_better:
                delta = -delta
            row = (" ".join(key.split("|")[1:-1]) + " " + key.split("|")[-1], impl, name, b, c, delta)
            if delta > threshold:
                regressions.append(row)
            elif delta < -threshold:
                improvements.append(row)
    return regressions, improvements, missing


def _show(rows, title) -> None:
    if not rows:
        return
    print(f"\n{title}")
    for shape, impl, name, b, c, d in sorted(rows, key=lambda r: -abs(r[5])):
        print(f"  {shape:30} {impl:16} {name:16} {b:14.3f} -> {c:14.3f}  {100 * d:+7.1f}%")


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--results", type=Path, default=RESULTS, help="directory holding sweep_*.json")
    ap.add_argument("--baseline", type=Path, default=BASELINE_FILE)
    ap.add_argument("--accept", action="store_true", help="bless the current run as the baseline")
    ap.add_argument("--threshold", type=float, default=0.07, help="fractional regression allowed")
    ap.add_argument("--all-impls", action="store_true", help="gate on every implementation")
    args = ap.parse_args(argv)

    cur, cur_env = load_results(args.results)
    if not cur:
        print(f"no sweep_*.json under {args.results}; run bench.py --sweep --json-out first", file=sys.stderr)
        return 2
    if args.accept:
        args.baseline.parent.mkdir(parents=True, exist_ok=True)
        args.baseline.write_text(json.dumps({"environment": cur_env, "metrics": compact(cur)}, indent=1,
                                            sort_keys=True))
        print(f"blessed {len(cur)} measurements into {args.baseline}")
        return 0
    if not args.baseline.exists():
        print(f"no baseline at {args.baseline}; create one with --accept", file=sys.stderr)
        return 2
    stored = json.loads(args.baseline.read_text())
    base_env = stored.get("environment", {})
    for field in ENV_FIELDS:
        if base_env.get(field) != cur_env.get(field):
            print(f"warning: baseline {field}={base_env.get(field)!r} but current {field}="
                  f"{cur_env.get(field)!r}; the comparison may be meaningless")
    regressions, improvements, missing = compare(stored["metrics"], compact(cur), args.threshold,
                                                 None if args.all_impls else GATED)
    _show(improvements, "IMPROVED")
    _show(regressions, "REGRESSED")
    if missing:
        print(f"\nMISSING from current run ({len(missing)}):")
        for key in missing[:10]:
            print(f"  {key}")
        if len(missing) > 10:
            print(f"  ... and {len(missing) - 10} more")
    if regressions:
        print(f"\nFAIL: {len(regressions)} measurement(s) regressed by more than {100 * args.threshold:.0f}%")
        return 1
    print(f"\nOK: no regression beyond {100 * args.threshold:.0f}% ({len(improvements)} improvement(s))")
    return 0


if __name__ == "__main__":
    sys.exit(main())
