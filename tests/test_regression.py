"""The performance regression gate (CPU): the decisions of
``switchyard.regression`` on synthetic results files, mirroring the behaviour
of the reference's scripts/check_regression.py."""

from __future__ import annotations

import json

from switchyard import regression

ENV = {"device_name": "AMD Instinct MI355X", "gcn_arch": "gfx950", "torch": "2.10.0", "hip": "7.0"}


def _rec(n=9, t=4096, fwd=30.0, fb=100.0, ws=8 << 20, impl="switchyard_hip", **kw):
    return dict(impl=impl, N=n, B=1, T=t, D=2048, fwd_us=fwd, fwd_bwd_us=fb, workspace_bytes=ws, **kw)


def _write(d, name, records, dtype="bf16", env=ENV):
    d.mkdir(parents=True, exist_ok=True)
    (d / name).write_text(json.dumps({"environment": env, "dtype": dtype, "results": records}))


def _gate(tmp_path, *extra):
    return regression.main(["--results", str(tmp_path / "results"),
                            "--baseline", str(tmp_path / "results" / "baseline" / "b.json"), *extra])


def test_no_results_and_no_baseline_are_usage_errors(tmp_path, capsys):
    assert _gate(tmp_path) == 2
    _write(tmp_path / "results", "sweep_bf16.json", [_rec()])
    assert _gate(tmp_path) == 2
    assert "--accept" in capsys.readouterr().err


def test_accept_keeps_only_tracked_numbers(tmp_path):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(extra_field=1.0), _rec(n=2, fwd=10.0)])
    assert _gate(tmp_path, "--accept") == 0
    stored = json.loads((tmp_path / "results" / "baseline" / "b.json").read_text())
    assert stored["environment"] == ENV
    entry = stored["metrics"]["switchyard_hip|N9|B1|T4096|D2048|bf16"]
    assert entry == {"forward us": 30.0, "fwd+bwd us": 100.0, "workspace bytes": 8 << 20}
    assert _gate(tmp_path) == 0


def test_regression_beyond_threshold_fails(tmp_path, capsys):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec()])
    _gate(tmp_path, "--accept")
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=33.0)])  # +10%
    assert _gate(tmp_path) == 1
    out = capsys.readouterr().out
    assert "REGRESSED" in out and "forward us" in out and "+10.0%" in out
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=31.5)])  # +5%: noise
    assert _gate(tmp_path) == 0
    assert _gate(tmp_path, "--threshold", "0.03") == 1


def test_improvements_pass_and_are_reported(tmp_path, capsys):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec()])
    _gate(tmp_path, "--accept")
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fb=80.0, ws=0)])
    assert _gate(tmp_path) == 0
    out = capsys.readouterr().out
    assert "IMPROVED" in out and "OK" in out and "(2 improvement(s))" in out  # fwd+bwd and workspace


def test_only_the_gated_implementation_fails_the_gate(tmp_path):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(), _rec(impl="torch_eager", fwd=500.0)])
    _gate(tmp_path, "--accept")
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(), _rec(impl="torch_eager", fwd=900.0)])
    assert _gate(tmp_path) == 0
    assert _gate(tmp_path, "--all-impls") == 1


def test_dtypes_and_batched_records_are_keyed_apart(tmp_path, capsys):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(), _rec(Q=8, fwd=120.0, fb=None, ws=None)])
    _write(tmp_path / "results", "sweep_fp32.json", [_rec(fwd=60.0)], dtype="fp32")
    _gate(tmp_path, "--accept")
    base = json.loads((tmp_path / "results" / "baseline" / "b.json").read_text())["metrics"]
    assert set(base) == {"switchyard_hip|N9|B1|T4096|D2048|bf16", "switchyard_hip|N9|B1|T4096|D2048|Q8|bf16",
                         "switchyard_hip|N9|B1|T4096|D2048|fp32"}
    (tmp_path / "results" / "sweep_fp32.json").unlink()
    assert _gate(tmp_path) == 0
    assert "MISSING from current run (1)" in capsys.readouterr().out


def test_environment_change_warns(tmp_path, capsys):
    _write(tmp_path / "results", "sweep_bf16.json", [_rec()])
    _gate(tmp_path, "--accept")
    _write(tmp_path / "results", "sweep_bf16.json", [_rec()], env=dict(ENV, torch="2.11.0"))
    assert _gate(tmp_path) == 0
    assert "warning: baseline torch='2.10.0'" in capsys.readouterr().out


def test_device_only_twins_are_gated_in_place_of_event_times(tmp_path, capsys):
    """Where both runs carry the graph-replayed (device-only) time, it is
    gated and the event-timed number (the host's time for tiny shapes) is not;
    a run without twins falls back to the event-timed numbers."""
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=5.0, fb=12.0, fwd_graph_us=3.0, fwd_bwd_graph_us=10.0)])
    _gate(tmp_path, "--accept")
    # host jitter: +20% on the event loops, the device times unchanged
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=6.0, fb=14.4, fwd_graph_us=3.0, fwd_bwd_graph_us=10.0)])
    assert _gate(tmp_path) == 0
    # a device-side slowdown fails
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=5.0, fb=12.0, fwd_graph_us=3.0, fwd_bwd_graph_us=11.0)])
    assert _gate(tmp_path) == 1
    assert "fwd+bwd us (device)" in capsys.readouterr().out
    # without twins in the current run the event-timed numbers gate again
    _write(tmp_path / "results", "sweep_bf16.json", [_rec(fwd=6.0, fb=12.0)])
    assert _gate(tmp_path) == 1
