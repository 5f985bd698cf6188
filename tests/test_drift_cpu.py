"""Drift protocol host logic against the reference's own drift results.

tests/golden/drift.npz and drift_summary.json hold what the reference's drift
benchmark wrote (results/precision_drift.json.gz, seed 11 of each scenario):
its schedule of sample ticks, the per-sample RMSE and max-abs curves of fp16,
fp8 and NVFP4 against FP32, and the summary figures it computed from them
(benchmarks/precision_drift.py:40-48,202-227).  Feeding those curves to
``neurosim_gpu.drift.summarize`` must give back the reference's figures.  The
time-weighted windows pin the trapezoid rule over the squared RMSE (a mean of
the RMSE itself, a left-endpoint rule or an unweighted mean of the samples
each miss by more than 1e-4 relative); both window ends, ticks 20,000 and
80,000, are sample ticks of this schedule.  The threshold ticks pin the ">="
crossing rule.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from neurosim_gpu import drift

GOLDEN = Path(__file__).resolve().parent / "golden"
SUMMARY = json.loads((GOLDEN / "drift_summary.json").read_text())
ARRAYS = np.load(GOLDEN / "drift.npz")
REF_MODES = ("fp16", "fp8", "nvfp4")


def reference_samples(scenario: str) -> list[dict]:
    rmse, max_abs = ARRAYS[f"{scenario}_s11_rmse"], ARRAYS[f"{scenario}_s11_max_abs"]
    return [{mode: {field: {"rmse": float(rmse[m, f, i]), "max_abs": float(max_abs[m, f, i])}
                    for f, field in enumerate(drift.FIELDS)}
             for m, mode in enumerate(REF_MODES)}
            for i in range(rmse.shape[2])]


def test_sample_ticks_match_the_reference_schedule():
    ticks = drift.sample_ticks(SUMMARY["steps"], SUMMARY["sample_interval"])
    assert ticks == ARRAYS["ticks"].tolist()
    assert len(ticks) == 429


@pytest.mark.parametrize("steps,interval", [(1, 1), (7, 3), (24_001, 5000), (50_000, 256)])
def test_sample_ticks_small_cases(steps, interval):
    ticks = drift.sample_ticks(steps, interval)
    assert ticks == sorted(set(ticks)) and ticks[0] == 0 and ticks[-1] == steps
    assert set(range(interval, steps + 1, interval)) <= set(ticks)
    for start in range(0, steps + 1, drift.GATE_PERIOD):
        for edge in (start, start + drift.GATE_ON):
            assert {t for t in (edge - 1, edge, edge + 1) if 0 <= t <= steps} <= set(ticks)


def test_sample_ticks_rejects_empty_runs():
    for steps, interval in ((0, 256), (10, 0)):
        with pytest.raises(ValueError):
            drift.sample_ticks(steps, interval)


@pytest.mark.parametrize("scenario", ["stable_drive", "slow_adaptation", "recurrent_stress"])
def test_summarize_reproduces_the_reference_summary(scenario):
    ticks = ARRAYS["ticks"].tolist()
    ours = drift.summarize(ticks, reference_samples(scenario), SUMMARY["steps"])
    theirs = SUMMARY["cases"][scenario]
    for mode in REF_MODES:
        for field in drift.FIELDS:
            got, want = ours[mode][field], theirs[mode][field]
            for key in ("peak_sampled_rmse", "peak_sampled_max_abs"):
                assert got[key] == want[key], (scenario, mode, field, key)
            for key in ("early_20_percent_time_weighted_rmse",
                        "late_20_percent_time_weighted_rmse", "late_to_early_rmse_ratio"):
                if want[key] is None:
                    assert got[key] is None, (scenario, mode, field, key)
                else:
                    assert math.isclose(got[key], want[key], rel_tol=1e-12, abs_tol=1e-300), \
                        (scenario, mode, field, key, got[key], want[key])
            assert got["first_sampled_rmse_threshold_tick"] == \
                want["first_sampled_rmse_threshold_tick"], (scenario, mode, field)


def test_window_rms_closed_forms():
    # A constant curve's window RMS is the constant; a curve whose square rises
    # linearly from 0 to c^2 over [0, T] has RMS c / sqrt(2) over the whole span.
    assert math.isclose(drift._window_rms([0, 10, 20], [3.0, 3.0, 3.0], 2, 17), 3.0)
    assert math.isclose(drift._window_rms([0, 100], [0.0, 2.0], 0, 100), 2.0 / math.sqrt(2))
    # The second half of that ramp: mean of t/100 * 4 over [50, 100] is 3.
    assert math.isclose(drift._window_rms([0, 100], [0.0, 2.0], 50, 100), math.sqrt(3.0))
    assert drift._window_rms([0, 100], [1.0, 1.0], 40, 40) == 0.0


def test_error_statistics_and_bounds():
    base = torch.zeros(2, 3)
    candidate = torch.tensor([[0.0, 3.0, 0.0], [0.0, -4.0, 0.0]])
    stats = drift.error_statistics(candidate, base)
    assert stats == {"mae": 7 / 6, "rmse": math.sqrt(25 / 6), "max_abs": 4.0, "bias": -1 / 6}
    ok = torch.full((2, 3), 0.5)
    assert drift.state_bounds_hold(ok, -ok, ok)
    assert not drift.state_bounds_hold(ok + 0.6, ok, ok)
    assert not drift.state_bounds_hold(ok, ok * 2.1, ok)
    assert not drift.state_bounds_hold(ok, ok, ok.clone().fill_(float("nan")))


def test_scenario_drives_follow_the_protocol():
    neurons, batch = 37, 3
    for name in drift.SCENARIOS:
        soma, dendritic = drift.scenario_drives(name, 100, 5, neurons, batch)
        assert soma.shape == dendritic.shape == (5, batch, neurons)
        assert soma.dtype == dendritic.dtype == torch.float32
        assert soma.is_contiguous() and dendritic.is_contiguous()
    phase = 0.039 * 5 + 0.7 * 2     # neuron 5, batch row 2
    soma, dendritic = drift.scenario_drives("stable_drive", 1000, 1, neurons, batch)
    assert math.isclose(float(soma[0, 2, 5]), 0.20 + 0.05 * math.sin(1000 * 2 * math.pi / 257 + phase),
                        abs_tol=2e-6)
    assert math.isclose(float(dendritic[0, 2, 5]),
                        0.025 + 0.015 * math.sin(1000 * 2 * math.pi / 503 + phase), abs_tol=2e-6)
    soma, dendritic = drift.scenario_drives("recurrent_stress", 0, 4, neurons, batch)
    assert torch.equal(soma[0], soma[3]) and not bool(dendritic.any())
    assert math.isclose(float(soma[1, 2, 5]), 0.13 + 0.08 * math.sin(phase), abs_tol=2e-6)
    # slow_adaptation: inputs on for ticks [0, 8000) of every 24,000, offset by 0.15.
    gate = drift.GATE_ON
    soma, dendritic = drift.scenario_drives("slow_adaptation", gate - 1, 3, neurons, batch)
    plain, _ = drift.scenario_drives("stable_drive", gate - 1, 3, neurons, batch)
    assert torch.allclose(soma[0], plain[0] + 0.15)
    assert not bool(soma[1:].any()) and not bool(dendritic[1:].any())
    soma, _ = drift.scenario_drives("slow_adaptation", drift.GATE_PERIOD, 1, neurons, batch)
    assert bool((soma > 0).all())
    with pytest.raises(ValueError):
        drift.scenario_drives("no_such_scenario", 0, 1, neurons, batch)
