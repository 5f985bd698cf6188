"""Pins of the oracle three-state update.

* Reference-held FP64 probe (results/compartmental_probe_cpu.json, produced by
  experiments/compartmental_probe.py): isolated cells (no edges), five
  parameter variants, 400 ticks of per-tick population means.
* Closed forms from the reference's tests: impulse decay (1-rho_d)tanh(1)rho_d^t
  (test_compartmental.py:73-85), neutral coupling/strength == point model
  exactly (:30-39), boundedness under extreme currents (:207-216).
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np
import torch

from oracle import dynamics as od
from oracle import runtime as ort
from oracle import topology as otop

GOLDEN = Path(__file__).resolve().parent / "golden"


def float32_linspace(start: float, end: float, n: int) -> torch.Tensor:
    """torch.linspace(start, end, n) as the reference's build evaluated it.

    float32 step (end-start)/(n-1); the first half counts up from start, the
    second half down from end.  (This build's torch.linspace rounds some
    entries differently; the probe traces match the two-sided form to 1e-16.)
    """
    f = np.float32
    step = (f(end) - f(start)) / f(n - 1)
    values = [f(start) + step * f(i) if i < n // 2 else f(end) - step * f(n - 1 - i)
              for i in range(n)]
    return torch.from_numpy(np.array(values, dtype=np.float32))


def probe_params(coupling, strength, n=32):
    alpha = torch.full((n,), 0.7, dtype=torch.float64)
    gain = torch.full((n,), 0.8, dtype=torch.float64)
    return od.from_time_constants(alpha, gain, dt=1, tau_dendrite=float32_linspace(2, 8, n),
                                  tau_adaptation=float32_linspace(15, 30, n),
                                  coupling=coupling, adaptation_strength=strength)


def test_reference_probe_traces_fp64():
    probe = json.loads((GOLDEN / "probe_cpu.json").read_text())
    n, batch = 32, 2
    graph = otop.build(n, np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(0, np.float64))
    zero = torch.zeros(n, dtype=torch.float64)
    variants = {"disabled": (zero, zero), "dendrite_only": (0.7, zero),
                "adaptation_only": (zero, 1.0), "combined": (0.7, 1.0)}
    runs = {name: ort.MatrixOracle(graph, probe_params(*cs), torch.zeros(batch, n, dtype=torch.float64))
            for name, cs in variants.items()}
    point_state = torch.zeros(batch, n, dtype=torch.float64)
    alpha = torch.full((n,), 0.7, dtype=torch.float64)
    gain = torch.full((n,), 0.8, dtype=torch.float64)
    for t in range(400):
        drive = 0.6 if 20 <= t < 200 else 0.0
        ddrive = 1.0 if 280 <= t < 290 else 0.0
        for name, run in runs.items():
            run.step(drive, ddrive)
            ref = probe["traces"][name]
            assert ref["drive"][t] == drive and ref["dendritic_drive"][t] == ddrive
            for key, value in (("soma", run.state), ("dendrite", run.dendritic_state),
                               ("adaptation", run.adaptation_state)):
                assert abs(float(value.mean()) - ref[key][t]) <= 1e-14, (name, key, t)
        point_state = od.point_advance(alpha, gain, point_state, torch.zeros_like(point_state), drive)
        assert abs(float(point_state.mean()) - probe["traces"]["point"]["soma"][t]) <= 1e-14
        # neutral compartments reproduce the point model exactly (probe metric 0.0)
        assert torch.equal(runs["disabled"].state, point_state)
    combined = probe["traces"]["combined"]["soma"]
    assert max(combined[20:200]) == probe["metrics"]["combined_step_peak"]


def small_model(n=12, dtype=torch.float64):
    alpha = torch.full((n,), 0.7, dtype=dtype)
    gain = torch.full((n,), 0.8, dtype=dtype)
    return od.from_time_constants(alpha, gain, dt=1.0, tau_dendrite=torch.linspace(2, 5, n),
                                  tau_adaptation=20.0, coupling=0.6, adaptation_strength=0.3)


def test_impulse_decay_closed_form():
    p = small_model()
    p.coupling = torch.ones(12, dtype=torch.float64)
    p.adaptation_strength = torch.zeros(12, dtype=torch.float64)
    zero = torch.zeros(2, 12, dtype=torch.float64)
    s, d, a = od.advance(p, zero, zero, zero, zero, 0.0, 1.0)
    expected = (1 - p.dendrite_decay) * math.tanh(1.0)
    torch.testing.assert_close(d[0], expected)
    for t in range(1, 12):
        s, d, a = od.advance(p, s, d, a, zero)
        torch.testing.assert_close(d[0], expected * p.dendrite_decay ** t)
    assert float(s.sum()) > 0


def test_neutral_parameters_equal_point_model_exactly():
    p = small_model()
    p.coupling = torch.zeros(12, dtype=torch.float64)
    p.adaptation_strength = torch.zeros(12, dtype=torch.float64)
    rng = np.random.default_rng(3)
    s = torch.full((2, 12), 0.2, dtype=torch.float64)
    d = a = torch.zeros_like(s)
    point = s.clone()
    for t in range(30):
        j = torch.from_numpy(rng.standard_normal((2, 12)) * 0.1)
        drive = 0.15 + 0.05 * math.sin(t)
        s, d, a = od.advance(p, s, d, a, j, drive, 0.0)
        point = od.point_advance(p.alpha, p.gain, point, j, drive)
        assert torch.equal(s, point)


def test_bounded_under_extreme_currents():
    p = small_model()
    s = torch.full((2, 12), 0.2, dtype=torch.float64)
    d = a = torch.zeros_like(s)
    for t in range(1500):
        s, d, a = od.advance(p, s, d, a, torch.full_like(s, (-1) ** (t // 40) * 1e4), 0.3, 0.2)
    for value, low in ((s, 0), (a, 0), (d, -1)):
        assert bool((torch.isfinite(value) & (value >= low) & (value <= 1)).all())
