"""Long-horizon drift on the MI355X: 100,000 fixed-weight ticks of the native
float32 tick against the float32 oracle.

The protocol is the reference's drift benchmark
(benchmarks/precision_drift.py:23-71,231-282): N=1024, 16,384 candidate edges,
B=4, initial state 0.25, graph-captured 32-tick chunks whose per-tick drives
are staged into the graph's input buffers between replays, and the
"stable_drive" and "slow_adaptation" scenarios with their parameters and
drive formulas.  The drives are computed once on the CPU in float32, so the
native rollout and the oracle read the same values.  Every 1024 ticks all
three states are compared; the test prints the largest difference in each
10,000-tick window and requires every sample within 1e-5.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import dynamics as od
from oracle import runtime as ort
from oracle import topology as otop
from neurosim_gpu import (DendriticDynamics, Dynamics, MatrixRollout,
                          NativeDendriticMatrixRuntime, random_topology, topology_to)

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")
N, EDGES, BATCH, TICKS, CHUNK, SAMPLE, WINDOW = 1024, 16_384, 4, 100_000, 32, 1024, 10_000
BAR = 1e-5

# Scenario parameters of the drift protocol (precision_drift.py:27-37).
SCENARIOS = {
    "stable_drive": dict(weight_scale=0.15, alpha=0.72, gain=0.8, tau_dendrite=4.0,
                         tau_adaptation=20.0, coupling=0.45, adaptation_strength=0.15),
    "slow_adaptation": dict(weight_scale=0.15, alpha=0.72, gain=0.8, tau_dendrite=4.0,
                            tau_adaptation=5000.0, coupling=0.45, adaptation_strength=0.6),
}


def chunk_drives(scenario: str, first_tick: int):
    """[CHUNK, B, N] somatic and dendritic drives for ticks first_tick.. (float32, CPU):
    0.20 + 0.05 sin(2 pi t / 257 + phase) and 0.025 + 0.015 sin(2 pi t / 503 + phase),
    phase = 0.039 n + 0.7 b; slow_adaptation adds 0.15 to the somatic drive and
    gates both on for the first 8000 of every 24000 ticks."""
    t = torch.arange(first_tick, first_tick + CHUNK, dtype=torch.float32).view(-1, 1, 1)
    phase = (0.039 * torch.arange(N, dtype=torch.float32).view(1, 1, -1)
             + 0.7 * torch.arange(BATCH, dtype=torch.float32).view(1, -1, 1))
    soma = 0.20 + 0.05 * torch.sin(t * (2 * math.pi / 257) + phase)
    dendrite = 0.025 + 0.015 * torch.sin(t * (2 * math.pi / 503) + phase)
    if scenario == "slow_adaptation":
        on = ((t % 24000) < 8000).to(torch.float32)
        soma, dendrite = on * (soma + 0.15), on * dendrite
    return soma.contiguous(), dendrite.contiguous()


@pytest.mark.parametrize("scenario", list(SCENARIOS))
def test_100k_tick_drift_against_the_oracle(gpu, scenario):
    print(f"case drift {scenario}: N={N} candidate edges={EDGES} B={BATCH} "
          f"ticks={TICKS}", flush=True)
    torch.set_num_threads(1)
    p = SCENARIOS[scenario]
    seed = 11
    graph = otop.random_graph(N, EDGES, seed=seed, weight_scale=p["weight_scale"])
    topology = random_topology(N, EDGES, device="cpu", seed=seed, weight_scale=p["weight_scale"])
    for name in ("in_rowptr", "in_col", "in_weight"):
        assert np.array_equal(getattr(topology, name).numpy(), getattr(graph, name)), name
    full = lambda value: torch.full((N,), value)
    model = DendriticDynamics.from_time_constants(
        Dynamics(full(p["alpha"]), full(p["gain"])), dt=1.0, tau_dendrite=p["tau_dendrite"],
        tau_adaptation=p["tau_adaptation"], coupling=p["coupling"],
        adaptation_strength=p["adaptation_strength"])
    params = od.from_time_constants(full(p["alpha"]), full(p["gain"]), dt=1.0,
                                    tau_dendrite=p["tau_dendrite"],
                                    tau_adaptation=p["tau_adaptation"], coupling=p["coupling"],
                                    adaptation_strength=p["adaptation_strength"])
    gpu_model = DendriticDynamics(
        Dynamics(model.soma.alpha.to(gpu), model.soma.gain.to(gpu)),
        model.dendrite_decay.to(gpu), model.adaptation_decay.to(gpu), model.coupling.to(gpu),
        model.adaptation_strength.to(gpu))
    initial = torch.full((BATCH, N), 0.25)
    native = NativeDendriticMatrixRuntime(topology_to(topology, gpu), gpu_model, initial.to(gpu))
    oracle = ort.MatrixOracle(graph, params, initial)
    staged = [torch.zeros(CHUNK, BATCH, N, device=gpu) for _ in range(2)]
    rollout = MatrixRollout(native, CHUNK, drive=staged[0], dendritic_drive=staged[1])

    worst_by_window: dict[int, float] = {}
    worst = 0.0
    for first in range(0, TICKS, CHUNK):
        soma, dendrite = chunk_drives(scenario, first)
        rollout.stage(soma.to(gpu), dendrite.to(gpu))
        rollout.run()
        for k in range(CHUNK):
            oracle.step(soma[k], dendrite[k])
        tick = first + CHUNK
        if tick % SAMPLE == 0 or tick == TICKS:
            error = max(float((getattr(rollout, f).cpu() - getattr(oracle, f)).abs().max())
                        for f in FIELDS)
            window = (tick - 1) // WINDOW
            worst_by_window[window] = max(worst_by_window.get(window, 0.0), error)
            worst = max(worst, error)
            if tick % WINDOW < SAMPLE:
                print(f"  {scenario} tick {tick}: max error so far {worst:.3e}", flush=True)
    rows = ", ".join(f"{(w + 1) * WINDOW // 1000}k: {e:.2e}"
                     for w, e in sorted(worst_by_window.items()))
    print(f"drift {scenario}: max |native - oracle| per 10k-tick window: {rows}", flush=True)
    assert all(torch.isfinite(getattr(rollout, f)).all() for f in FIELDS)
    assert worst <= BAR, (scenario, worst)
