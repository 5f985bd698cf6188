"""The reference benchmark's own acceptance check at its five shapes.

benchmarks/compartmental.py:56-117 builds each graph (random_topology, seed 23,
on the GPU), model and runtime under torch.inference_mode, steps the torch and
native runtimes through the same eager inputs (initial state .2, drive
.2 + .1 sin(0.11 t), dendritic drive .1, theta .02) and then asserts the native
states against the torch ones: rtol 2e-4 / atol 2e-5 for the matrix tick,
atol 2e-3 for PELS (an empirical bound: threshold crossings may move by a
rounding).  Here 130 ticks stand for its 30 warm-up and 700 timed ones, and the
native PELS tick runs in all three propagations.
"""

from __future__ import annotations

import math

import pytest
import torch

from neurosim_gpu import (DendriticDynamics, DendriticMatrixRuntime, DendriticPELSRuntime,
                          Dynamics, NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime,
                          random_topology)

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


@pytest.mark.parametrize("n,candidates,batch", [(4096, 65_536, 1), (50_000, 1_000_000, 1),
                                                (50_000, 1_000_000, 8),
                                                (166_000, 10_000_000, 1),
                                                (166_000, 25_000_000, 1)])
def test_reference_benchmark_parity(gpu, n, candidates, batch):
    ticks = 130
    print(f"case benchmark protocol N={n} candidates={candidates} B={batch} ticks={ticks}",
          flush=True)
    with torch.inference_mode():
        graph = random_topology(n, candidates, device=gpu, seed=23)
        soma = Dynamics(torch.full((n,), .72, device=gpu), torch.full((n,), .8, device=gpu))
        model = DendriticDynamics.from_time_constants(soma, dt=1, tau_dendrite=4,
                                                      tau_adaptation=25)
        initial = torch.full((batch, n), .2, device=gpu)
        reference = DendriticMatrixRuntime(graph, model, initial.clone())
        reference_pels = DendriticPELSRuntime(graph, model, initial.clone(), theta=.02,
                                              propagation="matrix")
        native = NativeDendriticMatrixRuntime(graph, model, initial.clone())
        pels = {p: NativeDendriticPELSRuntime(graph, model, initial.clone(), theta=.02,
                                              propagation=p) for p in ("event", "matrix", "auto")}
        runtimes = (reference, reference_pels, native, *pels.values())
        for t in range(ticks):
            for runtime in runtimes:
                runtime.step(.2 + .1 * math.sin(t * .11), dendritic_drive=.1)
        worst = {}
        for f in FIELDS:
            torch.testing.assert_close(getattr(native, f), getattr(reference, f),
                                       rtol=2e-4, atol=2e-5)
            worst["matrix tick"] = max(worst.get("matrix tick", 0.0), float(
                (getattr(native, f) - getattr(reference, f)).abs().max()))
            for name, runtime in pels.items():
                torch.testing.assert_close(getattr(runtime, f), getattr(reference_pels, f),
                                           rtol=0, atol=2e-3)
                key = f"PELS {name}"
                worst[key] = max(worst.get(key, 0.0), float(
                    (getattr(runtime, f) - getattr(reference_pels, f)).abs().max()))
        assert bool(torch.isfinite(native.state).all())
    print(f"benchmark protocol N={n} B={batch} ({graph.n_edges} edges, kernel {native.kernel}): "
          + ", ".join(f"{k} {v:.2e}" for k, v in worst.items()), flush=True)
