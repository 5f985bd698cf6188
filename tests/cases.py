"""Shared builders for parity tests: one graph, two independent constructions.

The product graph comes from neurosim_gpu.random_topology on the CPU (then
copied to the GPU); the oracle graph from oracle.topology on the same draws.
The CPU tests assert the two are bitwise equal; here both are built and the
equality is re-checked for the arrays the kernels read.
"""

from __future__ import annotations

import sys
from dataclasses import dataclass

import numpy as np
import torch

from oracle import dynamics as od
from oracle import topology as otop
from neurosim_gpu import DendriticDynamics, Dynamics, random_topology, topology_to


@dataclass
class Case:
    graph: otop.Graph              # oracle graph (numpy, CPU)
    topology: object               # product SparseTopology on the GPU
    model: DendriticDynamics       # product parameters on the GPU
    params: od.Params              # oracle parameters (CPU)


def model_to(model: DendriticDynamics, device) -> DendriticDynamics:
    return DendriticDynamics(Dynamics(model.soma.alpha.to(device), model.soma.gain.to(device)),
                             model.dendrite_decay.to(device), model.adaptation_decay.to(device),
                             model.coupling.to(device), model.adaptation_strength.to(device))


def standard_model(n: int) -> tuple[DendriticDynamics, od.Params]:
    """alpha .72, gain .8, dt 1, tau_d 4, tau_a 25, c .5, k .2 (every config)."""
    soma = Dynamics(torch.full((n,), .72), torch.full((n,), .8))
    model = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4.,
                                                  tau_adaptation=25., coupling=.5,
                                                  adaptation_strength=.2)
    params = od.from_time_constants(torch.full((n,), .72), torch.full((n,), .8), dt=1.,
                                    tau_dendrite=4., tau_adaptation=25., coupling=.5,
                                    adaptation_strength=.2)
    return model, params


def reference_test_model(n: int) -> tuple[DendriticDynamics, od.Params]:
    """Heterogeneous parameters of the reference's native tests (test_native_compartmental.py:25-33)."""
    soma = Dynamics(torch.linspace(0.4, 0.95, n), torch.full((n,), 0.8))
    model = DendriticDynamics.from_time_constants(soma, dt=1, tau_dendrite=torch.linspace(2, 8, n),
                                                  tau_adaptation=25, coupling=0.6,
                                                  adaptation_strength=0.3)
    params = od.from_time_constants(torch.linspace(0.4, 0.95, n), torch.full((n,), 0.8), dt=1,
                                    tau_dendrite=torch.linspace(2, 8, n), tau_adaptation=25,
                                    coupling=0.6, adaptation_strength=0.3)
    return model, params


def make_case(n: int, m: int, seed: int, device, kind: str = "standard") -> Case:
    graph = otop.random_graph(n, m, seed=seed)
    topology_cpu = random_topology(n, m, device="cpu", seed=seed)
    for name in ("in_rowptr", "in_col", "in_weight", "out_rowptr", "dst", "out_weight_index"):
        assert np.array_equal(getattr(topology_cpu, name).numpy(), getattr(graph, name)), name
    model, params = (standard_model if kind == "standard" else reference_test_model)(n)
    for mine, theirs in zip((model.soma.alpha, model.soma.gain, model.dendrite_decay,
                             model.adaptation_decay, model.coupling, model.adaptation_strength),
                            params.as_list()):
        assert torch.equal(mine, theirs)
    return Case(graph, topology_to(topology_cpu, device), model_to(model, device), params)


def max_err(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a.detach().float().cpu() - b.detach().float().cpu()).abs().max()) if a.numel() else 0.0


def column_drive(batch: int, seed: int = 1) -> torch.Tensor:
    """Per-column drive U(0, 0.4) of shape [B, 1] from a CPU generator."""
    return torch.rand((batch, 1), generator=torch.Generator().manual_seed(seed)) * 0.4


def progress(message: str) -> None:
    """A line on the process's real stderr, past pytest's capture: long host
    phases of a GPU test (graph builds, oracle runs) show that they advance."""
    print(f"[progress] {message}", file=sys.__stderr__, flush=True)
