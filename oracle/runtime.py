"""Oracle matrix and PELS ticks on the CPU (test infrastructure only).

MatrixOracle restates DendriticMatrixRuntime.step at FP32 (reference
compartmental.py:288-293 on runtime.py:78-79): one torch CSR sparse product
over the destination-major view, then the three-state update.

PelsOracle restates DendriticPELSRuntime with propagation="matrix" (reference
compartmental.py:322-348, runtime.py:96-127,217-253): the compartments advance
every tick with the persistent current; residual = s' - emitted;
active = |residual| >= theta; current += W @ delta; emitted += delta.

Pins: tests/test_oracle_runtime.py checks both against an FP64 dense
recurrence written from the model equations (reference test_compartmental.py:
41-71), PELS invariants (|s - emitted| < theta, current == W @ emitted;
test_compartmental.py:126-137) and the reference-held brainwaves trajectory.
"""

from __future__ import annotations

import numpy as np
import torch

from .dynamics import Params, advance
from .topology import Graph


def csr_matrix(graph: Graph, dtype: torch.dtype = torch.float32,
               in_weight: np.ndarray | None = None) -> torch.Tensor:
    values = graph.in_weight if in_weight is None else in_weight
    return torch.sparse_csr_tensor(
        torch.from_numpy(np.ascontiguousarray(graph.in_rowptr)),
        torch.from_numpy(np.ascontiguousarray(graph.in_col)),
        torch.from_numpy(np.ascontiguousarray(values)).to(dtype),
        size=(graph.n, graph.n), check_invariants=False)


def propagate(matrix: torch.Tensor, source: torch.Tensor) -> torch.Tensor:
    """J = W @ S for S [B,N] (reference runtime.py:78-79)."""
    return torch.sparse.mm(matrix, source.T).T


class MatrixOracle:
    def __init__(self, graph: Graph, params: Params, initial_state: torch.Tensor, *,
                 in_weight: np.ndarray | None = None) -> None:
        dtype = initial_state.dtype
        self.matrix = csr_matrix(graph, dtype, in_weight)
        self.params = params
        self.state = initial_state.clone()
        self.dendritic_state = torch.zeros_like(self.state)
        self.adaptation_state = torch.zeros_like(self.state)

    def step(self, drive=0.0, dendritic_drive=0.0) -> torch.Tensor:
        current = propagate(self.matrix, self.state)
        self.state, self.dendritic_state, self.adaptation_state = advance(
            self.params, self.state, self.dendritic_state, self.adaptation_state,
            current, drive, dendritic_drive)
        return self.state


class PelsOracle:
    def __init__(self, graph: Graph, params: Params, initial_state: torch.Tensor, *,
                 theta) -> None:
        dtype = initial_state.dtype
        self.matrix = csr_matrix(graph, dtype)
        self.params = params
        theta = torch.as_tensor(theta, dtype=dtype)
        self.theta = theta.expand(graph.n) if theta.ndim == 0 else theta
        self.state = initial_state.clone()
        self.dendritic_state = torch.zeros_like(self.state)
        self.adaptation_state = torch.zeros_like(self.state)
        self.emitted_state = self.state.clone()
        self.persistent_current = propagate(self.matrix, self.emitted_state)
        self.last_active = torch.zeros_like(self.state, dtype=torch.bool)

    def step(self, drive=0.0, dendritic_drive=0.0) -> torch.Tensor:
        state, self.dendritic_state, self.adaptation_state = advance(
            self.params, self.state, self.dendritic_state, self.adaptation_state,
            self.persistent_current, drive, dendritic_drive)
        residual = state - self.emitted_state
        active = residual.abs() >= self.theta
        delta = torch.where(active, residual, torch.zeros_like(residual))
        self.persistent_current = self.persistent_current + propagate(self.matrix, delta)
        self.emitted_state = self.emitted_state + delta
        self.state = state
        self.last_active = active
        return self.state


def dense_recurrence(graph: Graph, params: Params, initial_state: np.ndarray, ticks: int,
                     drive: float, dendritic_drive: float) -> list[np.ndarray]:
    """FP64 dense restatement written from the model equations, for pinning."""
    w = graph.dense(np.float64)
    p = [np.asarray(v, dtype=np.float64) for v in params.as_list()]
    alpha, gain, rho_d, rho_a, c, k = p
    s = np.asarray(initial_state, dtype=np.float64)
    d = np.zeros_like(s)
    a = np.zeros_like(s)
    out = []
    for _ in range(ticks):
        j = s @ w.T
        d = rho_d * d + (1 - rho_d) * np.tanh(j + dendritic_drive)
        u = (1 - c) * j + c * d - k * a
        s = np.clip(alpha * s + (1 - alpha) * gain * np.tanh(u + drive), 0, 1)
        a = rho_a * a + (1 - rho_a) * s
        out.append((s.copy(), d.copy(), a.copy()))
    return out
