"""PyTorch (reference-backend) runtimes: matrix propagation and PELS.

API of the reference's runtime module (src/neurosim_gpu/runtime.py:12-253).
These are the portable torch paths behind ``--backend reference`` and the
explicit autograd/statistics fallbacks of the native runtimes; the native
runtimes in ``native_compartmental`` run the tick as HIP kernels.

PELS keeps a persistent synaptic current equal to W @ emitted.  A tick
advances the neurons with that current, emits the somatic residuals whose
magnitude reaches theta, and adds W @ delta to the current (matrix path) or
scatters the emitters' out-edges (event path).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch

from .dynamics import Dynamics
from .topology import SparseTopology

PropagationMode = Literal["auto", "matrix", "event"]


def _validate_emission_threshold(theta: torch.Tensor, topology: SparseTopology) -> torch.Tensor:
    """Scalar or per-neuron theta >= 0; +inf only for neurons without out-edges."""
    if theta.ndim == 0:
        theta = theta.expand(topology.n_neurons)
    if theta.shape != (topology.n_neurons,):
        raise ValueError("theta must be scalar or have one value per neuron")
    if bool(torch.any(theta < 0)) or bool(torch.any(torch.isnan(theta))):
        raise ValueError("theta must be non-negative and finite, except +inf for "
                         "zero-outdegree neurons")
    has_edges = topology.out_degree > 0
    if bool(torch.any(torch.isneginf(theta))) or bool(torch.any(torch.isposinf(theta) & has_edges)):
        raise ValueError("infinite theta is allowed only for zero-outdegree neurons")
    return theta


@dataclass(frozen=True)
class RuntimeStats:
    path: str
    active_neurons: int
    active_edges: int


class DenseOracle:
    """Small-network dense semantic oracle (FP64 or FP32)."""

    def __init__(self, topology: SparseTopology, dynamics: Dynamics,
                 initial_state: torch.Tensor) -> None:
        self.topology = topology
        self.dynamics = dynamics
        self.weight = topology.dense_matrix()
        self.state = initial_state

    def step(self, drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        self.state = self.dynamics.advance(self.state, self.state @ self.weight.T, drive)
        return self.state


class MatrixRuntime:
    """One sparse matrix product plus O(B*N) work per tick."""

    def __init__(self, topology: SparseTopology, dynamics: Dynamics,
                 initial_state: torch.Tensor) -> None:
        self.topology = topology
        self.dynamics = dynamics
        self.weight = topology.sparse_matrix()
        self.state = initial_state

    def _propagate(self, source: torch.Tensor) -> torch.Tensor:
        return torch.sparse.mm(self.weight, source.T).T

    def step(self, drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        self.state = self.dynamics.advance(self.state, self._propagate(self.state), drive)
        return self.state


class HybridPELSRuntime(MatrixRuntime):
    """Persistent synaptic current with matrix / event propagation of emitted deltas.

    At entry ``state`` is s_t and ``persistent_current`` is W @ emitted.  A tick
    computes s_{t+1}, then emits so the current is ready for the next tick.
    ``auto`` re-chooses the path every ``policy_interval`` ticks from the
    fraction of edges the emitters touch (a host synchronisation).
    """

    def __init__(self, topology: SparseTopology, dynamics: Dynamics,
                 initial_state: torch.Tensor, *, theta: float | torch.Tensor,
                 propagation: PropagationMode = "auto", event_edge_fraction: float = 0.12,
                 policy_interval: int = 16) -> None:
        super().__init__(topology, dynamics, initial_state)
        if propagation not in ("auto", "matrix", "event"):
            raise ValueError("propagation must be auto, matrix or event")
        if not 0.0 <= event_edge_fraction <= 1.0:
            raise ValueError("event_edge_fraction must be in [0, 1]")
        if policy_interval <= 0:
            raise ValueError("policy_interval must be positive")
        theta = torch.as_tensor(theta, dtype=initial_state.dtype, device=initial_state.device)
        self.theta = _validate_emission_threshold(theta, topology)
        self.propagation = propagation
        self.event_edge_fraction = event_edge_fraction
        self.policy_interval = policy_interval
        self.emitted_state = initial_state.clone()
        self.persistent_current = self._initial_current()
        self._tick = 0
        self._selected_path = "matrix"
        self._weight_version = topology.weight_version

    def _initial_current(self) -> torch.Tensor:
        return self._propagate(self.emitted_state)

    def _select_path(self, active: torch.Tensor, collect_stats: bool) -> tuple[str, int]:
        # The matrix path stays asynchronous; counting active edges syncs the
        # host, so it happens only for statistics or at an auto-policy tick.
        if self.propagation == "matrix" and not collect_stats:
            return "matrix", -1
        policy_tick = self._tick % self.policy_interval == 0
        if self.propagation == "auto" and not policy_tick and not collect_stats:
            return self._selected_path, -1
        pairs = torch.nonzero(active, as_tuple=False)
        if pairs.numel() == 0:
            if self.propagation == "auto":
                self._selected_path = "event"
            return "idle", 0
        active_edges = int(self.topology.out_degree[pairs[:, 1]].sum().item())
        if self.propagation != "auto":
            return self.propagation, active_edges
        if policy_tick:
            total = max(self.topology.n_edges * self.state.shape[0], 1)
            self._selected_path = ("event" if active_edges / total < self.event_edge_fraction
                                   else "matrix")
        return self._selected_path, active_edges

    def _event_propagate(self, emitted_delta: torch.Tensor, active: torch.Tensor) -> torch.Tensor:
        """Scatter the emitters' out-edges: sum_e delta[b, src] * weight[e] into dst."""
        pairs = torch.nonzero(active, as_tuple=False)
        batch, source = pairs[:, 0], pairs[:, 1]
        degree = self.topology.out_degree[source]
        owner = torch.repeat_interleave(torch.arange(source.numel(), device=source.device), degree)
        first = torch.cumsum(degree, dim=0) - degree
        within = (torch.arange(int(degree.sum().item()), device=source.device)
                  - torch.repeat_interleave(first, degree))
        edge = self.topology.out_rowptr[source[owner]] + within
        flat_target = batch[owner] * self.topology.n_neurons + self.topology.dst[edge]
        value = emitted_delta[batch[owner], source[owner]] * self.topology.weight[edge]
        result = torch.zeros_like(self.persistent_current).flatten()
        result.index_add_(0, flat_target, value)
        return result.view_as(self.persistent_current)

    def step(self, drive: torch.Tensor | float = 0.0, *, collect_stats: bool = False):
        self._refresh_current()
        next_state = self.dynamics.advance(self.state, self.persistent_current, drive)
        return self._emit(next_state, collect_stats=collect_stats)

    def _refresh_current(self) -> None:
        """Recompute W @ emitted after a versioned weight change."""
        if self._weight_version != self.topology.weight_version:
            self.persistent_current = self._propagate(self.emitted_state).contiguous()
            self._weight_version = self.topology.weight_version

    def _emit(self, next_state: torch.Tensor, *, collect_stats: bool):
        """Commit somatic activity after the compartments have advanced."""
        residual = next_state - self.emitted_state
        active = residual.detach().abs() >= self.theta
        emitted_delta = torch.where(active, residual, torch.zeros_like(residual))
        path, active_edges = self._select_path(active, collect_stats)
        if path == "matrix":
            current_delta = self._propagate(emitted_delta)
        elif path == "event":
            current_delta = self._event_propagate(emitted_delta, active)
        else:
            current_delta = torch.zeros_like(self.persistent_current)
        self.persistent_current = self.persistent_current + current_delta
        self.emitted_state = self.emitted_state + emitted_delta
        self.state = next_state
        self._tick += 1
        if not collect_stats:
            return self.state
        return self.state, RuntimeStats(path=path, active_neurons=int(active.sum().item()),
                                        active_edges=active_edges)
