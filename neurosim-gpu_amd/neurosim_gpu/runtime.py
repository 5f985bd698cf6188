"""Portable PyTorch runtimes: a dense oracle, matrix propagation and PELS.

Public surface of the reference's runtime module
(src/neurosim_gpu/runtime.py:12-253): ``RuntimeStats``, ``DenseOracle``,
``MatrixRuntime`` and ``HybridPELSRuntime`` with their constructor arguments,
``step`` signatures and error messages.  They are the torch paths behind
``--backend reference`` and the explicit autograd / statistics fallbacks of
the native runtimes; the native runtimes run the tick as HIP kernels.

PELS (propagate emitted local state) keeps a persistent synaptic current
equal to W @ e, where e is the last emitted copy of the state.  A tick
advances the neurons with that current, emits every somatic residual
|s' - e| >= theta, and brings the current up to date by adding the product of
the emitted deltas: a sparse matrix product, or a scatter of the emitters'
out-edges when few neurons emit.  The choice of propagation is made by a
``_PathPolicy`` (below), which needs a host synchronisation and so samples
activity only every ``policy_interval`` ticks.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Literal

import torch

from .dynamics import Dynamics
from .topology import SparseTopology

PropagationMode = Literal["auto", "matrix", "event"]


@dataclass(frozen=True)
class RuntimeStats:
    """What a PELS tick did: the propagation used and how much activity it moved."""

    path: str
    active_neurons: int
    active_edges: int


def emission_threshold(theta, topology: SparseTopology, like: torch.Tensor) -> torch.Tensor:
    """theta as one value per neuron on ``like``'s device and dtype.

    Reference rule (runtime.py:15-35): every value non-negative and not NaN;
    +inf (never emit) only where a neuron has no out-edges, since an emitter
    with edges would otherwise starve its targets silently.
    """
    value = torch.as_tensor(theta, dtype=like.dtype, device=like.device)
    per_neuron = value.expand(topology.n_neurons) if value.ndim == 0 else value
    if per_neuron.shape != (topology.n_neurons,):
        raise ValueError("theta must be scalar or have one value per neuron")
    if bool((torch.isnan(per_neuron) | (per_neuron < 0)).any()):
        raise ValueError("theta must be non-negative and finite, except +inf for "
                         "zero-outdegree neurons")
    if bool((torch.isposinf(per_neuron) & (topology.out_degree > 0)).any()):
        raise ValueError("infinite theta is allowed only for zero-outdegree neurons")
    return per_neuron


def scatter_out_edges(topology: SparseTopology, delta: torch.Tensor,
                      active: torch.Tensor) -> torch.Tensor:
    """Sum over the out-edges of every active (column, neuron) pair of
    delta[column, neuron] * weight[edge] into [column, destination].

    The active pairs' out-edge lists are consecutive runs of the source-major
    edge array; they are laid end to end, so the k-th edge of the expansion is
    out_rowptr[source] + (k - first position of its pair).  Contributions are
    added pair by pair, edges in out_rowptr order.
    """
    columns, sources = torch.nonzero(active, as_tuple=True)
    degree = topology.out_degree[sources]
    total = int(degree.sum().item())
    result = torch.zeros(delta.numel(), dtype=delta.dtype, device=delta.device)
    if total == 0:
        return result.view_as(delta)
    owner = torch.repeat_interleave(degree, output_size=total)
    start_of_pair = torch.cumsum(degree, 0) - degree
    edge = (torch.arange(total, device=delta.device)
            + (topology.out_rowptr[sources] - start_of_pair)[owner])
    emitted = delta[columns, sources]
    target = columns[owner] * topology.n_neurons + topology.dst[edge]
    result.index_add_(0, target, emitted[owner] * topology.weight[edge])
    return result.view_as(delta)


class _PathPolicy:
    """Chooses each PELS tick's propagation (reference runtime.py:129-165).

    A fixed mode is used as is; edges are counted (a host synchronisation)
    only when statistics are asked for.  ``auto`` samples activity every
    ``interval`` ticks: emitters touching less than ``fraction`` of the B*M
    edge slots choose the event scatter, more choose the matrix product, and
    the choice holds until the next sample.  A tick with no emitter is idle;
    under ``auto`` it also selects the event path.
    """

    def __init__(self, mode: str, fraction: float, interval: int) -> None:
        self.mode, self.fraction, self.interval = mode, fraction, interval
        self.selected = "matrix"

    def choose(self, tick: int, active: torch.Tensor, topology: SparseTopology,
               collect_stats: bool) -> tuple[str, int]:
        """(path, active out-edges or -1 when they were not counted)."""
        sample = tick % self.interval == 0
        if not collect_stats:
            if self.mode == "matrix":
                return "matrix", -1
            if self.mode == "auto" and not sample:
                return self.selected, -1
        sources = torch.nonzero(active, as_tuple=True)[1]
        if sources.numel() == 0:
            if self.mode == "auto":
                self.selected = "event"
            return "idle", 0
        edges = int(topology.out_degree[sources].sum().item())
        if self.mode != "auto":
            return self.mode, edges
        if sample:
            slots = max(topology.n_edges * active.shape[0], 1)
            self.selected = "event" if edges / slots < self.fraction else "matrix"
        return self.selected, edges


class DenseOracle:
    """Small-network semantic oracle: the dense matrix, in the state's dtype."""

    def __init__(self, topology: SparseTopology, dynamics: Dynamics,
                 initial_state: torch.Tensor) -> None:
        self.topology, self.dynamics = topology, dynamics
        self.weight = topology.dense_matrix()
        self.state = initial_state

    def step(self, drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        current = torch.matmul(self.state, self.weight.transpose(0, 1))
        self.state = self.dynamics.advance(self.state, current, drive)
        return self.state


class MatrixRuntime:
    """One sparse (CSR) product W @ s plus O(B*N) neuron work per tick."""

    def __init__(self, topology: SparseTopology, dynamics: Dynamics,
                 initial_state: torch.Tensor) -> None:
        self.topology, self.dynamics = topology, dynamics
        self.weight = topology.sparse_matrix()
        self.state = initial_state

    def _propagate(self, source: torch.Tensor) -> torch.Tensor:
        """[B,N] -> [B,N]: row b of the result is W @ source[b]."""
        return torch.sparse.mm(self.weight, source.transpose(0, 1)).transpose(0, 1)

    def step(self, drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        self.state = self.dynamics.advance(self.state, self._propagate(self.state), drive)
        return self.state


class HybridPELSRuntime(MatrixRuntime):
    """Persistent current W @ emitted, updated by matrix or event propagation.

    On entry to a tick ``state`` is s_t and ``persistent_current`` is
    W @ ``emitted_state``.  The tick computes s_{t+1} (``_advance_soma``, which
    subclasses replace), then ``_commit`` emits, so the current is ready for
    the next tick.  Which neurons emit is decided on detached values; the
    emitted values themselves stay differentiable.
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
        self.theta = emission_threshold(theta, topology, initial_state)
        self.propagation = propagation
        self.event_edge_fraction = event_edge_fraction
        self.policy_interval = policy_interval
        self._policy = _PathPolicy(propagation, event_edge_fraction, policy_interval)
        self.emitted_state = initial_state.clone()
        self.persistent_current = self._initial_current()
        self._tick = 0
        self._weight_version = topology.weight_version

    def _initial_current(self) -> torch.Tensor:
        return self._propagate(self.emitted_state)

    def _refresh_current(self) -> None:
        """After a versioned weight change, W @ emitted is recomputed whole."""
        if self._weight_version == self.topology.weight_version:
            return
        self.persistent_current = self._propagate(self.emitted_state).contiguous()
        self._weight_version = self.topology.weight_version

    def _advance_soma(self, drive, **_) -> torch.Tensor:
        return self.dynamics.advance(self.state, self.persistent_current, drive)

    def step(self, drive: torch.Tensor | float = 0.0, *, collect_stats: bool = False):
        self._refresh_current()
        return self._commit(self._advance_soma(drive), collect_stats=collect_stats)

    def _commit(self, next_state: torch.Tensor, *, collect_stats: bool):
        """Emit the residuals that reach theta, propagate them, advance the tick."""
        residual = next_state - self.emitted_state
        active = residual.detach().abs() >= self.theta
        delta = torch.where(active, residual, residual.new_zeros(()))
        path, edges = self._policy.choose(self._tick, active, self.topology, collect_stats)
        if path == "matrix":
            self.persistent_current = self.persistent_current + self._propagate(delta)
        elif path == "event":
            self.persistent_current = (self.persistent_current
                                       + scatter_out_edges(self.topology, delta, active))
        else:
            # idle: nothing emitted; the addition keeps the current a fresh tensor
            self.persistent_current = self.persistent_current + torch.zeros_like(
                self.persistent_current)
        self.emitted_state = self.emitted_state + delta
        self.state = next_state
        self._tick += 1
        if not collect_stats:
            return self.state
        return self.state, RuntimeStats(path=path, active_neurons=int(active.sum().item()),
                                        active_edges=edges)
