"""Oracle gradients of the matrix tick (test infrastructure only).

The reference obtains tick gradients by autograd through its torch step
(native_compartmental.py:104-108 falls back to it; the step is
compartmental.py:152-183 on runtime.py:78-79).  Here the same quantities come
from float64 autograd through this oracle's own update (oracle.dynamics.advance)
on the *dense* weight matrix: j = s @ W^T with W[row, col] set from the CSR.
No part of the shipped package is involved.  The gradient of a CSR weight is
the dense gradient at its (row, col) entry, read out in CSR order.

``tick_gradients`` runs ``ticks`` ticks from given states and drives and
returns the gradients of the loss sum(s' * ps) + sum(d' * pd) + sum(a' * pa)
with respect to the CSR weights, the three initial states, tensor drives and
the six parameter vectors (per neuron).

Pins (tests/test_oracle_grad.py), as the reference's own gradient test does
(tests/test_compartmental.py:139-170): central finite differences of the same
float64 tick at sampled entries of every gradient, and the closed form of one
tick's drive derivative, (1-alpha)*gain*(1 - tanh(u + drive)^2) times the
soma probe, where the clamp is inactive.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from .dynamics import Params, advance
from .topology import Graph

PARAM_NAMES = ("alpha", "gain", "rho_d", "rho_a", "coupling", "strength")


@dataclass
class TickInputs:
    """Float64 inputs of a tick sequence; drives are arrays (any shape that
    broadcasts to [B, N]) or numbers."""

    state: np.ndarray
    dendrite: np.ndarray
    adaptation: np.ndarray
    drive: np.ndarray | float
    dendritic: np.ndarray | float
    params: dict                  # PARAM_NAMES -> [N] arrays
    probe: dict                   # "s", "d", "a" -> [B, N] loss weights


def dense_weights(graph: Graph, in_weight: np.ndarray | None = None) -> torch.Tensor:
    values = graph.in_weight if in_weight is None else in_weight
    w = torch.zeros(graph.n, graph.n, dtype=torch.float64)
    rows = np.repeat(np.arange(graph.n), np.diff(graph.in_rowptr))
    w[torch.from_numpy(rows), torch.from_numpy(graph.in_col.astype(np.int64))] = \
        torch.from_numpy(np.asarray(values, np.float64))
    return w


def _rollout(graph: Graph, w: torch.Tensor, leaves: dict, ticks: int):
    p = Params(*(leaves[name] for name in PARAM_NAMES))
    s, d, a = leaves["state"], leaves["dendrite"], leaves["adaptation"]
    for _ in range(ticks):
        j = s @ w.T
        s, d, a = advance(p, s, d, a, j, leaves["drive"], leaves["dendritic"])
    return s, d, a


def _leaves(x: TickInputs) -> dict:
    def leaf(v):
        if isinstance(v, (int, float)):
            return float(v)
        return torch.tensor(np.asarray(v, np.float64), dtype=torch.float64, requires_grad=True)

    out = {"state": leaf(x.state), "dendrite": leaf(x.dendrite), "adaptation": leaf(x.adaptation),
           "drive": leaf(x.drive), "dendritic": leaf(x.dendritic)}
    out.update({name: leaf(x.params[name]) for name in PARAM_NAMES})
    return out


def loss_value(graph: Graph, x: TickInputs, ticks: int,
               in_weight: np.ndarray | None = None) -> float:
    """The loss alone, in float64 (for finite differences)."""
    with torch.no_grad():
        leaves = {k: (v.detach() if isinstance(v, torch.Tensor) else v)
                  for k, v in _leaves(x).items()}
        s, d, a = _rollout(graph, dense_weights(graph, in_weight), leaves, ticks)
        return float((s * torch.from_numpy(x.probe["s"])).sum()
                     + (d * torch.from_numpy(x.probe["d"])).sum()
                     + (a * torch.from_numpy(x.probe["a"])).sum())


def tick_gradients(graph: Graph, x: TickInputs, ticks: int) -> dict:
    """Gradients (float64 numpy) of the probe loss after ``ticks`` ticks:
    "weight" in CSR order, "state", "dendrite", "adaptation", "drive" and
    "dendritic" (tensor drives only, in their own shapes) and one [N] array per
    parameter name."""
    w = dense_weights(graph).requires_grad_(True)
    leaves = _leaves(x)
    s, d, a = _rollout(graph, w, leaves, ticks)
    loss = ((s * torch.from_numpy(x.probe["s"])).sum() + (d * torch.from_numpy(x.probe["d"])).sum()
            + (a * torch.from_numpy(x.probe["a"])).sum())
    names = [k for k, v in leaves.items() if isinstance(v, torch.Tensor)]
    grads = torch.autograd.grad(loss, [w] + [leaves[k] for k in names], allow_unused=True)
    rows = np.repeat(np.arange(graph.n), np.diff(graph.in_rowptr))
    out = {"weight": grads[0][torch.from_numpy(rows),
                              torch.from_numpy(graph.in_col.astype(np.int64))].numpy()}
    for name, g in zip(names, grads[1:]):
        out[name] = (np.zeros(leaves[name].shape) if g is None else g.numpy())
    return out
