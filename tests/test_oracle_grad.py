"""Pins of the oracle's tick gradients (oracle/grad.py) on the CPU.

As the reference's own gradient test does (tests/test_compartmental.py:139-170),
autograd is checked against an independent numerical derivative: central
finite differences of the same float64 ticks at sampled entries of every
gradient (weights in CSR order, the three states, tensor drives, all six
parameters), over one and several ticks.  One tick's drive derivative is also
checked against its closed form.  A planted mistake (the weight gradient read
at transposed positions, as a mix-up of W and W^T would give) must fail the
finite-difference check, so the check has the power to see it.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import grad as og
from oracle import topology as otop


def inputs(graph: otop.Graph, batch: int, seed: int) -> og.TickInputs:
    rng = np.random.default_rng(seed)
    n = graph.n
    return og.TickInputs(
        state=rng.uniform(0.05, 0.95, (batch, n)), dendrite=rng.uniform(-0.9, 0.9, (batch, n)),
        adaptation=rng.uniform(0.05, 0.95, (batch, n)), drive=rng.uniform(-0.3, 0.6, (batch, n)),
        dendritic=rng.uniform(-0.3, 0.3, (batch, 1)),
        params={"alpha": rng.uniform(0.5, 0.9, n), "gain": rng.uniform(0.5, 1.2, n),
                "rho_d": rng.uniform(0.5, 0.95, n), "rho_a": rng.uniform(0.8, 0.99, n),
                "coupling": rng.uniform(0.2, 0.8, n), "strength": rng.uniform(0.05, 0.4, n)},
        probe={k: rng.standard_normal((batch, n)) for k in ("s", "d", "a")})


def perturbed(x: og.TickInputs, name: str, index: tuple, h: float) -> og.TickInputs:
    params = {k: v.copy() for k, v in x.params.items()}
    fields = {f: (np.array(getattr(x, f), copy=True) if not isinstance(getattr(x, f), float)
                  else getattr(x, f)) for f in ("state", "dendrite", "adaptation", "drive", "dendritic")}
    target = params[name] if name in params else fields[name]
    target[index] += h
    return og.TickInputs(params=params, probe=x.probe, **fields)


def numerical(graph, x, ticks, name, index, h=1e-6) -> float:
    if name == "weight":
        plus, minus = graph.in_weight.astype(np.float64), graph.in_weight.astype(np.float64)
        plus[index] += h
        minus[index] -= h
        return (og.loss_value(graph, x, ticks, plus) - og.loss_value(graph, x, ticks, minus)) / (2 * h)
    return (og.loss_value(graph, perturbed(x, name, index, h), ticks)
            - og.loss_value(graph, perturbed(x, name, index, -h), ticks)) / (2 * h)


def sample_indices(shape, rng, count=5):
    flat = rng.choice(int(np.prod(shape)), size=min(count, int(np.prod(shape))), replace=False)
    return [np.unravel_index(i, shape) for i in flat]


def check_against_fd(graph, x, ticks, grads, rng) -> float:
    worst = 0.0
    for name, value in grads.items():
        for index in sample_indices(value.shape, rng):
            want = numerical(graph, x, ticks, name, index)
            got = float(value[index])
            err = abs(got - want)
            worst = max(worst, err / (1e-7 + abs(want)))
            assert err <= 1e-6 * max(1.0, abs(want)), (name, index, got, want)
    return worst


@pytest.mark.parametrize("ticks", [1, 4])
def test_oracle_gradients_match_finite_differences(ticks):
    graph = otop.random_graph(24, 240, seed=3)
    x = inputs(graph, 2, ticks)
    grads = og.tick_gradients(graph, x, ticks)
    assert set(grads) == {"weight", "state", "dendrite", "adaptation", "drive", "dendritic",
                          *og.PARAM_NAMES}
    for value in grads.values():
        assert np.abs(value).sum() > 0
    check_against_fd(graph, x, ticks, grads, np.random.default_rng(ticks))


def test_one_tick_drive_gradient_closed_form():
    """d loss / d drive = ps * (1-alpha) * gain * (1 - tanh(u + drive)^2) where
    the clamp is inactive, with u = (1-c) j + c d' - k a (one tick, probe on s')."""
    graph = otop.random_graph(30, 300, seed=8)
    x = inputs(graph, 3, 8)
    x.probe = {"s": x.probe["s"], "d": np.zeros_like(x.probe["d"]), "a": np.zeros_like(x.probe["a"])}
    grads = og.tick_gradients(graph, x, 1)
    p = x.params
    j = x.state @ graph.dense(np.float64).T
    d_new = p["rho_d"] * x.dendrite + (1 - p["rho_d"]) * np.tanh(j + x.dendritic)
    u = (1 - p["coupling"]) * j + p["coupling"] * d_new - p["strength"] * x.adaptation
    pre = p["alpha"] * x.state + (1 - p["alpha"]) * p["gain"] * np.tanh(u + x.drive)
    slope = x.probe["s"] * (1 - p["alpha"]) * p["gain"] * (1 - np.tanh(u + x.drive) ** 2)
    expected = np.where((pre > 0) & (pre < 1), slope, 0.0)
    np.testing.assert_allclose(grads["drive"], expected, rtol=1e-12, atol=1e-14)


def test_a_transposed_weight_gradient_fails_the_check():
    graph = otop.random_graph(16, 120, seed=5)
    x = inputs(graph, 2, 9)
    grads = og.tick_gradients(graph, x, 2)
    # Planted mistake: read the dense gradient at (col, row) instead of (row, col).
    import torch

    w = og.dense_weights(graph).requires_grad_(True)
    leaves = og._leaves(x)
    s, d, a = og._rollout(graph, w, leaves, 2)
    loss = sum((v * torch.from_numpy(x.probe[k])).sum() for v, k in ((s, "s"), (d, "d"), (a, "a")))
    dense = torch.autograd.grad(loss, w)[0].numpy()
    rows = np.repeat(np.arange(graph.n), np.diff(graph.in_rowptr))
    wrong = dict(grads, weight=dense[graph.in_col, rows])
    assert not np.allclose(wrong["weight"], grads["weight"])
    with pytest.raises(AssertionError):
        check_against_fd(graph, x, 2, {"weight": wrong["weight"]}, np.random.default_rng(0))
