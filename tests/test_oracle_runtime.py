"""Pins of the oracle matrix and PELS ticks.

* FP64 dense recurrence written from the model equations (reference
  test_compartmental.py:41-71): N=12, 48 candidate edges, B=2, 20 ticks.
* PELS invariants (test_compartmental.py:126-137): |s - emitted| < theta and
  current == W @ emitted after every tick.
* Reference-held FP32 trajectory: results/compartmental_brainwaves.json
  population-mean soma traces over 4096 ticks for a continued-input row and a
  withdrawn-input row after 512 shared warm-up ticks (reference run: native
  FP32 on its own GPU; its docs report GPU-vs-CPU agreement of 1.25e-7).
"""

from __future__ import annotations

import numpy as np
import torch

import brainwaves as bw
from oracle import dynamics as od
from oracle import runtime as ort
from oracle import topology as otop


def small_case(dtype=torch.float64):
    graph = otop.random_graph(12, 48, seed=17, dtype=dtype)
    alpha = torch.full((12,), 0.7, dtype=dtype)
    gain = torch.full((12,), 0.8, dtype=dtype)
    params = od.from_time_constants(alpha, gain, dt=1.0, tau_dendrite=torch.linspace(2, 5, 12),
                                    tau_adaptation=20.0, coupling=0.6, adaptation_strength=0.3)
    return graph, params, torch.full((2, 12), 0.2, dtype=dtype)


def test_matrix_and_pels_match_dense_fp64_recurrence():
    graph, params, initial = small_case()
    expected = ort.dense_recurrence(graph, params, initial.numpy(), 20, 0.2, 0.1)
    matrix = ort.MatrixOracle(graph, params, initial)
    pels = ort.PelsOracle(graph, params, initial, theta=0.0)
    for s, d, a in expected:
        for run in (matrix, pels):
            run.step(0.2, 0.1)
            np.testing.assert_allclose(run.state.numpy(), s, rtol=1e-11, atol=1e-12)
            np.testing.assert_allclose(run.dendritic_state.numpy(), d, rtol=1e-11, atol=1e-12)
            np.testing.assert_allclose(run.adaptation_state.numpy(), a, rtol=1e-11, atol=1e-12)


def test_dense_recurrence_catches_planted_mistakes():
    # A recurrence with the coupling terms swapped must disagree: the pin is not vacuous.
    graph, params, initial = small_case()
    expected = ort.dense_recurrence(graph, params, initial.numpy(), 5, 0.2, 0.1)
    wrong = od.Params(params.alpha, params.gain, params.dendrite_decay, params.adaptation_decay,
                      1.0 - params.coupling, params.adaptation_strength)
    run = ort.MatrixOracle(graph, wrong, initial)
    for _ in range(5):
        run.step(0.2, 0.1)
    assert np.abs(run.state.numpy() - expected[-1][0]).max() > 1e-4


def test_pels_invariants_nonzero_theta():
    graph, params, initial = small_case()
    pels = ort.PelsOracle(graph, params, initial, theta=0.02)
    dense = torch.from_numpy(graph.dense(np.float64))
    for _ in range(20):
        pels.step(0.2)
        assert float((pels.state - pels.emitted_state).abs().max()) < 0.02 + 1e-12
        torch.testing.assert_close(pels.persistent_current, pels.emitted_state @ dense.T,
                                   rtol=1e-11, atol=1e-12)


def brainwaves_run(matrix_factory):
    """Run the brainwaves protocol; return (warm-up means, driven trace, zero trace)."""
    meta = bw.meta()
    ticks = meta["ticks_per_condition"]
    soma, dend = bw.neuron_inputs(bw.WARMUP + ticks)
    run = matrix_factory()
    for t in range(bw.WARMUP):
        run.step(torch.from_numpy(soma[t]), torch.from_numpy(dend[t]))
    means = {name: float(getattr(run, name)[0].mean())
             for name in ("state", "dendritic_state", "adaptation_state")}
    driven, zero = np.empty(ticks), np.empty(ticks)
    zeros = np.zeros(bw.NEURONS, np.float32)
    for t in range(ticks):
        drive = torch.from_numpy(np.stack([soma[bw.WARMUP + t], zeros]))
        ddrive = torch.from_numpy(np.stack([dend[bw.WARMUP + t], zeros]))
        state = run.step(drive, ddrive)
        trace = state.numpy().astype(np.float64)
        driven[t], zero[t] = trace[0].mean(), trace[1].mean()
    return means, driven, zero


def brainwaves_params(n=bw.NEURONS):
    return od.from_time_constants(torch.full((n,), .72), torch.full((n,), .8), dt=1.,
                                  tau_dendrite=4., tau_adaptation=25., coupling=.5,
                                  adaptation_strength=.2)


def test_brainwaves_inputs_regenerate_exactly():
    meta, gold = bw.meta(), bw.golden()
    soma, dend = bw.group_inputs(bw.WARMUP + meta["ticks_per_condition"])
    assert np.array_equal(soma[bw.WARMUP:].T, gold["somatic"])
    assert np.array_equal(dend[bw.WARMUP:].T, gold["dendritic"])


def test_brainwaves_trajectory_fp32():
    meta, gold = bw.meta(), bw.golden()
    graph = otop.random_graph(bw.NEURONS, bw.CANDIDATES, seed=meta["graph_seed"])
    assert graph.n_edges == meta["actual_edges"]
    params = brainwaves_params()
    means, driven, zero = brainwaves_run(
        lambda: ort.MatrixOracle(graph, params, torch.zeros(2, bw.NEURONS)))
    for name, value in means.items():
        assert abs(value - meta["shared_initial_state_means"][name]) < 5e-7, name
    assert np.abs(driven - gold["driven_mean"]).max() < 5e-7
    assert np.abs(zero - gold["zero_mean"]).max() < 5e-7
    assert zero[-512:].mean() == meta["mean_last_512_ticks"]["zero_input"] == 0.0


def test_block_diagonal_union_evolves_each_block_exactly_as_alone():
    """The long-horizon drift tests run several graphs (seeds, and each weight
    mode's decoded weights) as one oracle over their block-diagonal union.  Each
    block must follow its own graph's run bit for bit, at the drift tests' shape."""
    from oracle import precision as op
    n, edges, batch, ticks = 1024, 16_384, 4, 60
    base = [otop.random_graph(n, edges, seed=seed, weight_scale=0.15) for seed in (11, 23)]
    graphs = [otop.with_in_weight(g, op.quantize_dequantize(g.in_weight, mode))
              for g in base for mode in ("fp32", "fp16", "fp8", "nvfp4")]
    union = otop.block_diagonal(graphs)
    assert union.n == n * len(graphs) and union.n_edges == sum(g.n_edges for g in graphs)
    key = union.src.astype(np.int64) * union.n + union.dst
    assert (np.diff(key) > 0).all()
    assert np.array_equal(union.in_weight[union.out_weight_index], union.weight)

    def params(count):
        full = lambda value: torch.full((n * count,), value)
        return od.from_time_constants(full(0.72), full(0.8), dt=1.0, tau_dendrite=4.0,
                                      tau_adaptation=20.0, coupling=0.45,
                                      adaptation_strength=0.15)

    gen = torch.Generator().manual_seed(3)
    drives = torch.rand((ticks, batch, n), generator=gen) * 0.4
    joint = ort.MatrixOracle(union, params(len(graphs)), torch.full((batch, union.n), 0.25))
    alone = [ort.MatrixOracle(g, params(1), torch.full((batch, n), 0.25)) for g in graphs]
    for t in range(ticks):
        joint.step(drives[t].repeat(1, len(graphs)), 0.05)
        for run in alone:
            run.step(drives[t], 0.05)
    for name in ("state", "dendritic_state", "adaptation_state"):
        expected = torch.cat([getattr(run, name) for run in alone], dim=1)
        assert torch.equal(getattr(joint, name), expected), name
    # The blocks are really different runs (decoded weights change the states).
    assert not torch.equal(alone[0].state, alone[2].state)


def test_block_diagonal_catches_a_shifted_column():
    # Plant a mistake: the second block's sources not shifted.  Its rows then
    # read the first block's states, which must show.
    graphs = [otop.random_graph(40, 200, seed=s) for s in (1, 2)]
    union = otop.block_diagonal(graphs)
    wrong_col = union.in_col.copy()
    start = union.in_rowptr[40]
    wrong_col[start:] -= 40
    wrong = otop.Graph(union.n, union.src, union.dst, union.weight, union.out_rowptr,
                       union.in_rowptr, wrong_col, union.in_weight, union.out_weight_index)
    full = lambda value: torch.full((80,), value)
    p = od.from_time_constants(full(0.72), full(0.8), dt=1.0, tau_dendrite=4.0,
                               tau_adaptation=20.0)
    initial = torch.cat([torch.full((1, 40), 0.1), torch.full((1, 40), 0.6)], dim=1)
    right = ort.MatrixOracle(union, p, initial)
    bad = ort.MatrixOracle(wrong, p, initial)
    for _ in range(3):
        right.step(0.1)
        bad.step(0.1)
    assert float((right.state[:, 40:] - bad.state[:, 40:]).abs().max()) > 1e-4
