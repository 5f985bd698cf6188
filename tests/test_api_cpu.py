"""The package's PyTorch runtimes, checkpoint and CLI on the CPU.

Mirrors the reference's CPU tests for the dendritic mainline
(test_compartmental.py, test_simulate.py, test_topology_io.py) and checks the
product's reference-backend runtimes against the oracle bitwise (both run the
same torch CPU ops in the same order).
"""

from __future__ import annotations

import io
import math
from dataclasses import replace

import numpy as np
import pytest
import torch

from oracle import dynamics as od
from oracle import runtime as ort
from oracle import topology as otop
from neurosim_gpu import (DendriticDynamics, DendriticMatrixRuntime, DendriticPELSRuntime,
                          Dynamics, MatrixRuntime, SparseTopology, capture_runtime,
                          load_runtime_checkpoint, load_topology, random_topology,
                          restore_runtime, save_runtime_checkpoint, save_topology)


def make(dtype=torch.float64):
    graph = random_topology(12, 48, device="cpu", dtype=dtype, seed=17)
    soma = Dynamics(torch.full((12,), 0.7, dtype=dtype), torch.full((12,), 0.8, dtype=dtype))
    dynamics = DendriticDynamics.from_time_constants(soma, dt=1.0,
                                                     tau_dendrite=torch.linspace(2, 5, 12),
                                                     tau_adaptation=20.0, coupling=0.6,
                                                     adaptation_strength=0.3)
    return graph, dynamics, torch.full((2, 12), 0.2, dtype=dtype)


def test_matrix_and_pels_paths_match_dense_recurrence():
    graph, dynamics, initial = make()
    matrix = DendriticMatrixRuntime(graph, dynamics, initial.clone())
    paths = [DendriticPELSRuntime(graph, dynamics, initial.clone(), theta=0, propagation=mode)
             for mode in ("matrix", "event", "auto")]
    weight = graph.dense_matrix()
    state, dendrite, adaptation = initial.clone(), torch.zeros_like(initial), torch.zeros_like(initial)
    for _ in range(20):
        current = state @ weight.T
        dendrite = (dynamics.dendrite_decay * dendrite
                    + (1 - dynamics.dendrite_decay) * torch.tanh(current + 0.1))
        combined = 0.4 * current + 0.6 * dendrite - 0.3 * adaptation
        state = (0.7 * state + 0.3 * 0.8 * torch.tanh(combined + 0.2)).clamp(0, 1)
        adaptation = dynamics.adaptation_decay * adaptation + (1 - dynamics.adaptation_decay) * state
        torch.testing.assert_close(matrix.step(0.2, dendritic_drive=0.1), state, rtol=1e-11, atol=1e-12)
        for path in paths:
            torch.testing.assert_close(path.step(0.2, dendritic_drive=0.1), state,
                                       rtol=1e-11, atol=1e-12)
            torch.testing.assert_close(path.dendritic_state, dendrite)
            torch.testing.assert_close(path.adaptation_state, adaptation)


def test_reference_backend_equals_oracle_bitwise_fp32():
    n, m = 300, 6000
    graph = otop.random_graph(n, m, seed=9)
    topology = random_topology(n, m, device="cpu", seed=9)
    soma = Dynamics(torch.full((n,), .72), torch.full((n,), .8))
    model = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4., tau_adaptation=25.)
    params = od.from_time_constants(torch.full((n,), .72), torch.full((n,), .8), dt=1.,
                                    tau_dendrite=4., tau_adaptation=25.)
    runtime = DendriticMatrixRuntime(topology, model, torch.zeros(3, n))
    pels = DendriticPELSRuntime(topology, model, torch.zeros(3, n), theta=0.01, propagation="matrix")
    oracle = ort.MatrixOracle(graph, params, torch.zeros(3, n))
    oracle_pels = ort.PelsOracle(graph, params, torch.zeros(3, n), theta=0.01)
    drive = torch.tensor([[0.1], [0.2], [0.3]])
    for _ in range(30):
        runtime.step(drive, dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        pels.step(drive, dendritic_drive=0.1)
        oracle_pels.step(drive, 0.1)
    for name in ("state", "dendritic_state", "adaptation_state"):
        assert torch.equal(getattr(runtime, name), getattr(oracle, name))
        assert torch.equal(getattr(pels, name), getattr(oracle_pels, name))
    assert torch.equal(pels.persistent_current, oracle_pels.persistent_current)


def test_neutral_parameters_recover_point_model():
    graph, dynamics, initial = make()
    zero = torch.zeros(12, dtype=torch.float64)
    dynamics = replace(dynamics, coupling=zero, adaptation_strength=zero)
    baseline = MatrixRuntime(graph, dynamics.soma, initial.clone())
    extended = DendriticMatrixRuntime(graph, dynamics, initial.clone())
    for t in range(30):
        drive = 0.15 + 0.05 * math.sin(t)
        assert torch.equal(extended.step(drive), baseline.step(drive))


def test_pels_residual_bound_and_weight_refresh():
    graph, dynamics, initial = make()
    runtime = DendriticPELSRuntime(graph, dynamics, initial, theta=0.02, propagation="event")
    for t in range(20):
        if t == 5:
            graph.apply_source_weights_(graph.weight * 0.7)
        runtime.step(0.2)
        assert float((runtime.state - runtime.emitted_state).abs().max()) < 0.02 + 1e-12
        torch.testing.assert_close(runtime.persistent_current,
                                   runtime.emitted_state @ graph.dense_matrix().T,
                                   rtol=1e-11, atol=1e-12)


def test_idle_pels_updates_local_states():
    graph, dynamics, initial = make()
    runtime = DendriticPELSRuntime(graph, dynamics, initial, theta=2, propagation="event")
    state, stats = runtime.step(0.5, dendritic_drive=0.5, collect_stats=True)
    assert stats.path == "idle" and stats.active_edges == 0
    assert float(runtime.adaptation_state.sum()) > 0
    assert not torch.equal(state, initial)


def test_gradients_match_dense_recurrence():
    graph, dynamics, initial = make()
    weights = graph.weight.detach().clone().requires_grad_()
    graph = SparseTopology.from_edges(12, graph.src, graph.dst, weights)
    drive = torch.full_like(initial, 0.3, requires_grad=True)
    matrix = DendriticMatrixRuntime(graph, dynamics, initial.clone())
    pels = DendriticPELSRuntime(graph, dynamics, initial.clone(), theta=0, propagation="event")
    state, dendrite, adaptation = initial.clone(), torch.zeros_like(initial), torch.zeros_like(initial)
    for _ in range(8):
        matrix.step(drive, dendritic_drive=0.2)
        pels.step(drive, dendritic_drive=0.2)
        state, dendrite, adaptation = dynamics.advance(state, dendrite, adaptation,
                                                       state @ graph.dense_matrix().T, drive,
                                                       dendritic_drive=0.2)
    expected = torch.autograd.grad(state.square().sum(), (weights, drive), retain_graph=True)
    for output in (matrix.state, pels.state):
        actual = torch.autograd.grad(output.square().sum(), (weights, drive), retain_graph=True)
        for a, e in zip(actual, expected):
            torch.testing.assert_close(a, e, rtol=1e-9, atol=1e-11)


def test_checkpoint_restores_all_states_exactly():
    graph, dynamics, initial = make()
    for kind, kwargs in ((DendriticMatrixRuntime, {}),
                         (DendriticPELSRuntime, {"theta": 0.01, "propagation": "event"})):
        runtime = kind(graph, dynamics, initial.clone(), **kwargs)
        for _ in range(10):
            runtime.step(0.2, dendritic_drive=0.4)
        buffer = io.BytesIO()
        save_runtime_checkpoint(runtime, buffer)
        restored = kind(graph, dynamics, initial.clone(), **kwargs)
        buffer.seek(0)
        load_runtime_checkpoint(buffer, restored)
        for _ in range(10):
            assert torch.equal(runtime.step(0.3), restored.step(0.3))
            assert torch.equal(runtime.dendritic_state, restored.dendritic_state)
            assert torch.equal(runtime.adaptation_state, restored.adaptation_state)


def test_incomplete_or_incompatible_checkpoint_rejected_before_mutation():
    graph, dynamics, initial = make()
    runtime = DendriticMatrixRuntime(graph, dynamics, initial.clone())
    runtime.step(0.3)
    payload = capture_runtime(runtime)
    with pytest.raises(ValueError, match="runtime type"):
        restore_runtime(DendriticPELSRuntime(graph, dynamics, initial.clone(), theta=0), payload)
    for field in ("dendrite_decay", "adaptation_decay", "coupling", "adaptation_strength"):
        other = replace(dynamics, **{field: getattr(dynamics, field) * 0.9})
        with pytest.raises(ValueError, match="parameters"):
            restore_runtime(DendriticMatrixRuntime(graph, other, initial.clone()), payload)
    del payload["tensors"]["adaptation_state"]
    before = runtime.state.clone()
    with pytest.raises(ValueError, match="missing tensor adaptation_state"):
        restore_runtime(runtime, payload)
    assert torch.equal(runtime.state, before)


def test_invalid_parameters_and_drives_rejected():
    graph, dynamics, initial = make()
    for field, value in (("dendrite_decay", 1.0), ("adaptation_decay", -0.1), ("coupling", 1.1),
                         ("adaptation_strength", -0.1), ("coupling", float("nan"))):
        with pytest.raises(ValueError):
            replace(dynamics, **{field: torch.full((12,), value, dtype=torch.float64)})
    with pytest.raises(ValueError, match="dtype"):
        replace(dynamics, coupling=dynamics.coupling.float())
    for tau in (0, -1, float("nan"), float("inf")):
        with pytest.raises(ValueError, match="finite and positive"):
            DendriticDynamics.from_time_constants(dynamics.soma, dt=1, tau_dendrite=tau,
                                                  tau_adaptation=10)
    with pytest.raises(ValueError, match="shape"):
        DendriticMatrixRuntime(graph, dynamics, initial[0])
    with pytest.raises(ValueError, match="finite"):
        DendriticMatrixRuntime(graph, dynamics, initial * float("nan"))
    runtime = DendriticMatrixRuntime(graph, dynamics, initial)
    with pytest.raises(ValueError, match="broadcast"):
        runtime.step(dendritic_drive=torch.ones(3, 2, 12))
    assert torch.equal(runtime.dendritic_state, torch.zeros_like(initial))


def test_theta_validation():
    graph, dynamics, initial = make()
    with pytest.raises(ValueError, match="non-negative"):
        DendriticPELSRuntime(graph, dynamics, initial, theta=-0.1)
    theta = torch.zeros(12, dtype=torch.float64)
    theta[int(torch.argmax(graph.out_degree))] = float("inf")
    with pytest.raises(ValueError, match="zero-outdegree"):
        DendriticPELSRuntime(graph, dynamics, initial, theta=theta)


def test_topology_round_trip(tmp_path):
    graph = random_topology(50, 400, device="cpu", seed=4)
    path = tmp_path / "g.pt"
    save_topology(graph, path, include_destination_weights=True)
    loaded = load_topology(path)
    for name in ("src", "dst", "weight", "out_rowptr", "in_rowptr", "in_col",
                 "out_weight_index", "in_weight"):
        assert torch.equal(getattr(loaded, name), getattr(graph, name)), name


def test_cli_reference_paths(tmp_path):
    from neurosim_gpu.simulate import build_runtime, parser, run

    def args(*extra):
        return parser().parse_args(["--neurons", "12", "--edges", "48", "--batch", "2",
                                    "--steps", "5", *extra])

    runtime = build_runtime(args())
    assert type(runtime).__name__ == "DendriticMatrixRuntime"
    result = run(args())
    assert result["backend"] == "reference" and not result["approximate"]
    matrix, pels = build_runtime(args()), build_runtime(args("--propagation", "pels"))
    for _ in range(30):
        matrix.step(0.2, dendritic_drive=0.1)
        pels.step(0.2, dendritic_drive=0.1)
    for name in ("state", "dendritic_state", "adaptation_state"):
        torch.testing.assert_close(getattr(matrix, name), getattr(pels, name), atol=2e-6, rtol=2e-4)
    checkpoint, summary = tmp_path / "s.pt", tmp_path / "s.json"
    for path in ("matrix", "pels"):
        extra = ["--propagation", path] + (["--theta", "0.02"] if path == "pels" else [])
        run(args(*extra, "--checkpoint", str(checkpoint)))
        result = run(args(*extra, "--resume", str(checkpoint), "--checkpoint", str(checkpoint),
                          "--output", str(summary)))
        assert result["resumed"] and result["approximate"] == (path == "pels")
        resumed, continuous = build_runtime(args(*extra)), build_runtime(args(*extra))
        load_runtime_checkpoint(checkpoint, resumed)
        for _ in range(10):
            continuous.step(0.2, dendritic_drive=0.1)
        expected = capture_runtime(continuous)["tensors"]
        for name, value in capture_runtime(resumed)["tensors"].items():
            assert torch.equal(value, expected[name]), name
    for extra in (("--backend", "native"), ("--theta", "0.1"), ("--theta", "nan"),
                  ("--drive", "inf"), ("--neurons", "0"), ("--edges", "-1"), ("--steps", "0"),
                  ("--batch", "0"), ("--tau-dendrite", "0"), ("--coupling", "2"),
                  ("--propagation", "pels", "--theta", "-1"), ("--precision", "fp16")):
        with pytest.raises(ValueError):
            build_runtime(args(*extra))


def test_cpu_quantized_simulation_reports_execution():
    from neurosim_gpu.simulate import parser, run

    for name in ("fp8", "nvfp4"):
        result = run(parser().parse_args(["--neurons", "12", "--edges", "48", "--batch", "2",
                                          "--steps", "5", "--precision", name,
                                          "--propagation", "pels"]))
        assert result["precision"] == name and "qdq-emulation" in result["precision_execution"]


def test_native_runtime_requires_a_gpu_tensor():
    graph, dynamics, initial = make(torch.float32)
    from neurosim_gpu import NativeDendriticMatrixRuntime

    with pytest.raises(ValueError, match="requires CUDA float32"):
        NativeDendriticMatrixRuntime(graph, dynamics, initial)


def test_event_scatter_equals_matrix_product_of_the_deltas():
    from neurosim_gpu.runtime import scatter_out_edges

    graph = random_topology(200, 3000, device="cpu", seed=3, dtype=torch.float64)
    rng = torch.Generator().manual_seed(5)
    delta = torch.randn(3, 200, generator=rng, dtype=torch.float64)
    active = torch.rand(3, 200, generator=rng) < 0.1
    delta = torch.where(active, delta, torch.zeros_like(delta))
    expected = delta @ graph.dense_matrix().T
    torch.testing.assert_close(scatter_out_edges(graph, delta, active), expected,
                               rtol=1e-12, atol=1e-12)
    none = torch.zeros_like(active)
    assert torch.equal(scatter_out_edges(graph, delta, none), torch.zeros_like(delta))


def test_auto_policy_samples_every_interval_and_picks_by_edge_fraction():
    from neurosim_gpu.runtime import _PathPolicy

    graph = random_topology(100, 1000, device="cpu", seed=1)
    policy = _PathPolicy("auto", 0.12, 4)
    few = torch.zeros(1, 100, dtype=torch.bool)
    few[0, int(torch.argmax(graph.out_degree))] = True
    many = torch.ones(1, 100, dtype=torch.bool)
    assert policy.choose(0, many, graph, False) == ("matrix", graph.n_edges)
    assert policy.choose(1, few, graph, False) == ("matrix", -1)      # held until tick 4
    path, edges = policy.choose(4, few, graph, False)
    assert path == "event" and edges == int(graph.out_degree.max())
    assert policy.choose(5, many, graph, True) == ("event", graph.n_edges)   # stats: counted, held
    assert policy.choose(8, torch.zeros_like(few), graph, False) == ("idle", 0)
    fixed = _PathPolicy("matrix", 0.12, 4)
    assert fixed.choose(3, many, graph, False) == ("matrix", -1)
    assert fixed.choose(3, many, graph, True) == ("matrix", graph.n_edges)


def test_row_plans_of_an_inference_mode_rowptr():
    """The reference's benchmark builds its graphs under torch.inference_mode, whose
    tensors carry no version counter: the row-plan cache keys them by identity."""
    from neurosim_gpu.native import load_native_extension

    extension = load_native_extension()
    with torch.inference_mode():
        graph = random_topology(40, 400, device="cpu", seed=3)
        assert torch.is_inference(graph.in_rowptr)
        first = extension.plan_tensors(graph.in_rowptr, 1)
    assert extension.plan_tensors(graph.in_rowptr, 1) is first
    bounds, blocks, capacity = first
    assert blocks >= 1 and capacity > 0 and bounds.numel() == 2 * (blocks + 1)
    # A versioned rowptr edited in place gets a new plan.
    rowptr = graph.in_rowptr.clone()
    before = extension.plan_tensors(rowptr, 1)
    rowptr.add_(0)
    assert extension.plan_tensors(rowptr, 1) is not before


@pytest.mark.parametrize("edges,published", [
    (16_273, {"fp32": 65_092, "fp16": 32_546, "fp8": 16_277, "nvfp4": 9_159}),
    (999_787, {"fp32": 3_999_148, "fp16": 1_999_574, "fp8": 999_791, "nvfp4": 562_385})])
def test_weight_storage_bytes_equal_the_published_payloads(edges, published):
    """results/precision_native.json:362,417,472,527 (and the small workload's rows)
    give each mode's logical payload for the reference's two graphs; the property
    reads only the edge count and the mode, so it is checked without a GPU."""
    from types import SimpleNamespace
    from neurosim_gpu import NativeDendriticMatrixRuntime

    modes = {"fp32": (torch.float32, None), "fp16": (torch.float16, None),
             "fp8": (torch.float32, "fp8"), "nvfp4": (torch.float32, "nvfp4")}
    for mode, (dtype, fmt) in modes.items():
        runtime = SimpleNamespace(topology=SimpleNamespace(n_edges=edges),
                                  weight_dtype=dtype, weight_format=fmt)
        assert NativeDendriticMatrixRuntime.weight_storage_bytes.fget(runtime) == published[mode]
