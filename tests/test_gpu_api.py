"""Runtime API behaviour of the native path (MI355X): fallbacks, validation,
checkpoint/resume on a non-default stream, the CLI, and the reference-held
brainwaves trajectory (results/compartmental_brainwaves.json) through the
native tick.
"""

from __future__ import annotations

import argparse
import io
from dataclasses import replace

import numpy as np
import pytest
import torch

import brainwaves as bw
from cases import make_case, max_err, model_to, standard_model
from neurosim_gpu import (DendriticMatrixRuntime, Dynamics, NativeDendriticMatrixRuntime,
                          NativeDendriticPELSRuntime, SparseTopology, load_native_extension,
                          load_runtime_checkpoint, random_topology, save_runtime_checkpoint,
                          topology_to)

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


def test_parameter_and_drive_gradients_use_reference(gpu):
    """Reference test_native_compartmental.py:180-204."""
    case = make_case(17, 80, 83, gpu, kind="reference")
    model = case.model
    model = replace(model, soma=Dynamics(model.soma.alpha.clone().requires_grad_(),
                                         model.soma.gain.clone().requires_grad_()),
                    dendrite_decay=model.dendrite_decay.clone().requires_grad_(),
                    adaptation_decay=model.adaptation_decay.clone().requires_grad_(),
                    coupling=model.coupling.clone().requires_grad_(),
                    adaptation_strength=model.adaptation_strength.clone().requires_grad_())
    state = torch.full((2, 17), 0.2, device=gpu)
    for kind, kwargs in ((NativeDendriticMatrixRuntime, {}),
                         (NativeDendriticPELSRuntime, {"theta": 0.0})):
        starting = state.clone().requires_grad_()
        drive = torch.full_like(state, 0.3, requires_grad=True)
        dd = torch.full_like(state, 0.2, requires_grad=True)
        native = kind(case.topology, model, starting, **kwargs)
        reference = DendriticMatrixRuntime(case.topology, model, starting)
        for _ in range(10):
            native.step(drive, dendritic_drive=dd)
            reference.step(drive, dendritic_drive=dd)
        values = [*native._parameters(), drive, dd, starting]
        actual = torch.autograd.grad(native.state.sum(), values, retain_graph=True)
        expected = torch.autograd.grad(reference.state.sum(), values)
        for a, e in zip(actual, expected):
            torch.testing.assert_close(a, e, atol=2e-5, rtol=2e-4)
            assert float(a.abs().sum()) > 0
        # The reference's native runtimes both fall back to the torch step here;
        # the matrix runtime here differentiates its own kernels instead.
        expected_backend = ("native-autograd" if kind is NativeDendriticMatrixRuntime
                            else "reference-autograd")
        assert native.last_backend == expected_backend


def test_parameters_remain_live_under_no_grad(gpu):
    """Reference test_native_compartmental.py:218-229."""
    case = make_case(97, 600, 83, gpu, kind="reference")
    model = replace(case.model, coupling=case.model.coupling.clone().requires_grad_())
    state = torch.full((3, 97), 0.2, device=gpu)
    native = NativeDendriticMatrixRuntime(case.topology, model, state.clone())
    reference = DendriticMatrixRuntime(case.topology, model, state.clone())
    with torch.no_grad():
        for _ in range(6):
            model.coupling.mul_(0.9)
            native.step(0.2)
            reference.step(0.2)
    for field in FIELDS:
        torch.testing.assert_close(getattr(native, field), getattr(reference, field),
                                   atol=2e-6, rtol=2e-4)
    assert native.last_backend == "native"


def test_checkpoint_resume_on_a_non_default_stream(gpu):
    """Reference test_native_compartmental.py:231-252."""
    case = make_case(97, 600, 83, gpu, kind="reference")
    state = torch.full((3, 97), 0.2, device=gpu)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for kind, kwargs in ((NativeDendriticMatrixRuntime, {}),
                             (NativeDendriticPELSRuntime, {"theta": 0.01})):
            native = kind(case.topology, case.model, state.clone(), **kwargs)
            for _ in range(8):
                native.step(0.2)
            buffer = io.BytesIO()
            save_runtime_checkpoint(native, buffer)
            restored = kind(case.topology, case.model, state.clone(), **kwargs)
            buffer.seek(0)
            load_runtime_checkpoint(buffer, restored)
            for _ in range(8):
                native.step(0.3)
                restored.step(0.3)
            for field in FIELDS:
                torch.testing.assert_close(getattr(native, field), getattr(restored, field),
                                           atol=2e-6, rtol=2e-4)
            if kind is NativeDendriticPELSRuntime:
                assert native._tick == restored._tick
    torch.cuda.current_stream().wait_stream(stream)


def test_matrix_checkpoint_resume_is_exact(gpu):
    case = make_case(500, 8000, 1, gpu)
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(2, 500, device=gpu))
    for _ in range(5):
        runtime.step(0.2, dendritic_drive=0.1)
    buffer = io.BytesIO()
    save_runtime_checkpoint(runtime, buffer)
    restored = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(2, 500, device=gpu))
    buffer.seek(0)
    load_runtime_checkpoint(buffer, restored)
    for _ in range(5):
        a = runtime.step(0.2, dendritic_drive=0.1)
        b = restored.step(0.2, dendritic_drive=0.1)
        assert torch.equal(a, b)


def test_invalid_inputs_fail_before_state_mutation(gpu):
    """Reference test_native_compartmental.py:254-266."""
    case = make_case(97, 600, 83, gpu, kind="reference")
    state = torch.full((3, 97), 0.2, device=gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, state.clone())
    for value in (torch.zeros(3, 3, 97, device=gpu), torch.zeros(97),
                  torch.zeros(97, device=gpu, dtype=torch.float64)):
        with pytest.raises(ValueError):
            native.step(value)
        assert torch.equal(native.state, state)
    with pytest.raises(ValueError, match="threads_per_row"):
        NativeDendriticMatrixRuntime(case.topology, case.model, state, threads_per_row=7)
    ext = load_native_extension()
    graph = case.topology
    with pytest.raises(RuntimeError, match="parameter"):
        ext.dendritic_step(state, state, state, [state], graph.in_rowptr, graph.in_col,
                           graph.in_weight, None, 0., None, 0., 32)
    with pytest.raises(RuntimeError, match="width"):
        ext.dendritic_step(state, state, state, native._parameters(), graph.in_rowptr,
                           graph.in_col, graph.in_weight, None, 0., None, 0., 7)


def test_returned_states_stay_valid_after_later_ticks(gpu):
    case = make_case(200, 2000, 5, gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(2, 200, device=gpu))
    first = native.step(0.2)
    saved = first.clone()
    for _ in range(5):
        native.step(0.2)
    assert torch.equal(first, saved)


@pytest.mark.parametrize("batch", [1, 4])
def test_runtimes_built_under_inference_mode(gpu, batch):
    """The reference's benchmark builds graph, model and runtimes inside
    torch.inference_mode (benchmarks/compartmental.py:57-70), so none of its
    tensors carry a version counter.  Every native kernel and propagation must
    run there and agree with the torch runtimes within that benchmark's own
    tolerances (rtol 2e-4, atol 2e-5 matrix; atol 2e-3 PELS at theta .02)."""
    import math
    import warnings
    from neurosim_gpu import DendriticDynamics, DendriticPELSRuntime, MatrixRollout

    n, candidates, ticks = 4096, 65_536, 40
    print(f"case inference-mode runtimes N={n} candidates={candidates} B={batch}", flush=True)
    kernels = ("rows", "panels") if batch == 1 else ("rows", "bands")
    with torch.inference_mode(), warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        graph = random_topology(n, candidates, device=gpu, seed=23)
        soma = Dynamics(torch.full((n,), .72, device=gpu), torch.full((n,), .8, device=gpu))
        model = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4.,
                                                      tau_adaptation=25.)
        initial = torch.full((batch, n), .2, device=gpu)
        matrix = {k: NativeDendriticMatrixRuntime(graph, model, initial.clone(), kernel=k)
                  for k in kernels}
        pels = {p: NativeDendriticPELSRuntime(graph, model, initial.clone(), theta=.02,
                                              propagation=p) for p in ("event", "matrix", "auto")}
        reference = DendriticMatrixRuntime(graph, model, initial.clone())
        reference_pels = DendriticPELSRuntime(graph, model, initial.clone(), theta=.02,
                                              propagation="matrix")
        for t in range(ticks):
            drive = .2 + .1 * math.sin(t * .11)
            for runtime in (*matrix.values(), *pels.values(), reference, reference_pels):
                runtime.step(drive, dendritic_drive=.1)
        rollout = MatrixRollout(matrix[kernels[-1]], 20, drive=.2, dendritic_drive=.1)
        rollout.run()
        assert bool(torch.isfinite(rollout.state).all())
    # The slot-order weight copy of panels and bands cannot see in-place edits of
    # an unversioned in_weight: the runtime says so once.
    assert any("inference_mode" in str(w.message) for w in caught)
    for name, runtime in matrix.items():
        assert runtime.kernel == name
        for f in FIELDS:
            torch.testing.assert_close(getattr(runtime, f), getattr(reference, f),
                                       rtol=2e-4, atol=2e-5)
    for name, runtime in pels.items():
        for f in FIELDS:
            torch.testing.assert_close(getattr(runtime, f), getattr(reference_pels, f),
                                       rtol=0, atol=2e-3)


def test_cli_native_matrix_and_pels(gpu, tmp_path):
    from neurosim_gpu.simulate import parser, run

    base = ["--device", "cuda", "--backend", "native", "--neurons", "300", "--edges", "4000",
            "--batch", "2", "--steps", "20"]
    for extra in ([], ["--precision", "fp8"], ["--precision", "nvfp4"], ["--precision", "fp16"],
                  ["--propagation", "pels", "--theta", "0.02"]):
        args = parser().parse_args(base + extra)
        result = run(args)
        assert result["runtime"].startswith("Native")
        assert result["backend"].startswith("native")
    checkpoint = tmp_path / "c.pt"
    run(parser().parse_args(base + ["--checkpoint", str(checkpoint)]))
    resumed = run(parser().parse_args(base + ["--resume", str(checkpoint)]))
    continuous = run(parser().parse_args(base[:-1] + ["40"]))
    assert resumed["resumed"]
    for name in FIELDS:
        assert resumed["states"][name]["mean"] == pytest.approx(
            continuous["states"][name]["mean"], abs=1e-6)


def test_brainwaves_reference_trajectory_native(gpu):
    """Native tick against the reference-held 4096-tick population-mean traces."""
    print("case brainwaves N=1024 B=2 ticks=4608", flush=True)
    meta, gold = bw.meta(), bw.golden()
    topology = random_topology(bw.NEURONS, bw.CANDIDATES, device="cpu", seed=meta["graph_seed"])
    assert topology.n_edges == meta["actual_edges"]
    model, _ = standard_model(bw.NEURONS)
    runtime = NativeDendriticMatrixRuntime(topology_to(topology, gpu), model_to(model, gpu),
                                           torch.zeros(2, bw.NEURONS, device=gpu))
    ticks = meta["ticks_per_condition"]
    soma, dend = bw.neuron_inputs(bw.WARMUP + ticks)
    soma_t = torch.from_numpy(soma).to(gpu)
    dend_t = torch.from_numpy(dend).to(gpu)
    with torch.inference_mode():
        for t in range(bw.WARMUP):
            runtime.step(soma_t[t], dendritic_drive=dend_t[t])
        for name in FIELDS:
            value = float(getattr(runtime, name)[0].mean())
            assert abs(value - meta["shared_initial_state_means"][name]) < 5e-7
        zeros = torch.zeros(bw.NEURONS, device=gpu)
        trace = torch.empty(ticks, 2, device=gpu)
        for t in range(ticks):
            drive = torch.stack([soma_t[bw.WARMUP + t], zeros])
            ddrive = torch.stack([dend_t[bw.WARMUP + t], zeros])
            trace[t] = runtime.step(drive, dendritic_drive=ddrive).double().mean(dim=1).float()
    state_trace = trace.double().cpu().numpy()
    assert np.abs(state_trace[:, 0] - gold["driven_mean"]).max() < 5e-7
    assert np.abs(state_trace[:, 1] - gold["zero_mean"]).max() < 5e-7
