"""Native PELS event tick vs the CPU oracle (MI355X).

Tolerances: theta=0 within 1e-5 of the oracle (which is then the matrix
tick); theta>0 within 1e-3 of the oracle PELS at the same theta (float32
atomics reorder the current's sums, which can move an emission by a tick near
the threshold; the reference accepts 2e-3 for the same comparison).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import make_case, max_err
from oracle import runtime as ort
from neurosim_gpu import NativeDendriticPELSRuntime
from neurosim_gpu import native as native_mod

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


def state_error(native, oracle) -> float:
    return max(max_err(getattr(native, f), getattr(oracle, f)) for f in FIELDS)


# one launch (scatter into pending buffers), two launches (advance, scatter),
# or matrix propagation (advance only, then current += W @ delta)
MODES = {"one_launch": dict(one_launch=True), "two_launch": dict(one_launch=False),
         "matrix": dict(propagation="matrix"),
         "matrix_two_launch": dict(propagation="matrix", one_launch=False),
         "auto": dict(propagation="auto", policy_interval=2),
         # the matrix propagation's product on the column-panel kernel (batch 1 or 2)
         "matrix_panels": dict(propagation="matrix", kernel="panels"),
         "auto_panels": dict(propagation="auto", policy_interval=2, kernel="panels")}


@pytest.mark.parametrize("mode", list(MODES))
def test_theta_zero_long_rollout_matches_matrix(gpu, mode):
    """Reference test_native_compartmental.py:99-110 (N=1024, B=2, 16000 edges, 500 ticks)."""
    case = make_case(1024, 16000, 83, gpu, kind="reference")
    state = torch.full((2, 1024), 0.2)
    native = NativeDendriticPELSRuntime(case.topology, case.model, state.to(gpu), theta=0,
                                        **MODES[mode])
    matrix = ort.MatrixOracle(case.graph, case.params, state)
    for t in range(500):
        value = 0.2 if t % 70 < 35 else 0.05
        native.step(value, dendritic_drive=0.1)
        matrix.step(value, 0.1)
    assert state_error(native, matrix) <= 8e-6
    current = ort.propagate(ort.csr_matrix(case.graph), native.emitted_state.cpu())
    assert max_err(native.persistent_current, current) <= 1e-5


@pytest.mark.parametrize("mode", list(MODES))
def test_nonzero_theta_emission_and_weight_mutation(gpu, mode):
    """Reference test_native_compartmental.py:142-164 (theta .02, weights x0.7 at tick 25)."""
    from oracle import topology as otop

    case = make_case(97, 600, 83, gpu, kind="reference")
    batch = 2 if MODES[mode].get("kernel") == "panels" else 3
    state = torch.full((batch, 97), 0.2)
    native = NativeDendriticPELSRuntime(case.topology, case.model, state.to(gpu), theta=0.02,
                                        **MODES[mode])
    assert native.kernel == MODES[mode].get("kernel", "rows")
    oracle = ort.PelsOracle(case.graph, case.params, state, theta=0.02)
    for t in range(50):
        if t == 25:
            case.topology.apply_source_weights_(case.topology.weight * 0.7)
            new_graph = otop.with_weights(case.graph, case.topology.weight.cpu().numpy())
            oracle.matrix = ort.csr_matrix(new_graph)
            oracle.persistent_current = ort.propagate(oracle.matrix, oracle.emitted_state)
            case = case.__class__(new_graph, case.topology, case.model, case.params)
        native.step(0.3, dendritic_drive=0.1)
        oracle.step(0.3, 0.1)
        assert float((native.state - native.emitted_state).abs().max()) < 0.020001
        exact = ort.propagate(ort.csr_matrix(case.graph), native.emitted_state.cpu())
        assert max_err(native.persistent_current, exact) <= 1e-5
    assert state_error(native, oracle) <= 1e-3
    _, stats = native.step(0.3, collect_stats=True)
    oracle.step(0.3)
    assert native.last_backend == "reference-stats" and stats.active_edges >= 0
    path = native.selected_path
    native.step(0.3)
    oracle.step(0.3)
    expected = "native-matrix" if MODES[mode].get("propagation") == "matrix" else "native"
    if mode == "auto":
        expected = "native-matrix" if path == "matrix" else "native"
    assert native.last_backend == expected
    assert state_error(native, oracle) <= 1e-3


def test_idle_updates_traces_and_retains_returned_state(gpu):
    """Reference test_native_compartmental.py:166-178 (theta 2: nothing emits)."""
    case = make_case(97, 600, 83, gpu, kind="reference")
    native = NativeDendriticPELSRuntime(case.topology, case.model,
                                        torch.full((3, 97), 0.2, device=gpu), theta=2)
    previous = native.step(0.5)
    saved = previous.clone()
    current = native.persistent_current.clone()
    first_adaptation = native.adaptation_state.clone()
    for _ in range(10):
        native.step(0.5)
    assert torch.equal(previous, saved)
    assert torch.equal(native.persistent_current, current)
    assert not torch.equal(first_adaptation, native.adaptation_state)


@pytest.mark.parametrize("propagation,kernel", [("event", "auto"), ("matrix", "auto"),
                                                ("auto", "auto"), ("matrix", "panels"),
                                                ("auto", "panels")])
@pytest.mark.parametrize("theta", [0.0, 0.02])
def test_cfg4_event_path_warmup_then_withdrawn(gpu, theta, propagation, kernel):
    """N=50000, M~1M, B=1: 512 ticks drive .2/.1, then 4096 ticks with inputs withdrawn."""
    print(f"case cfg4 N=50000 M=1000000 theta={theta} propagation={propagation} "
          f"kernel={kernel}", flush=True)
    case = make_case(50_000, 1_000_000, 0, gpu)
    native = NativeDendriticPELSRuntime(case.topology, case.model,
                                        torch.zeros(1, 50_000, device=gpu), theta=theta,
                                        propagation=propagation, kernel=kernel)
    oracle = ort.PelsOracle(case.graph, case.params, torch.zeros(1, 50_000), theta=theta)
    bar = 1e-5 if theta == 0 else 1e-3
    worst = worst_current = 0.0
    mismatches = checked = 0
    paths = {"event": 0, "matrix": 0}
    for tick in range(512 + 4096):
        drive, ddrive = (0.2, 0.1) if tick < 512 else (0.0, 0.0)
        before_native, before_oracle = native.emitted_state, oracle.emitted_state
        paths[native.selected_path] += 1
        native.step(drive, dendritic_drive=ddrive)
        oracle.step(drive, ddrive)
        if tick % 64 == 63 or tick == 511:
            worst = max(worst, state_error(native, oracle))
            worst_current = max(worst_current,
                                max_err(native.persistent_current, oracle.persistent_current))
            if theta > 0:
                # emission mask: active <=> |s' - emitted| >= theta > 0 <=> emitted changed
                emitted_native = (native.emitted_state != before_native).cpu()
                mismatches += int((emitted_native != oracle.last_active).sum())
                checked += emitted_native.numel()
            else:
                # theta = 0: every pair is active, so emitted tracks the state itself
                assert max_err(native.emitted_state, native.state) <= 1e-6
    print(f"cfg4 theta={theta} {propagation} ({native.kernel} product): state {worst:.3e} "
          f"current {worst_current:.3e} "
          f"emit-mask mismatches {mismatches}/{checked}; ticks by path {paths}")
    if propagation == "auto":
        # theta = 0: every pair is active (|0| >= 0), so after the first sample every
        # tick multiplies; theta = .02: only the onset from the zero state is that
        # active, and the withdrawn phase scatters.
        if theta == 0:
            assert paths["matrix"] >= 512 + 4096 - 4 * native.policy_interval
        else:
            assert paths["event"] >= 4096
    assert worst <= bar
    assert worst_current <= bar
    assert max_err(native.emitted_state, oracle.emitted_state) <= bar
    assert mismatches <= 1e-3 * max(checked, 1)


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_one_launch_pending_reads_and_assignments(gpu, batch):
    """Reads of the persistent current fold the outstanding pending buffer; an
    assignment replaces the current and discards it.  Either way the run goes on
    matching the oracle and the two-launch tick (which gathers its weights
    through out_weight_index instead of streaming the source-major copy, and
    here scatters into an assigned row-major current as well)."""
    case = make_case(2000, 40_000, 7, gpu)
    matrix = ort.csr_matrix(case.graph)
    state = torch.full((batch, 2000), 0.1)
    native = NativeDendriticPELSRuntime(case.topology, case.model, state.to(gpu), theta=0.01)
    two = NativeDendriticPELSRuntime(case.topology, case.model, state.to(gpu), theta=0.01,
                                     one_launch=False)
    two.source_major_weights.enabled = False    # the scatter gathers through out_weight_index
    oracle = ort.PelsOracle(case.graph, case.params, state, theta=0.01)
    for tick in range(60):
        drive = 0.3 if tick < 40 else 0.0
        for runtime in (native, two):
            runtime.step(drive, dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        exact = ort.propagate(matrix, native.emitted_state.cpu())
        if tick % 7 == 3:
            assert max_err(native.persistent_current, exact) <= 1e-5
        if tick % 11 == 5:
            # the exact current, assigned while a scatter is outstanding
            native.persistent_current = exact.to(gpu)
            # a row-major current for the two-launch tick to scatter into
            two.persistent_current = ort.propagate(matrix, two.emitted_state.cpu()).to(gpu)
        if tick % 11 == 6:
            assert max_err(native.persistent_current, exact) <= 1e-5
    assert state_error(native, oracle) <= 1e-3
    assert state_error(native, two) <= 1e-3
    assert max_err(native.persistent_current, oracle.persistent_current) <= 1e-3


def test_one_launch_graph_replay_matches_eager(gpu):
    """Ticks captured in a HIP graph (an odd count, so the pending buffers swap
    roles between replays) against eager ticks, theta 0."""
    case = make_case(3000, 60_000, 8, gpu)
    state = torch.full((2, 3000), 0.1, device=gpu)
    eager = NativeDendriticPELSRuntime(case.topology, case.model, state.clone(), theta=0.0)
    rolled = NativeDendriticPELSRuntime(case.topology, case.model, state.clone(), theta=0.0)
    for runtime in (eager, rolled):
        for _ in range(3):
            runtime.step(0.2, dendritic_drive=0.1)
    fields = ("state", "dendritic_state", "adaptation_state", "emitted_state")
    start = [getattr(rolled, f) for f in fields]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(5):
            rolled.step(0.2, dendritic_drive=0.1)
    end = [getattr(rolled, f) for f in fields]
    for replay in range(3):
        if replay:
            # the next replay starts from this replay's end; the graph's pending
            # buffers swap roles, which the captured ticks cannot do, so the
            # outstanding buffer is folded into the current first
            for first, last in zip(start, end):
                first.copy_(last)
            rolled.persistent_current
            assert not rolled._pending.any()
        graph.replay()
        for _ in range(5):
            eager.step(0.2, dendritic_drive=0.1)
        torch.cuda.synchronize()
        for name, value in zip(fields, end):
            assert max_err(value, getattr(eager, name)) <= 1e-5, (replay, name)
        assert max_err(rolled.persistent_current, eager.persistent_current) <= 1e-5, replay


@pytest.mark.parametrize("batch", [2, 3, 4, 8, 64])
@pytest.mark.parametrize("one_launch", [True, False])
@pytest.mark.parametrize("theta", [0.0, 0.01])
def test_hub_sources_scatter_many_rounds(gpu, one_launch, theta, batch):
    """Sources with thousands of out-edges next to ordinary ones: one
    wavefront's emitters then span dozens of 64-edge rounds, and an edge's
    emitter is found among neighbours of very different degree.  At B = 2, 4, 8
    and 64 the scatter takes each source's emitting columns together (B=3 walks
    pair by pair); the columns get different drives and initial states, so a
    source emits in some columns and not in others."""
    from oracle import topology as otop
    from neurosim_gpu import SparseTopology, topology_to
    from cases import model_to, standard_model

    print(f"case pels hubs theta={theta} one_launch={one_launch} B={batch}", flush=True)
    n = 3000
    rng = np.random.default_rng(21)
    hubs = [(5, 2900), (6, 1500), (64, 2999), (2999, 2000)]
    src = [rng.integers(0, n, 20 * n)]
    dst = [rng.integers(0, n, 20 * n)]
    for source, degree in hubs:
        src.append(np.full(degree, source))
        dst.append(rng.permutation(n)[:degree])
    src, dst = np.concatenate(src), np.concatenate(dst)
    weight = (rng.standard_normal(src.size) * 0.02).astype(np.float32)
    graph = otop.build(n, src, dst, weight)
    topology = topology_to(SparseTopology.from_edges(n, torch.from_numpy(src), torch.from_numpy(dst),
                                                     torch.from_numpy(weight)), gpu)
    model, params = standard_model(n)
    columns = torch.linspace(0.0, 1.0, batch)[:, None]
    state = 0.1 + 0.05 * columns.expand(batch, n).contiguous()
    native = NativeDendriticPELSRuntime(topology, model_to(model, gpu), state.to(gpu), theta=theta,
                                        one_launch=one_launch)
    oracle = ort.PelsOracle(graph, params, state, theta=theta)
    matrix = ort.csr_matrix(graph)
    for tick in range(40):
        drive = (0.3 if tick < 25 else 0.05) * (0.5 + columns)
        native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
    exact = ort.propagate(matrix, native.emitted_state.cpu())
    bar = 1e-5 if theta == 0 else 1e-3
    assert max_err(native.persistent_current, exact) <= 1e-5
    assert state_error(native, oracle) <= bar


def test_propagation_modes_are_checked(gpu):
    case = make_case(97, 600, 83, gpu, kind="reference")
    with pytest.raises(ValueError, match="'event', 'matrix' or 'auto'"):
        NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(1, 97, device=gpu),
                                   theta=0.0, propagation="dense")
    with pytest.raises(ValueError, match="one-launch"):
        NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(1, 97, device=gpu),
                                   theta=0.0, propagation="auto", one_launch=False)
    with pytest.raises(ValueError, match="event_edge_fraction"):
        NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(1, 97, device=gpu),
                                   theta=0.0, propagation="auto", event_edge_fraction=1.5)
    with pytest.raises(ValueError, match="'auto', 'rows' or 'panels'"):
        NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(1, 97, device=gpu),
                                   theta=0.0, propagation="matrix", kernel="bands")
    with pytest.raises(ValueError, match="batch 1 or 2"):
        NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(3, 97, device=gpu),
                                   theta=0.0, propagation="matrix", kernel="panels")
    scatter = NativeDendriticPELSRuntime(case.topology, case.model,
                                         torch.zeros(1, 97, device=gpu), theta=0.0,
                                         kernel="panels")
    assert scatter.kernel == "rows"      # the event path multiplies nothing: no layout


@pytest.mark.parametrize("batch,theta", [(1, 0.0), (1, 0.02), (3, 0.01), (2, 2.0)])
def test_activity_counters_count_the_active_out_edges(gpu, batch, theta):
    """The tick's activity counters sum to the out-degrees of the pairs with
    |s' - emitted| >= theta: the reference policy's active_edges (runtime.py:150-155),
    in the scattering and in the fused advance-only launch."""
    case = make_case(3000, 60_000, 8, gpu)
    native = NativeDendriticPELSRuntime(case.topology, case.model,
                                        torch.zeros(batch, 3000, device=gpu), theta=theta)
    for _ in range(5):
        native.step(0.3, dendritic_drive=0.1)
    degree = (case.topology.out_rowptr[1:] - case.topology.out_rowptr[:-1]).long()
    ext, t = native.extension, case.topology
    for advance_only in (False, True):
        emitted = native.emitted_state.clone()
        current = native.persistent_current.contiguous().clone()
        before = current.clone()
        folded = torch.rand(batch * 3000, generator=torch.Generator().manual_seed(batch)) * 1e-3
        pending = (folded.to(gpu),
                   None if advance_only else torch.zeros(batch * 3000, device=gpu))
        counters = torch.zeros(native_mod.EVENT_ACTIVITY_SLOTS * native_mod.EVENT_ACTIVITY_STRIDE,
                               dtype=torch.int64, device=gpu)
        counters[1::native_mod.EVENT_ACTIVITY_STRIDE] = 7      # between slots: untouched
        extra = {"delta": torch.empty(batch * 3000, device=gpu)} if advance_only else {}
        s, _, _, _ = ext.dendritic_event(
            native.state, native.dendritic_state, native.adaptation_state, native._parameters(),
            current, emitted, native.theta, t.out_rowptr, t.dst, t.out_weight_index,
            t.in_weight, None, 0.3, None, 0.1, pending=pending, activity=counters,
            advance_only=advance_only, **extra)
        active = (s - emitted).abs() >= native.theta
        expected = int((active.long() * degree).sum())
        slots = counters.view(native_mod.EVENT_ACTIVITY_SLOTS, native_mod.EVENT_ACTIVITY_STRIDE)
        print(f"activity batch={batch} theta={theta} advance_only={advance_only}: "
              f"{int(slots[:, 0].sum())} counted, {expected} expected", flush=True)
        assert int(slots[:, 0].sum()) == expected
        assert bool((slots[:, 1] == 7).all()) and int(slots[:, 2:].abs().sum()) == 0
        # Both forms fold pending_in into the current and zero it.
        assert torch.equal(current, before + folded.to(gpu).view(3000, batch).t())
        assert int(torch.count_nonzero(pending[0])) == 0


def test_auto_switches_with_activity(gpu):
    """theta = 0 makes every pair active: "auto" turns to the matrix product after its
    first sample; quiescent (theta above every residual) it scatters; both stay on the
    oracle."""
    case = make_case(4000, 80_000, 9, gpu)
    for theta, want in ((0.0, "matrix"), (2.0, "event")):
        native = NativeDendriticPELSRuntime(case.topology, case.model,
                                            torch.zeros(2, 4000, device=gpu), theta=theta,
                                            propagation="auto", policy_interval=4)
        oracle = ort.PelsOracle(case.graph, case.params, torch.zeros(2, 4000), theta=theta)
        seen = []
        for _ in range(40):
            seen.append(native.selected_path)
            native.step(0.25, dendritic_drive=0.1)
            oracle.step(0.25, 0.1)
            torch.cuda.synchronize()
        print(f"auto theta={theta}: paths {''.join(p[0] for p in seen)}", flush=True)
        assert seen[0] == "event" and seen[-1] == want
        assert set(seen[8:]) == {want}
        assert state_error(native, oracle) <= (1e-5 if theta == 0 else 1e-3)
        assert max_err(native.persistent_current,
                       ort.propagate(ort.csr_matrix(case.graph), native.emitted_state.cpu())) <= 1e-5


@pytest.mark.parametrize("batch", [1, 3])
def test_csr_spmm_accumulates_in_place(gpu, batch):
    """ns_csr_spmm with accumulate: out += W @ S, any distinct-element strides."""
    case = make_case(2000, 30_000, 7, gpu)
    gen = torch.Generator().manual_seed(batch)
    source = torch.rand(batch, 2000, generator=gen).to(gpu)
    start = torch.rand(2000, batch, generator=gen).to(gpu).t()     # neuron-major view
    out = start.clone().t().contiguous().t()
    native = NativeDendriticPELSRuntime(case.topology, case.model,
                                        torch.zeros(batch, 2000, device=gpu), theta=0.0)
    t = case.topology
    product = native.extension.csr_spmm(source, t.in_rowptr, t.in_col, t.in_weight)
    returned = native.extension.csr_spmm(source, t.in_rowptr, t.in_col, t.in_weight,
                                         accumulate_into=out)
    assert returned is out
    assert torch.equal(out, start + product)
    expected = ort.propagate(ort.csr_matrix(case.graph), source.cpu()) + start.cpu()
    assert max_err(out, expected) <= 1e-5
    with pytest.raises(RuntimeError, match="must not overlap itself"):
        native.extension.csr_spmm(source, t.in_rowptr, t.in_col, t.in_weight,
                                  accumulate_into=torch.zeros(1, device=gpu).expand(batch, 2000))
