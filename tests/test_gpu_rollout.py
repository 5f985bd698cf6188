"""Graph-captured multi-tick rollouts (MI355X): bitwise equal to eager native
ticks, with fixed and per-tick staged inputs, and on the reference-held
brainwaves trajectory (chunks of 32 and 100 ticks) within 5e-7."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import brainwaves as bw
from cases import column_drive, make_case, model_to, standard_model
from neurosim_gpu import MatrixRollout, NativeDendriticMatrixRuntime, random_topology, topology_to

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


@pytest.mark.parametrize("batch,fmt", [(1, None), (8, None), (1, "fp8"), (3, "nvfp4")])
def test_graph_rollout_matches_eager(gpu, batch, fmt):
    print(f"case rollout fixed drives B={batch} fmt={fmt}", flush=True)
    case = make_case(4000, 80_000, 2, gpu)
    drive = column_drive(batch).to(gpu)
    kwargs = {} if fmt is None else {"weight_format": fmt}
    eager = NativeDendriticMatrixRuntime(case.topology, case.model,
                                         torch.zeros(batch, 4000, device=gpu), **kwargs)
    seeded = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(batch, 4000, device=gpu), **kwargs)
    for _ in range(3):            # non-trivial starting states
        eager.step(drive, dendritic_drive=0.1)
        seeded.step(drive, dendritic_drive=0.1)
    rollout = MatrixRollout(seeded, 16, drive=drive, dendritic_drive=0.1)
    for replay in range(3):
        rollout.run()
        # eager work between replays, then compare every replay
        for _ in range(16):
            eager.step(drive, dendritic_drive=0.1)
        torch.cuda.synchronize()
        for field in FIELDS:
            assert torch.equal(getattr(rollout, field), getattr(eager, field)), (replay, field)
    rollout.write_back()
    seeded.step(drive, dendritic_drive=0.1)
    eager.step(drive, dendritic_drive=0.1)
    assert torch.equal(seeded.state, eager.state)


@pytest.mark.parametrize("batch,shape", [(1, "full"), (2, "column"), (4, "neuron"), (16, "full")])
def test_staged_per_tick_inputs_match_eager(gpu, batch, shape):
    """Per-tick drives read from [T, B|1, N|1] buffers inside the graph, refilled
    between replays, plus an odd eager tail: bitwise the eager ticks."""
    print(f"case rollout staged drives B={batch} shape={shape}", flush=True)
    n, ticks = 3000, 12
    case = make_case(n, 60_000, 5, gpu)
    dims = {"full": (batch, n), "column": (batch, 1), "neuron": (1, n)}[shape]
    gen = torch.Generator().manual_seed(batch)

    def inputs():
        return (torch.rand((ticks, *dims), generator=gen) * 0.4,
                torch.rand((ticks, *dims), generator=gen) * 0.2)

    eager = NativeDendriticMatrixRuntime(case.topology, case.model,
                                         torch.zeros(batch, n, device=gpu))
    seeded = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(batch, n, device=gpu))
    soma, dend = inputs()
    staged = (soma.to(gpu), dend.to(gpu))
    rollout = MatrixRollout(seeded, ticks, drive=staged[0], dendritic_drive=staged[1])
    for replay in range(4):
        if replay:
            soma, dend = inputs()
            rollout.stage(soma.to(gpu), dend.to(gpu))
        rollout.run()
        for t in range(ticks):
            eager.step(soma[t].to(gpu).expand(batch, n),
                       dendritic_drive=dend[t].to(gpu).expand(batch, n))
        torch.cuda.synchronize()
        for field in FIELDS:
            assert torch.equal(getattr(rollout, field), getattr(eager, field)), (replay, field)
    soma, dend = inputs()
    rollout.stage(soma.to(gpu), dend.to(gpu))
    rollout.advance(5)                       # eager tail of an odd count, then a replay
    for t in range(5):
        eager.step(soma[t].to(gpu).expand(batch, n), dendritic_drive=dend[t].to(gpu).expand(batch, n))
    rollout.advance(ticks)
    for t in range(ticks):
        eager.step(soma[t].to(gpu).expand(batch, n), dendritic_drive=dend[t].to(gpu).expand(batch, n))
    for field in FIELDS:
        assert torch.equal(getattr(rollout, field), getattr(eager, field)), field


@pytest.mark.parametrize("batch", [1, 16])
def test_rollout_keeps_its_weights_after_the_runtime_moves_on(gpu, batch):
    """The captured ticks read the construction-time slot-order weights.  Two
    recorded (autograd) ticks and a weight change on the runtime rebuild its
    slot copies; the replays must still equal eager ticks on the old weights."""
    print(f"case rollout weight lifetime B={batch}", flush=True)
    n = 140_000 if batch == 16 else 5000     # "auto" takes bands from 131,072 neurons
    topology_cpu = random_topology(n, 10 * n, device="cpu", seed=9)
    model, _ = standard_model(n)
    model = model_to(model, gpu)
    kernel = "panels" if batch == 1 else "bands"
    runtime = NativeDendriticMatrixRuntime(topology_to(topology_cpu, gpu), model,
                                           torch.zeros(batch, n, device=gpu), kernel=kernel)
    assert runtime.kernel == kernel
    witness = NativeDendriticMatrixRuntime(topology_to(topology_cpu, gpu), model,
                                           torch.zeros(batch, n, device=gpu), kernel=kernel)
    rollout = MatrixRollout(runtime, 8, drive=0.2, dendritic_drive=0.1)
    if batch == 1:
        runtime.state = torch.full((1, n), 0.3, device=gpu, requires_grad=True)
        for _ in range(2):                   # the second recorded tick builds a slot copy
            runtime.step(0.2, dendritic_drive=0.1)
        runtime.state.sum().backward()
    with torch.no_grad():
        runtime.topology.in_weight.mul_(2.0)  # new values: a rebuilt copy differs
    with torch.inference_mode():
        runtime.step(0.2, dendritic_drive=0.1)
    junk = [torch.full((runtime.topology.n_edges * 2,), 7.0, device=gpu) for _ in range(4)]
    for _ in range(3):
        rollout.run()
        for _ in range(8):
            witness.step(0.2, dendritic_drive=0.1)
        torch.cuda.synchronize()
        for field in FIELDS:
            assert torch.equal(getattr(rollout, field), getattr(witness, field)), field
    del junk


def test_rollout_rejects_odd_ticks_and_bad_staging(gpu):
    case = make_case(100, 1000, 2, gpu)
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 100, device=gpu))
    with pytest.raises(ValueError, match="even"):
        MatrixRollout(runtime, 3)
    with pytest.raises(ValueError, match="one slice per tick"):
        MatrixRollout(runtime, 4, drive=torch.zeros(3, 1, 100, device=gpu))
    with pytest.raises(ValueError, match="broadcast"):
        MatrixRollout(runtime, 4, drive=torch.zeros(4, 2, 100, device=gpu))
    rollout = MatrixRollout(runtime, 4, drive=0.2)
    with pytest.raises(ValueError, match="not staged"):
        rollout.stage(torch.zeros(4, 1, 100, device=gpu))


@pytest.mark.parametrize("chunk", [32, 100])
def test_brainwaves_through_graph_chunks(gpu, chunk):
    """The reference-held brainwaves protocol (experiments/compartmental_brainwaves.py)
    driven through graph-captured chunks with per-tick staged inputs: 512 shared
    warm-up ticks, then 4096 ticks with row 0 driven and row 1 input-free.  The
    per-tick population means must match the reference's within 5e-7."""
    print(f"case brainwaves rollout chunk={chunk} ticks=4608", flush=True)
    meta, gold = bw.meta(), bw.golden()
    topology = random_topology(bw.NEURONS, bw.CANDIDATES, device="cpu", seed=meta["graph_seed"])
    assert topology.n_edges == meta["actual_edges"]
    model, _ = standard_model(bw.NEURONS)
    runtime = NativeDendriticMatrixRuntime(topology_to(topology, gpu), model_to(model, gpu),
                                           torch.zeros(2, bw.NEURONS, device=gpu))
    ticks = meta["ticks_per_condition"]
    total = bw.WARMUP + ticks
    soma, dend = bw.neuron_inputs(total)
    # Per tick and row: rows share the input during warm-up; row 1 gets none after.
    rows = np.ones((total, 2, 1), np.float32)
    rows[bw.WARMUP:, 1] = 0.0
    soma_rows = torch.from_numpy(soma[:, None, :] * rows)
    dend_rows = torch.from_numpy(dend[:, None, :] * rows)
    staged = (torch.empty(chunk, 2, bw.NEURONS, device=gpu),
              torch.empty(chunk, 2, bw.NEURONS, device=gpu))
    rollout = MatrixRollout(runtime, chunk, drive=staged[0], dendritic_drive=staged[1], trace=True)
    means = torch.empty(total, 2, dtype=torch.float64, device=gpu)
    done = 0
    while done < total:
        count = min(chunk, total - done)
        part = slice(done, done + count)
        rollout.stage(_pad(soma_rows[part], chunk).to(gpu), _pad(dend_rows[part], chunk).to(gpu))
        rollout.advance(count)
        means[done:done + count] = rollout.trace[:count].double().mean(dim=2)
        if done < bw.WARMUP <= done + count:
            at = bw.WARMUP - done - 1        # the last warm-up tick's state
            assert abs(float(rollout.trace[at, 0].double().mean())
                       - meta["shared_initial_state_means"]["state"]) < 5e-7
        done += count
    trace = means[bw.WARMUP:].float().double().cpu().numpy()
    err_driven = np.abs(trace[:, 0] - gold["driven_mean"]).max()
    err_zero = np.abs(trace[:, 1] - gold["zero_mean"]).max()
    print(f"brainwaves chunk {chunk}: max error driven {err_driven:.3e} zero {err_zero:.3e}")
    assert err_driven < 5e-7 and err_zero < 5e-7


def _pad(values: torch.Tensor, ticks: int) -> torch.Tensor:
    """The last chunk's inputs padded to a whole chunk (the padding is not read)."""
    out = torch.zeros((ticks, *values.shape[1:]), dtype=values.dtype)
    out[: values.shape[0]] = values
    return out
