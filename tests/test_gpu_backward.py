"""Native float32 backward of the matrix tick (ns_dendritic_step_backward)
against the oracle's gradients.

The reference's native runtime records no graph of its own: whenever a
gradient is needed it runs its torch step (native_compartmental.py:104-108),
and autograd differentiates torch.sparse.mm and the update ops.  Here the
same gradients come from HIP kernels.  The expected values come from
oracle/grad.py: float64 autograd through the oracle's update on the dense
weight matrix, pinned by finite differences (tests/test_oracle_grad.py), on
the same float32 inputs, so the tolerance (1e-4 of the largest gradient of
each tensor) covers only the native float32 arithmetic.  Covers one tick with every input requiring a
gradient (states, [B,N] and [B,1] drives, the six parameters, the weights),
eight-tick backpropagation through time, scalar drives, stride-0 parameters,
repeatability, and the source-major weight copy the transposed product streams
from the second backward of a weight version on.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import grad as og
from oracle import topology as otop
from neurosim_gpu import (DendriticDynamics, Dynamics, NativeDendriticMatrixRuntime,
                          SparseTopology)

pytestmark = pytest.mark.gpu


def graph(n: int, m: int, seed: int) -> otop.Graph:
    return otop.random_graph(n, m, seed=seed)


def topology(g: otop.Graph, dtype, device) -> SparseTopology:
    fields = dict(src=g.src, dst=g.dst, weight=g.weight, out_rowptr=g.out_rowptr,
                  in_rowptr=g.in_rowptr, in_col=g.in_col, out_weight_index=g.out_weight_index,
                  in_weight=g.in_weight)
    tensors = {k: torch.from_numpy(np.asarray(v)) for k, v in fields.items()}
    for k in ("weight", "in_weight"):
        tensors[k] = tensors[k].to(dtype)
    return SparseTopology(n_neurons=g.n, **{k: v.to(device) for k, v in tensors.items()})


def leaf(value: np.ndarray, dtype, device) -> torch.Tensor:
    return torch.tensor(value, dtype=dtype, device=device).requires_grad_(True)


def model(values: dict, dtype, device, expanded: bool) -> DendriticDynamics:
    def vec(name):
        if expanded and name in ("coupling", "strength"):
            return leaf(values[name][:1], dtype, device)[0].expand(values["alpha"].size)
        return leaf(values[name], dtype, device)
    return DendriticDynamics(Dynamics(vec("alpha"), vec("gain")), vec("rho_d"), vec("rho_a"),
                             vec("coupling"), vec("strength"))


def params_of(m: DendriticDynamics):
    return [m.soma.alpha, m.soma.gain, m.dendrite_decay, m.adaptation_decay, m.coupling,
            m.adaptation_strength]


def base(p):
    """The leaf behind a parameter (an expanded scalar's 0-d base)."""
    return p._base if p._base is not None else p


def run(runtime_cls, g, inputs, dtype, device, ticks, *, scalar_drives, expanded,
        source_major=True, transposed_panels=True, **kw):
    topo = topology(g, dtype, device)
    topo.in_weight.requires_grad_(True)
    mdl = model(inputs["params"], dtype, device, expanded)
    state0 = leaf(inputs["state"], dtype, device)
    rt = runtime_cls(topo, mdl, state0.detach(), **kw)
    if hasattr(rt, "source_major_weights"):
        rt.source_major_weights.enabled = source_major
    if hasattr(rt, "transposed_panels_enabled"):
        rt.transposed_panels_enabled = transposed_panels
    rt.state = state0
    rt.dendritic_state = leaf(inputs["dendrite"], dtype, device)
    rt.adaptation_state = leaf(inputs["adaptation"], dtype, device)
    dendrite0, adaptation0 = rt.dendritic_state, rt.adaptation_state
    if scalar_drives:
        drive, dendritic = 0.2, 0.1
    else:
        drive = leaf(inputs["drive"], dtype, device)
        dendritic = leaf(inputs["dendritic"], dtype, device)
    for _ in range(ticks):
        rt.step(drive, dendritic_drive=dendritic)
    r = {k: torch.tensor(v, dtype=dtype, device=device) for k, v in inputs["probe"].items()}
    loss = (rt.state * r["s"]).sum() + (rt.dendritic_state * r["d"]).sum() + \
        (rt.adaptation_state * r["a"]).sum()
    loss.backward()
    grads = {"weight": topo.in_weight.grad, "state": state0.grad, "dendrite": dendrite0.grad,
             "adaptation": adaptation0.grad}
    if not scalar_drives:
        grads["drive"], grads["dendritic"] = drive.grad, dendritic.grad
    for name, p in zip(("alpha", "gain", "rho_d", "rho_a", "coupling", "strength"), params_of(mdl)):
        grads[name] = base(p).grad
    return grads, rt


def inputs_for(g, batch, seed):
    rng = np.random.default_rng(seed)
    n = g.n
    return {
        "state": rng.uniform(0, 1, (batch, n)), "dendrite": rng.uniform(-1, 1, (batch, n)),
        "adaptation": rng.uniform(0, 1, (batch, n)),
        "drive": rng.uniform(-0.5, 0.8, (batch, n)), "dendritic": rng.uniform(-0.3, 0.3, (batch, 1)),
        "params": {"alpha": rng.uniform(0.5, 0.9, n), "gain": rng.uniform(0.5, 1.5, n),
                   "rho_d": rng.uniform(0.5, 0.95, n), "rho_a": rng.uniform(0.8, 0.99, n),
                   "coupling": rng.uniform(0.2, 0.8, n), "strength": rng.uniform(0.05, 0.4, n)},
        "probe": {"s": rng.standard_normal((batch, n)), "d": rng.standard_normal((batch, n)),
                  "a": rng.standard_normal((batch, n))},
    }


def oracle_gradients(g, inputs, ticks, *, scalar_drives, expanded) -> dict:
    """The oracle's gradients on the inputs as the native run sees them
    (rounded to float32), keyed like ``run``'s."""
    f32 = lambda v: np.asarray(v, np.float32).astype(np.float64)  # noqa: E731
    n = g.n
    params = {}
    for name, key in zip(og.PARAM_NAMES, ("alpha", "gain", "rho_d", "rho_a", "coupling", "strength")):
        value = f32(inputs["params"][key])
        params[name] = np.full(n, value[0]) if expanded and key in ("coupling", "strength") else value
    x = og.TickInputs(state=f32(inputs["state"]), dendrite=f32(inputs["dendrite"]),
                      adaptation=f32(inputs["adaptation"]),
                      drive=0.2 if scalar_drives else f32(inputs["drive"]),
                      dendritic=0.1 if scalar_drives else f32(inputs["dendritic"]),
                      params=params, probe={k: f32(inputs["probe"][k]) for k in ("s", "d", "a")})
    got = og.tick_gradients(g, x, ticks)
    out = {"weight": got["weight"], "state": got["state"], "dendrite": got["dendrite"],
           "adaptation": got["adaptation"]}
    if not scalar_drives:
        out["drive"], out["dendritic"] = got["drive"], got["dendritic"]
    for name in og.PARAM_NAMES:
        value = got[name]
        if expanded and name in ("coupling", "strength"):
            value = value.sum()                  # the gradient of the 0-d base
        out[name] = value
    return {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in out.items()}


def compare(native: dict, reference: dict, rtol: float = 1e-4) -> None:
    assert native.keys() == reference.keys()
    for name, want in reference.items():
        got = native[name]
        assert got is not None and want is not None, name
        got = got.detach().double().cpu().reshape(want.shape)
        scale = float(want.abs().max())
        err = float((got - want.cpu()).abs().max())
        assert err <= rtol * max(scale, 1e-12), f"{name}: max error {err:.3e}, scale {scale:.3e}"


@pytest.mark.parametrize("ticks,batch,scalar_drives,expanded", [
    (1, 3, False, False), (1, 1, True, True), (8, 2, False, True), (8, 4, True, False)])
def test_gradients_match_the_oracle(gpu, ticks, batch, scalar_drives, expanded):
    print(f"case backward ticks={ticks} batch={batch} scalar_drives={scalar_drives} "
          f"expanded={expanded}", flush=True)
    g = graph(600, 12_000, 9)
    inputs = inputs_for(g, batch, ticks * 10 + batch)
    kw = dict(scalar_drives=scalar_drives, expanded=expanded)
    native, rt = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, ticks, **kw)
    assert rt.last_backend == "native-autograd"
    compare(native, oracle_gradients(g, inputs, ticks, **kw))


@pytest.mark.parametrize("ticks,batch,width", [(2, 1, 1000), (4, 2, 1000), (3, 1, None)])
def test_transposed_product_on_panels_matches_the_oracle(gpu, ticks, batch, width):
    """With the forward on column panels the backward's transposed product
    W^T @ g runs, from the second backward of a weight version on, on a panel
    layout of the transposed matrix (rows = sources; three panels at width
    1000, so a second kernel adds the per-panel sums into d_state); the
    gradients through several ticks match the oracle, and the out-edge walk
    to float32 summation order."""
    print(f"case backward transposed panels ticks={ticks} batch={batch} width={width}",
          flush=True)
    g = graph(3000, 90_000, 17)
    inputs = inputs_for(g, batch, 40 + batch)
    kw = dict(scalar_drives=False, expanded=False, kernel="panels", panel_width=width)
    native, rt = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, ticks, **kw)
    assert rt._transposed is not None and rt._transposed._seen == ticks
    assert rt._transposed.layout._slot_weights is not None     # the panels ran
    assert rt._transposed.layout.n_panels == (3 if width else 1)
    compare(native, oracle_gradients(g, inputs, ticks, scalar_drives=False, expanded=False))
    walked, rt2 = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, ticks,
                      transposed_panels=False, **kw)
    assert rt2._transposed is None
    compare(native, {k: v.detach().double().cpu() for k, v in walked.items()}, rtol=1e-5)


@pytest.mark.parametrize("batch", [1, 2])
def test_first_backward_of_a_weight_version_reads_the_weights_in_place(gpu, batch):
    """One recorded tick per weight version (an optimizer step before every pass):
    the transposed product runs on the indexed plan, reading the CSR weights
    through the slots' edge numbers, where it used to walk the out-edges.  The
    gradients match the oracle and equal bitwise those of a second backward of the
    same version, which streams the slot-order copy."""
    print(f"case backward indexed transposed plan batch={batch}", flush=True)
    g = graph(3000, 90_000, 17)
    inputs = inputs_for(g, batch, 60 + batch)
    kw = dict(scalar_drives=False, expanded=False, kernel="panels", panel_width=1000)
    first, rt = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, 1, **kw)
    assert rt._transposed is not None and rt._transposed._seen == 1
    assert rt._transposed.layout._slot_weights is None      # the indexed plan ran
    compare(first, oracle_gradients(g, inputs, 1, scalar_drives=False, expanded=False))

    def again():
        """The same tick and loss once more, on the same weights (leaves reset)."""
        topo, mdl = rt.topology, rt.compartment_dynamics
        for t in [topo.in_weight, *params_of(mdl)]:
            base(t).grad = None
        state0 = leaf(inputs["state"], torch.float32, gpu)
        rt.state = state0
        rt.dendritic_state = leaf(inputs["dendrite"], torch.float32, gpu)
        rt.adaptation_state = leaf(inputs["adaptation"], torch.float32, gpu)
        drive = leaf(inputs["drive"], torch.float32, gpu)
        dendritic = leaf(inputs["dendritic"], torch.float32, gpu)
        rt.step(drive, dendritic_drive=dendritic)
        r = {k: torch.tensor(v, dtype=torch.float32, device=gpu)
             for k, v in inputs["probe"].items()}
        loss = (rt.state * r["s"]).sum() + (rt.dendritic_state * r["d"]).sum() + \
            (rt.adaptation_state * r["a"]).sum()
        loss.backward()
        return {"weight": topo.in_weight.grad, "state": state0.grad}

    second = again()
    assert rt._transposed.layout._slot_weights is not None  # the slot-order copy ran
    for name in second:
        assert torch.equal(first[name], second[name]), name


def test_backward_is_repeatable(gpu):
    print("case backward repeatable", flush=True)
    g = graph(2000, 60_000, 3)
    inputs = inputs_for(g, 2, 5)
    first, _ = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, 4,
                   scalar_drives=False, expanded=False)
    second, _ = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, 4,
                    scalar_drives=False, expanded=False)
    for name in first:
        assert torch.equal(first[name], second[name]), name


def test_source_major_weight_copy_changes_no_gradient(gpu):
    """Backpropagation through 6 ticks: from the second backward on, the transposed
    product streams a source-major copy of the weights instead of gathering them;
    the gradients are bitwise those of the gather."""
    print("case backward source-major weights", flush=True)
    g = graph(3000, 90_000, 12)
    inputs = inputs_for(g, 2, 21)
    kw = dict(scalar_drives=False, expanded=False)
    copied, rt = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, 6, **kw)
    assert rt.source_major_weights._values is not None, "the copy was built"
    assert rt.source_major_weights._seen == 6
    gathered, rt2 = run(NativeDendriticMatrixRuntime, g, inputs, torch.float32, gpu, 6,
                        source_major=False, **kw)
    assert rt2.source_major_weights._values is None
    for name in copied:
        assert torch.equal(copied[name], gathered[name]), name


def test_recorded_ticks_move_to_panels_for_a_reused_weight_version(gpu):
    """A recorded tick takes the row kernel the first time it sees a weight
    version and the panel kernel from the second on; an in-place weight update
    sends it back to the row kernel.  The states follow the inference ticks
    (panels) to float32 summation-order differences."""
    print("case backward recorded panel ticks", flush=True)
    g = graph(4000, 100_000, 6)
    topo = topology(g, torch.float32, gpu)
    topo.in_weight.requires_grad_(True)
    soma = Dynamics(torch.full((4000,), .72, device=gpu), torch.full((4000,), .8, device=gpu))
    mdl = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4., tau_adaptation=25.)
    plain = NativeDendriticMatrixRuntime(topo, mdl, torch.zeros(1, 4000, device=gpu),
                                         kernel="panels")
    recorded = NativeDendriticMatrixRuntime(topo, mdl, torch.zeros(1, 4000, device=gpu),
                                            kernel="panels")
    assert recorded.kernel == "panels"
    for tick in range(5):
        with torch.no_grad():
            plain.step(0.2, dendritic_drive=0.1)
        recorded.step(0.2, dendritic_drive=0.1)
        assert (recorded._panel_struct_key is not None) == (tick >= 1)
    for name in ("state", "dendritic_state", "adaptation_state"):
        err = float((getattr(recorded, name) - getattr(plain, name)).abs().max())
        assert err <= 2e-6, (name, err)
    recorded.state.sum().backward()
    assert topo.in_weight.grad is not None and bool(torch.isfinite(topo.in_weight.grad).all())
    with torch.no_grad():
        topo.in_weight.mul_(0.5)                 # a new weight version: rows again, once
    recorded.step(0.2, dendritic_drive=0.1)
    assert recorded._recorded_seen == 1


def test_forward_of_a_recorded_tick_equals_the_inference_tick(gpu):
    """Recording for autograd changes nothing in the forward values."""
    print("case backward forward values", flush=True)
    g = graph(1000, 20_000, 0)
    topo = topology(g, torch.float32, gpu)
    soma = Dynamics(torch.full((1000,), .72, device=gpu), torch.full((1000,), .8, device=gpu))
    mdl = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4., tau_adaptation=25.)
    plain = NativeDendriticMatrixRuntime(topo, mdl, torch.zeros(2, 1000, device=gpu), kernel="rows")
    recorded = NativeDendriticMatrixRuntime(topo, mdl, torch.zeros(2, 1000, device=gpu), kernel="rows")
    drive = torch.full((2, 1000), 0.2, device=gpu, requires_grad=True)
    for _ in range(5):
        with torch.no_grad():
            plain.step(drive.detach(), dendritic_drive=0.1)
        recorded.step(drive, dendritic_drive=0.1)
    assert recorded.last_backend == "native-autograd"
    assert torch.equal(plain.state, recorded.state.detach())
    assert torch.equal(plain.dendritic_state, recorded.dendritic_state.detach())
