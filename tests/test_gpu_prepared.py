"""The eager ticks' prepared launches (PreparedTick, PreparedEvent) against the
validated extension calls they stand in for (dendritic_step, dendritic_event).

Both launch the same kernels on the same argument values, so the matrix tick is
compared bitwise over several ticks, in every kernel family and weight format,
with scalar and tensor drives.  The PELS tick is compared bitwise on the
advance outputs of a tick from identical inputs; its scatter adds float32
atomics in an arbitrary order, so the buffers it writes, and later ticks, are
compared within 1e-6.  Both also reject a mismatched state before launching.
"""

from __future__ import annotations

from dataclasses import replace

import pytest
import torch

from cases import column_drive, make_case
from neurosim_gpu import NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime
from neurosim_gpu.native import (EVENT_ACTIVITY_SLOTS, EVENT_ACTIVITY_STRIDE, PreparedEvent,
                                 PreparedTick, load_native_extension)

pytestmark = pytest.mark.gpu
N, M, SEED = 3000, 60_000, 7


def clone_planes(planes):
    """Neuron-major copies, as the kernels write their outputs."""
    out = []
    for p in planes:
        q = torch.empty(p.shape[1], p.shape[0], device=p.device).t()
        out.append(q.copy_(p))
    return out


@pytest.mark.parametrize("kernel,batch", [("rows", 1), ("rows", 3), ("panels", 1),
                                          ("panels", 2), ("bands", 4), ("bands", 8)])
@pytest.mark.parametrize("fmt", ["fp32", "fp16", "fp8", "nvfp4"])
def test_prepared_tick_equals_dendritic_step(gpu, kernel, batch, fmt):
    print(f"case prepared tick kernel={kernel} B={batch} fmt={fmt}", flush=True)
    case = make_case(N, M, SEED, gpu)
    options = ({} if fmt == "fp32" else {"weight_dtype": torch.float16} if fmt == "fp16"
               else {"weight_format": fmt})
    if kernel == "panels":
        options.update(panel_width=1024, panel_tiles=5)
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model,
                                           torch.full((batch, N), 0.2, device=gpu),
                                           kernel=kernel, **options)
    assert runtime.kernel == kernel
    ext = load_native_extension()
    weight, scales, _ = runtime._weights()
    extra = {}
    if kernel == "panels":
        extra["panels"] = runtime._panel_plan(weight, scales, reuse=True)
    elif kernel == "bands":
        extra["bands"] = runtime._band_plan(weight, scales)
    topo, params = case.topology, runtime._parameters()
    state = [torch.full((batch, N), 0.2, device=gpu), torch.zeros(batch, N, device=gpu),
             torch.zeros(batch, N, device=gpu)]
    tick = PreparedTick(ext, state[0], params, topo.in_rowptr, topo.in_col, weight, *scales,
                        **extra)
    assert tick.matches(state[0], params, topo.in_rowptr, topo.in_col, weight, *scales, **extra)
    drive = column_drive(batch).to(gpu).expand(batch, N)
    planes_a, planes_b = clone_planes(state), clone_planes(state)
    for t in range(6):
        u, us = (drive, 0.0) if t % 2 else (None, 0.2)
        planes_a = ext.dendritic_step(*planes_a, params, topo.in_rowptr, topo.in_col, weight,
                                      u, us, None, 0.1, 16, *scales, **extra)
        planes_b = tick(*planes_b, u, us, None, 0.1)
        for a, b in zip(planes_a, planes_b):
            assert b.stride() == a.stride()
            assert torch.equal(a, b), (kernel, batch, fmt, t)
    # A state plane that is not the last output is validated before the launch.
    with pytest.raises(RuntimeError, match="float32"):
        tick(planes_b[0].double(), planes_b[1], planes_b[2], None, 0.2, None, 0.1)
    with pytest.raises(RuntimeError, match="shape"):
        tick(planes_b[0][:, :-1], planes_b[1], planes_b[2], None, 0.2, None, 0.1)
    assert not tick.matches(torch.zeros(batch + 1, N, device=gpu), params, topo.in_rowptr,
                            topo.in_col, weight, *scales, **extra)


@pytest.mark.parametrize("mode", ["one_launch", "advance_only", "two_launch", "sampled"])
def test_prepared_event_equals_dendritic_event(gpu, mode):
    print(f"case prepared event mode={mode}", flush=True)
    batch = 2
    case = make_case(N, M, SEED, gpu)
    topo = case.topology
    runtime = NativeDendriticPELSRuntime(topo, case.model, torch.zeros(batch, N, device=gpu),
                                         theta=0.02)
    ext = load_native_extension()
    params = runtime._parameters()
    out_weight = topo.in_weight[topo.out_weight_index.long()].contiguous()
    use_pending = mode != "two_launch"
    advance_only = mode == "advance_only"
    sample = mode == "sampled"

    def buffers():
        return {"current": torch.zeros(batch, N, device=gpu),
                "pending": torch.zeros(2, batch * N, device=gpu),
                "delta": torch.zeros(batch * N, device=gpu),
                "activity": torch.zeros(EVENT_ACTIVITY_SLOTS * EVENT_ACTIVITY_STRIDE,
                                        dtype=torch.int64, device=gpu)}

    a, b = buffers(), buffers()
    tick = PreparedEvent(ext, runtime.state, params, runtime.theta, topo.out_rowptr, topo.dst,
                         topo.out_weight_index, topo.in_weight, delta=b["delta"],
                         pending=b["pending"] if use_pending else None,
                         activity=b["activity"])
    start = [torch.full((batch, N), 0.1, device=gpu), torch.zeros(batch, N, device=gpu),
             torch.zeros(batch, N, device=gpu), torch.zeros(batch, N, device=gpu)]
    planes_a, planes_b = clone_planes(start), clone_planes(start)
    for t in range(6):
        parity = t % 2
        extra = {"advance_only": advance_only}
        if advance_only or not use_pending:
            extra["delta"] = a["delta"]
        if use_pending:
            extra["pending"] = (a["pending"][parity],
                                None if advance_only else a["pending"][1 - parity])
        if sample:
            extra["activity"] = a["activity"]
        if not advance_only:
            extra["out_weight"] = out_weight
        planes_a = ext.dendritic_event(*planes_a[:3], params, a["current"], planes_a[3],
                                       runtime.theta, topo.out_rowptr, topo.dst,
                                       topo.out_weight_index, topo.in_weight, None, 0.3, None,
                                       0.1, **extra)
        planes_b = tick(*planes_b[:3], planes_b[3], b["current"], None, 0.3, None, 0.1,
                        parity=parity if use_pending else None, advance_only=advance_only,
                        sample=sample, out_weight=None if advance_only else out_weight)
        exact = t == 0
        for x, y in zip(planes_a, planes_b):
            if exact:
                assert torch.equal(x, y), (mode, t)
            else:
                torch.testing.assert_close(y, x, rtol=0, atol=1e-6)
        for key in ("current", "pending", "delta"):
            # Scatter targets (the pending buffers, or the current of the two-launch
            # tick) take float32 atomics in an arbitrary order.
            scattered = key == "pending" or (key == "current" and not use_pending)
            if exact and not scattered:
                assert torch.equal(a[key], b[key]), (mode, key)
            else:
                torch.testing.assert_close(b[key], a[key], rtol=0, atol=1e-6)
        if sample:
            assert torch.equal(a["activity"], b["activity"])
            assert int(a["activity"].sum()) > 0
    with pytest.raises(RuntimeError, match="shape"):
        tick(planes_b[0][:1], planes_b[1], planes_b[2], planes_b[3], b["current"], None, 0.3,
             None, 0.1, parity=0 if use_pending else None)


def test_runtime_steps_through_the_prepared_launch_and_revalidates(gpu):
    """The runtimes reuse one prepared launch while their arguments stay the same
    objects, and build a new one when the weights or parameters are replaced."""
    case = make_case(N, M, SEED, gpu)
    matrix = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(1, N, device=gpu), kernel="rows")
    pels = NativeDendriticPELSRuntime(case.topology, case.model, torch.zeros(1, N, device=gpu),
                                      theta=0.02)
    for runtime in (matrix, pels):
        runtime.step(0.2, dendritic_drive=0.1)
        first = runtime._prepared
        assert first is not None
        for _ in range(3):
            runtime.step(0.2, dendritic_drive=0.1)
        assert runtime._prepared is first
        # A restored (reassigned) state is validated, not trusted.
        runtime.state = runtime.state.clone()
        runtime.step(0.2, dendritic_drive=0.1)
        assert runtime._prepared is first
        model = runtime.compartment_dynamics
        runtime.compartment_dynamics = replace(model, coupling=model.coupling.clone())
        runtime.step(0.2, dendritic_drive=0.1)
        assert runtime._prepared is not first
        assert bool(torch.isfinite(runtime.state).all())


@pytest.mark.parametrize("batch", [1, 3])
def test_prepared_accumulate_equals_csr_spmm(gpu, batch):
    """current += W @ delta: the PELS matrix propagation's prepared launch against
    csr_spmm(accumulate_into=...), bitwise (no atomics: one lane group per row)."""
    print(f"case prepared accumulate B={batch}", flush=True)
    from neurosim_gpu.native import PreparedAccumulate

    case = make_case(N, M, SEED, gpu)
    topo = case.topology
    ext = load_native_extension()
    delta_storage = torch.randn(batch * N, generator=torch.Generator().manual_seed(3)).to(gpu)
    delta = torch.as_strided(delta_storage, (batch, N), (1, batch))
    a = torch.rand(batch, N, device=gpu)
    b = a.clone()
    product = PreparedAccumulate(ext, delta, topo.in_rowptr, topo.in_col, topo.in_weight, b)
    assert product.matches(delta, topo.in_rowptr, topo.in_col, topo.in_weight, b)
    assert not product.matches(delta, topo.in_rowptr, topo.in_col, topo.in_weight, a)
    for _ in range(3):
        ext.csr_spmm(delta, topo.in_rowptr, topo.in_col, topo.in_weight, accumulate_into=a)
        product()
        assert torch.equal(a, b)


@pytest.mark.parametrize("batch,drives,upstream,extras", [
    (1, "scalar", "all", "none"), (2, "tensor", "all", "current"),
    (1, "tensor", "state_only", "out_weight"), (2, "scalar", "all", "panels"),
    (3, "tensor", "state_only", "current")])
def test_prepared_backward_equals_dendritic_step_backward(gpu, batch, drives, upstream, extras):
    """The recorded tick's backward through PreparedBackward against the validated
    call, bitwise (every backward kernel is deterministic)."""
    print(f"case prepared backward B={batch} drives={drives} upstream={upstream} "
          f"extras={extras}", flush=True)
    from neurosim_gpu.native import PreparedBackward
    from neurosim_gpu.native_compartmental import TransposedPanels

    case = make_case(N, M, SEED, gpu)
    topo = case.topology
    runtime = NativeDendriticMatrixRuntime(topo, case.model, torch.zeros(batch, N, device=gpu),
                                           kernel="rows")
    ext, params = load_native_extension(), runtime._parameters()
    gen = torch.Generator().manual_seed(batch)
    planes = clone_planes([torch.rand(batch, N, generator=gen).to(gpu) for _ in range(3)])
    if drives == "tensor":
        u = column_drive(batch).to(gpu).expand(batch, N)
        v = torch.rand(batch, N, generator=gen).to(gpu)
        us = vs = 0.0
        need_drive = need_dendritic = True
    else:
        u = v = None
        us, vs = 0.2, 0.1
        need_drive = need_dendritic = False
    grads = [torch.randn(batch, N, generator=gen).to(gpu) for _ in range(3)]
    if upstream == "state_only":
        grads[1] = grads[2] = None
    extra = {}
    if extras == "current":
        current = clone_planes([torch.rand(batch, N, generator=gen).to(gpu)])[0]
        extra["current"] = current
    elif extras == "out_weight":
        extra["out_weight"] = topo.in_weight[topo.out_weight_index.long()].contiguous()
    elif extras == "panels":
        layout = TransposedPanels(topo, batch, gpu, max_panel_width=1024)
        from neurosim_gpu.native import PANEL_INDEXED

        # The first request gives the indexed plan, the second the slot-order copy.
        assert layout.plan(topo.in_weight).flags & PANEL_INDEXED
        extra["transposed_panels"] = layout.plan(topo.in_weight)
        assert not extra["transposed_panels"].flags & PANEL_INDEXED
    fixed = (topo.in_rowptr, topo.in_col, topo.in_weight, topo.out_rowptr, topo.dst,
             topo.out_weight_index)
    flags = dict(need_drive=need_drive, need_dendritic=need_dendritic, need_weight=True,
                 need_params=(True, False, True, True, False, True))
    expected = ext.dendritic_step_backward(*planes, params, fixed[0], fixed[1], fixed[2], u, us,
                                           v, vs, fixed[3], fixed[4], fixed[5], *grads,
                                           **flags, **extra)
    prepared = PreparedBackward(ext, planes[0], params, *fixed)
    assert prepared.matches(planes[0], params, *fixed)
    for _ in range(2):
        got = prepared(*planes, u, us, v, vs, *grads, **flags, **extra)
        for a, b in zip(expected[:6], got[:6]):
            assert (a is None) == (b is None)
            if a is not None:
                assert torch.equal(a, b)
        for a, b in zip(expected[6], got[6]):
            assert (a is None) == (b is None)
            if a is not None:
                assert torch.equal(a, b)
