"""Ticks captured into a HIP graph straight after construction.

A runtime builds derived weight arrays (slot-order copies, encoded payloads,
the source-major copy for the scatter) on its first eager ticks.  Built while
a stream is captured, such an array would be filled only when the graph
replays, and the eager ticks after the capture would read it unfilled.  So
under capture the runtimes build none: float32 panels read in_weight in place
(the indexed plan), the scatter gathers through out_weight_index, and the
arrays with no in-place form (band slots, fp8/NVFP4/fp16 payloads) raise,
asking for one eager tick first.  Each case here captures four ticks of a fresh
runtime, puts its states back, runs eager ticks and compares them with a twin
that never saw a capture; the replayed graph must give the twin's four ticks.
"""

from __future__ import annotations

import pytest
import torch

from cases import make_case
from neurosim_gpu import NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime

pytestmark = pytest.mark.gpu
N, M, SEED = 3000, 60_000, 11
MATRIX_FIELDS = ("state", "dendritic_state", "adaptation_state")
PELS_FIELDS = MATRIX_FIELDS + ("emitted_state", "persistent_current")


def capture(runtime, fields, ticks=4):
    """Capture ``ticks`` steps; returns the graph, its last tick's three state
    planes and the planes its first tick reads (kept alive for the replays).
    The runtime's states are put back to copies of those read planes."""
    originals = [getattr(runtime, f) for f in fields]
    saved = [value.clone() for value in originals]
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _ in range(ticks):
                runtime.step(0.3, dendritic_drive=0.1)
    torch.cuda.current_stream().wait_stream(side)
    outputs = [getattr(runtime, f) for f in MATRIX_FIELDS]
    for f, value in zip(fields, saved):
        setattr(runtime, f, value)
    return graph, outputs, originals


@pytest.mark.parametrize("kernel,batch", [("rows", 2), ("panels", 1), ("panels", 2)])
def test_matrix_ticks_captured_first_then_eager(gpu, kernel, batch):
    print(f"case capture-first matrix kernel={kernel} B={batch}", flush=True)
    case = make_case(N, M, SEED, gpu)
    options = dict(kernel=kernel, **({"panel_width": 1024} if kernel == "panels" else {}))
    initial = torch.full((batch, N), 0.2, device=gpu)
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model, initial.clone(), **options)
    twin = NativeDendriticMatrixRuntime(case.topology, case.model, initial.clone(), **options)
    graph, outputs, _inputs = capture(runtime, MATRIX_FIELDS)
    for _ in range(4):
        runtime.step(0.3, dendritic_drive=0.1)
        twin.step(0.3, dendritic_drive=0.1)
    for f in MATRIX_FIELDS:
        assert torch.equal(getattr(runtime, f), getattr(twin, f)), (kernel, f)
    graph.replay()
    torch.cuda.synchronize()
    for f, value in zip(MATRIX_FIELDS, outputs):
        assert torch.equal(value, getattr(twin, f)), (kernel, f)


@pytest.mark.parametrize("options", [dict(weight_format="fp8", kernel="panels"),
                                     dict(weight_format="nvfp4", kernel="panels"),
                                     dict(weight_dtype=torch.float16, kernel="rows"),
                                     dict(kernel="bands")])
def test_capture_before_any_eager_tick_needs_one_where_no_in_place_form_exists(gpu, options):
    print(f"case capture-first refused {options}", flush=True)
    case = make_case(N, M, SEED, gpu)
    batch = 4 if options.get("kernel") == "bands" else 1
    runtime = NativeDendriticMatrixRuntime(case.topology, case.model,
                                           torch.full((batch, N), 0.2, device=gpu), **options)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with pytest.raises(RuntimeError, match="run one eager tick before capturing"):
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                runtime.step(0.3, dendritic_drive=0.1)
    torch.cuda.synchronize()
    del graph
    # After one eager tick the same capture works.
    runtime.step(0.3, dendritic_drive=0.1)
    again, _, _inputs = capture(runtime, MATRIX_FIELDS, ticks=2)
    again.replay()
    torch.cuda.synchronize()


@pytest.mark.parametrize("options", [dict(), dict(propagation="matrix"),
                                     dict(propagation="matrix", kernel="panels")])
def test_pels_ticks_captured_first_then_eager(gpu, options):
    print(f"case capture-first PELS {options}", flush=True)
    case = make_case(N, M, SEED, gpu)
    initial = torch.zeros(1, N, device=gpu)
    runtime = NativeDendriticPELSRuntime(case.topology, case.model, initial.clone(),
                                         theta=0.02, **options)
    twin = NativeDendriticPELSRuntime(case.topology, case.model, initial.clone(), theta=0.02,
                                      **options)
    graph, outputs, _inputs = capture(runtime, PELS_FIELDS)
    for _ in range(6):
        runtime.step(0.3, dendritic_drive=0.1)
        twin.step(0.3, dendritic_drive=0.1)
    # The scatter adds float32 atomics in any order: the runs agree to rounding.
    for f in PELS_FIELDS:
        torch.testing.assert_close(getattr(runtime, f), getattr(twin, f), rtol=0, atol=1e-5)
    # The graph shares the runtime's current and pending buffers, so it is replayed
    # only now, once, to show the captured ticks run.
    graph.replay()
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(value).all()) for value in outputs)
