"""The C-ABI library loads on a host without a GPU, exports every declared
symbol, plans rows correctly and rejects invalid arguments before launching.
No kernel runs here: every call either is host-only or fails validation.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from neurosim_gpu import native

HEADER = Path(__file__).resolve().parents[1] / "include" / "neurosim_hip.h"


@pytest.fixture(scope="module")
def lib():
    return native.load_library()


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    return re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(ns_\w+)\s*\(", text, flags=re.M)


def test_every_declared_symbol_is_exported(lib):
    names = declared_functions()
    assert set(names) == {"ns_abi_version", "ns_last_error", "ns_block_edges",
                          "ns_plan_row_blocks", "ns_dendritic_step", "ns_dendritic_event",
                          "ns_csr_spmm", "ns_plan_panels", "ns_panel_geometry",
                          "ns_encode_workspace_bytes", "ns_encode_weights",
                          "ns_encode_weights_no_alloc",
                          "ns_topology_workspace_bytes", "ns_build_topology",
                          "ns_step_backward_workspace_floats", "ns_dendritic_step_backward",
                          "ns_plan_bands", "ns_band_max_block_rows", "ns_dendritic_step_bands",
                          "ns_gather_slot_weights"}
    for name in names:
        assert hasattr(lib, name), name
    assert lib.ns_abi_version() == native.ABI_VERSION


def test_block_capacity_per_batch(lib):
    caps = {b: lib.ns_block_edges(b) for b in (0, 1, 2, 3, 4, 8, 16, 64)}
    assert caps[1] == caps[0] == 2048 and caps[2] == 2048
    assert caps[3] == caps[4] == caps[8] == caps[16] == caps[64] == 1024


def plan(lib, rowptr, capacity):
    rowptr = np.ascontiguousarray(rowptr, dtype=np.int32)
    count = ctypes.c_int64()
    rc = lib.ns_plan_row_blocks(rowptr.ctypes.data, rowptr.size - 1, capacity, None, 0,
                                ctypes.byref(count))
    assert rc == 0, lib.ns_last_error()
    bounds = np.empty(2 * (count.value + 1), np.int32)
    rc = lib.ns_plan_row_blocks(rowptr.ctypes.data, rowptr.size - 1, capacity,
                                bounds.ctypes.data, bounds.size, ctypes.byref(count))
    assert rc == 0, lib.ns_last_error()
    return bounds.reshape(-1, 2)


@pytest.mark.parametrize("degrees", [
    [20] * 1000, [0] * 700, [150] * 300, [5000, 3, 0, 2100, 1] + [7] * 50,
    list(np.random.default_rng(1).poisson(30, 2000)), [2045, 2046, 2047, 2048, 2049, 1]])
def test_planner_blocks_cover_rows_and_fit(lib, degrees):
    capacity = 2048
    rowptr = np.concatenate([[0], np.cumsum(degrees)]).astype(np.int32)
    bounds = plan(lib, rowptr, capacity)
    rows = bounds[:, 0]
    assert rows[0] == 0 and rows[-1] == len(degrees)
    assert np.all(np.diff(rows) >= 1)
    assert np.array_equal(bounds[:, 1], rowptr[rows])
    for r0, r1 in zip(rows[:-1], rows[1:]):
        span = rowptr[r1] - (rowptr[r0] & ~3)
        assert (r1 - r0 <= 256 and span <= capacity) or r1 - r0 == 1
        if r1 < len(degrees) and r1 - r0 < 256 and span <= capacity:
            # greedy: the next row would not have fit
            assert rowptr[r1 + 1] - (rowptr[r0] & ~3) > capacity


def test_planner_rejects_bad_rowptr(lib):
    count = ctypes.c_int64()
    bad = np.array([0, 5, 3], np.int32)
    assert lib.ns_plan_row_blocks(bad.ctypes.data, 2, 2048, None, 0, ctypes.byref(count)) != 0
    assert b"non-decreasing" in lib.ns_last_error()
    bad = np.array([1, 5], np.int32)
    assert lib.ns_plan_row_blocks(bad.ctypes.data, 1, 2048, None, 0, ctypes.byref(count)) != 0
    small = np.array([0, 5, 9], np.int32)
    bounds = np.empty(2, np.int32)
    assert lib.ns_plan_row_blocks(small.ctypes.data, 2, 2048, bounds.ctypes.data, 2,
                                  ctypes.byref(count)) != 0
    assert b"capacity" in lib.ns_last_error()


def fake_step_args(n=8, batch=2):
    """Host-memory pointers: valid for validation only (never launched)."""
    keep = [np.zeros((batch, n), np.float32) for _ in range(6)]
    params = [np.ones(n, np.float32) for _ in range(6)]
    rowptr = np.zeros(n + 1, np.int32)
    args = native._StepArgs()
    args.n_neurons, args.batch = n, batch
    planes = [native._Plane(k.ctypes.data, n, 1, 0.0) for k in keep[:3]]
    args.state, args.dendrite, args.adaptation = planes
    args.drive = native._Plane(None, 0, 0, 0.2)
    args.dendritic_drive = native._Plane(None, 0, 0, 0.1)
    for i, p in enumerate(params):
        args.params[i] = native._Vector(p.ctypes.data, 1)
    args.matrix = native._Csr(n, 0, rowptr.ctypes.data, None, None, native.WEIGHT_F32, None, None)
    bounds = np.array([0, 0, n, 0], np.int32)
    args.plan = native._RowPlan(bounds.ctypes.data, 1, 2048, 0)
    outs = [native._OutPlane(k.ctypes.data, n, 1) for k in keep[3:]]
    args.out_state, args.out_dendrite, args.out_adaptation = outs
    return args, (keep, params, rowptr, bounds)


def call(lib, args):
    rc = lib.ns_dendritic_step(ctypes.byref(args), None)
    return rc, lib.ns_last_error().decode()


def test_step_validation_messages(lib):
    args, keep = fake_step_args()
    args.params[3] = native._Vector(None, 1)
    assert call(lib, args) == (1, "six neuron parameter vectors are required")
    args, keep = fake_step_args()
    args.n_neurons = 0
    assert "N > 0" in call(lib, args)[1]
    for edges in (4096, 1022, 4):   # above the kernels' capacity, unaligned, too small
        args, keep = fake_step_args()
        args.plan.block_edges = edges
        assert "edges per block" in call(lib, args)[1]
    args, keep = fake_step_args()
    args.out_dendrite = native._OutPlane(args.state.data, 8, 1)
    assert "overlap" in call(lib, args)[1]
    args, keep = fake_step_args()
    args.matrix.format = 9
    assert "format" in call(lib, args)[1]
    args, keep = fake_step_args()
    args.matrix.format = native.WEIGHT_E4M3
    assert "global scale" in call(lib, args)[1]
    args, keep = fake_step_args()
    args.matrix.n_rows = 7
    assert "row count" in call(lib, args)[1]


def fake_band_plan(n, width=4, rows=4):
    tables = [np.zeros(native.BAND_WAVES * (-(-n // rows)) + 1, np.int32), np.zeros(4, np.int32),
              np.full(64, 0xFFFFFF, np.uint32), np.full(8 * 64, 0xFFFF, np.uint16),
              np.zeros(8 * 64, np.float32)]
    plan = native._BandPlan()
    plan.band_width, plan.n_bands = width, -(-n // width)
    plan.block_rows, plan.n_row_blocks = rows, -(-n // rows)
    plan.n_blocks, plan.n_groups, plan.block_steps, plan.n_slots = 0, 1, 8, 8 * 64
    plan.wave_blocks, plan.blocks, plan.rows, plan.col, plan.weight = (t.ctypes.data for t in tables)
    return plan, tables


def test_band_step_validation_messages(lib):
    """Rejections of ns_dendritic_step_bands, all before anything is launched."""
    def band_call(args, plan):
        rc = lib.ns_dendritic_step_bands(ctypes.byref(args), ctypes.byref(plan), None)
        return rc, lib.ns_last_error().decode()

    args, keep = fake_step_args(n=8, batch=6)
    plan, tables = fake_band_plan(8)
    assert "multiple of 4" in band_call(args, plan)[1]
    args, keep = fake_step_args(n=8, batch=16)
    assert "neuron-major" in band_call(args, plan)[1]
    # neuron-major [16,8] planes from here on
    args.state = native._Plane(args.state.data, 1, 16, 0.0)
    for bad, message in (({"band_width": 0}, "band width"), ({"n_bands": 3}, "do not cover"),
                         ({"block_rows": 0}, "block_rows"), ({"n_row_blocks": 1}, "do not cover"),
                         ({"block_steps": 5}, "register blocks"), ({"n_groups": 0}, "sentinel"),
                         ({"n_slots": 64}, "tail padding"), ({"rows": None}, "tables")):
        plan, tables = fake_band_plan(8)
        for field, value in bad.items():
            setattr(plan, field, value)
        rc, text = band_call(args, plan)
        assert rc != 0 and message in text, (bad, text)
    plan, tables = fake_band_plan(8)
    plan.col = tables[3].ctypes.data + 2          # lane runs need 16-byte alignment
    assert "misaligned" in band_call(args, plan)[1]
    plan, tables = fake_band_plan(8)
    args.matrix.format = native.WEIGHT_E4M3
    assert "global scale" in band_call(args, plan)[1]
    args, keep = fake_step_args(n=8, batch=0)
    assert band_call(args, plan) == (0, "")
    assert [lib.ns_band_max_block_rows(b) for b in (16, 32, 8, 4, 12)] == [2496, 2496] + [4095] * 3


def test_empty_batch_is_a_no_op(lib):
    args, keep = fake_step_args(batch=0)
    assert call(lib, args) == (0, "")


def test_encoder_validation_messages(lib):
    """ns_encode_weights rejects bad arguments before any launch."""
    assert lib.ns_encode_workspace_bytes() == 4096

    def call(**fields):
        base = dict(weight=None, n_edges=0, format=native.WEIGHT_E4M3, reserved=0, codes=None,
                    block_scales=None, global_scale=16, workspace=16)
        base.update(fields)
        args = native._EncodeArgs(**base)
        rc = lib.ns_encode_weights(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    rc, message = call(format=native.WEIGHT_F32)
    assert rc != 0 and "E4M3 or NVFP4" in message
    rc, message = call(global_scale=None)
    assert rc != 0 and "global_scale and workspace" in message
    rc, message = call(n_edges=10)
    assert rc != 0 and "weight and codes" in message
    rc, message = call(n_edges=10, weight=16, codes=16, format=native.WEIGHT_NVFP4)
    assert rc != 0 and "block_scales" in message
    rc, message = call(n_edges=10, weight=20, codes=16)
    assert rc != 0 and "16-byte aligned" in message
    rc, message = call(n_edges=10, weight=16, codes=18)
    assert rc != 0 and "4-byte aligned" in message
    rc, message = call(n_edges=-1)
    assert rc != 0 and "n_edges" in message
    rc, message = call(workspace=None)
    assert rc != 0 and "workspace" in message

    def no_alloc(**fields):
        base = dict(weight=None, n_edges=0, format=native.WEIGHT_E4M3, reserved=0, codes=None,
                    block_scales=None, global_scale=16, workspace=None)
        base.update(fields)
        args = native._EncodeArgs(**base)
        rc = lib.ns_encode_weights_no_alloc(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    # The same argument checks, before the device is touched, plus: no workspace.
    rc, message = no_alloc(workspace=16)
    assert rc != 0 and "takes no workspace" in message
    rc, message = no_alloc(format=native.WEIGHT_F32)
    assert rc != 0 and "E4M3 or NVFP4" in message
    rc, message = no_alloc(n_edges=1 << 40)
    assert rc != 0 and "n_edges" in message
    rc, message = no_alloc(n_edges=10, weight=16, codes=16, format=native.WEIGHT_NVFP4)
    assert rc != 0 and "block_scales" in message


def test_topology_builder_validation(lib):
    """ns_build_topology and its workspace query reject bad sizes before any launch."""
    assert lib.ns_topology_workspace_bytes(0, 10) == -1
    assert b"N must be" in lib.ns_last_error()
    assert lib.ns_topology_workspace_bytes(10, -1) == -1
    # The sort's scratch size comes from the device, so without a GPU the
    # query reports that instead of a size.
    small = lib.ns_topology_workspace_bytes(1000, 20_000)
    assert small > 0 or b"temporary storage" in lib.ns_last_error()

    def call(**fields):
        base = dict(n_neurons=10, n_candidates=0, out_rowptr=256, in_rowptr=256, n_edges=256,
                    workspace=256, workspace_bytes=1 << 30)
        base.update(fields)
        rc = lib.ns_build_topology(ctypes.byref(native._TopologyArgs(**base)), None)
        return rc, lib.ns_last_error().decode()

    rc, message = call(n_candidates=1 << 31)
    assert rc != 0 and "2^31 edges" in message
    rc, message = call(n_candidates=5)
    assert rc != 0 and "src, dst and weight" in message
    rc, message = call(n_candidates=5, src=256, dst=256, weight=256)
    assert rc != 0 and "every edge output" in message
    rc, message = call(workspace_bytes=16)
    assert rc != 0 and ("workspace" in message or "temporary storage" in message)


def test_backward_validation_messages(lib):
    """ns_dendritic_step_backward rejects bad arguments before any launch."""
    assert lib.ns_step_backward_workspace_floats(100, 3) == 600

    def call(**fields):
        args = native._StepGradArgs()
        args.n_neurons, args.batch = 10, 1
        for i in range(6):
            args.params[i] = native._Vector(256, 1)
        args.matrix = native._Csr(10, 0, 256, None, 256, native.WEIGHT_F32, None, None)
        for name, value in fields.items():
            setattr(args, name, value)
        rc = lib.ns_dendritic_step_backward(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    rc, message = call(n_neurons=0)
    assert rc != 0 and "N must be" in message
    rc, message = call(matrix=native._Csr(10, 0, 256, None, 256, native.WEIGHT_E4M3, None, None))
    assert rc != 0 and "float32 weights" in message
    params = (native._Vector * 6)(*[native._Vector(256, 1)] * 5, native._Vector(None, 0))
    rc, message = call(params=params)
    assert rc != 0 and "parameter" in message
    rc, message = call(batch=0)
    assert rc == 0
    rc, message = call()
    assert rc != 0 and "state, dendrite and adaptation" in message
    # complete host-memory arguments: the forward's current must not overlap the workspace
    buf = np.zeros(16 * 10, np.float32)
    base = buf.ctypes.data
    plane = lambda k: native._Plane(base + 40 * k, 1, 1, 0.0)          # noqa: E731
    out = lambda k: native._OutPlane(base + 40 * k, 1, 1)               # noqa: E731
    index = np.zeros(11, np.int32)
    rc, message = call(state=plane(0), dendrite=plane(1), adaptation=plane(2),
                       d_state=out(3), d_dendrite=out(4), d_adaptation=out(5),
                       out_rowptr=index.ctypes.data, dst=index.ctypes.data,
                       out_weight_index=index.ctypes.data, workspace=base + 40 * 6,
                       current=base + 40 * 7)
    assert rc != 0 and "current must not overlap the workspace" in message


def fake_event_args(n=8, batch=2):
    """Valid-looking host buffers for ns_dendritic_event; used only for calls
    that fail validation, so nothing is launched."""
    keep = [np.zeros(batch * n, np.float32) for _ in range(12)]
    params = [np.ones(n, np.float32) for _ in range(7)]
    rowptr = np.zeros(n + 1, np.int32)
    args = native._EventArgs()
    args.n_neurons, args.batch = n, batch
    args.state, args.dendrite, args.adaptation, args.emitted = (
        native._Plane(k.ctypes.data, n, 1, 0.0) for k in keep[:4])
    args.drive = native._Plane(None, 0, 0, 0.2)
    args.dendritic_drive = native._Plane(None, 0, 0, 0.1)
    for i in range(6):
        args.params[i] = native._Vector(params[i].ctypes.data, 1)
    args.theta = native._Vector(params[6].ctypes.data, 1)
    args.current, args.current_stride_b, args.current_stride_n = keep[4].ctypes.data, n, 1
    args.out_rowptr, args.n_edges = rowptr.ctypes.data, 0
    args.out_state, args.out_dendrite, args.out_adaptation, args.out_emitted = (
        native._OutPlane(k.ctypes.data, n, 1) for k in keep[5:9])
    args.delta = keep[9].ctypes.data
    return args, (keep, params, rowptr)


def test_event_validation_messages(lib):
    """ns_dendritic_event's rejections, for the two-launch and the one-launch
    (pending buffers) tick, all before any launch."""
    def call(args):
        rc = lib.ns_dendritic_event(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    args, keep = fake_event_args()
    args.delta = None
    assert "delta workspace" in call(args)[1]
    args, keep = fake_event_args()
    args.pending_in = keep[0][10].ctypes.data
    assert "go together" in call(args)[1]
    args, keep = fake_event_args()
    args.out_dendrite = native._OutPlane(args.state.data, 8, 1)
    assert "output planes must not overlap inputs" in call(args)[1]
    args, keep = fake_event_args()
    args.delta = args.current
    assert "workspaces must not overlap inputs" in call(args)[1]
    for pending_in, pending_out, message in (
            (4, 10, "workspaces must not overlap inputs"),          # the current
            (10, 5, "must not overlap outputs"),                    # out_state
            (10, 10, "must not overlap outputs or each other")):
        args, keep = fake_event_args()
        buffers = keep[0]
        args.delta = None
        args.pending_in = buffers[pending_in].ctypes.data
        args.pending_out = buffers[pending_out].ctypes.data
        rc, text = call(args)
        assert rc != 0 and message in text, text
    for strides in ((0, 1), (1, 1), (4, 1), (1, 0)):         # zero or interleaved strides
        args, keep = fake_event_args()
        args.current_stride_b, args.current_stride_n = strides
        rc, text = call(args)
        assert rc != 0 and "must not overlap itself" in text, (strides, text)
    args, keep = fake_event_args(batch=0)
    assert call(args) == (0, "")


def fake_panel_plan(n, batch):
    """A structurally valid one-panel plan over host arrays (validation only)."""
    tables = [np.zeros(4, np.int32), np.zeros(17, np.int32), np.zeros(4, np.int32),
              np.zeros(1, np.uint16), np.zeros(4, np.uint32), np.zeros(2048, np.uint16),
              np.zeros(2048, np.float32), np.zeros(2 * n * batch, np.float32)]
    plan = native._PanelPlan()
    plan.panel_width, plan.n_panels, plan.n_tiles, plan.n_groups = max(4, -(-n // 4) * 4), 1, 1, 0
    plan.waves, plan.flags, plan.n_slots, plan.n_step_words = 16, 0, 2048, 4
    (plan.tiles, plan.wave_groups, plan.groups, plan.rows, plan.last_steps, plan.col,
     plan.weight, plan.partials) = (t.ctypes.data for t in tables)
    return plan, tables


def test_panel_workspace_must_not_overlap_any_operand(lib):
    """Tiles write the partials workspace while other workgroups still read the
    state and drives: an overlap with any input or output is rejected."""
    n, batch = 8, 1
    for field in ("state", "dendrite", "adaptation", "drive", "dendritic_drive",
                  "out_state", "out_current"):
        args, keep = fake_step_args(n=n, batch=batch)
        plan, tables = fake_panel_plan(n, batch)
        args.panels = ctypes.addressof(plan)
        workspace = tables[-1].ctypes.data
        if field.startswith("out_"):
            setattr(args, field, native._OutPlane(workspace, n, 1))
        else:
            setattr(args, field, native._Plane(workspace, n, 1, 0.0))
        rc, text = call(lib, args)
        kind = "output" if field.startswith("out_") else "input"
        assert rc != 0 and f"partials workspace overlaps an {kind}" in text, (field, text)


def fake_two_panel_plan(n, batch):
    """Two panels of one row range each, over host arrays (validation only)."""
    plan, tables = fake_panel_plan(n, batch)
    width = max(4, -(-n // 8) * 4)
    partials = np.zeros(2 * 2 * n * batch, np.float32)
    ranges, counters = np.zeros(2, np.int32), np.zeros(1, np.uint32)
    tables += [partials, ranges, counters]
    plan.panel_width, plan.n_panels, plan.n_tiles, plan.n_ranges = width, 2, 2, 1
    plan.partials, plan.tile_ranges = partials.ctypes.data, ranges.ctypes.data
    plan.range_counters = counters.ctypes.data
    return plan, tables


def test_panel_range_counters_are_checked(lib):
    """With several panels the tick kernel's last tile of each row range
    combines the panels: the ranges and their counters are required, the tiles
    must be one per panel and range, and the counters may overlap no operand
    nor the partials workspace."""
    n, batch = 16, 1
    args, keep = fake_step_args(n=n, batch=batch)
    plan, tables = fake_two_panel_plan(n, batch)
    args.panels = ctypes.addressof(plan)
    plan.range_counters = None
    rc, text = call(lib, args)
    assert rc != 0 and "range counters are required" in text, text
    plan.range_counters = tables[-1].ctypes.data
    plan.n_ranges = 2
    rc, text = call(lib, args)
    assert rc != 0 and "one per panel for each of 2 row ranges" in text, text
    plan.n_ranges = 1
    plan.range_counters = plan.partials
    rc, text = call(lib, args)
    assert rc != 0 and "range counters overlap the partials" in text, text
    plan.range_counters = args.state.data
    rc, text = call(lib, args)
    assert rc != 0 and "range counters overlap an input" in text, text
    plan.range_counters = args.out_state.data
    rc, text = call(lib, args)
    assert rc != 0 and "range counters overlap an output" in text, text
    plan.flags = 8
    rc, text = call(lib, args)
    assert rc != 0 and "unknown panel plan flags 8" in text, text
    plan.flags = native.PANEL_INDEXED
    args.matrix.format = native.WEIGHT_F16
    rc, text = call(lib, args)
    assert rc != 0 and "an indexed panel plan reads float32 CSR weights" in text, text


def test_slot_gather_validation(lib):
    """Rejected before any launch (host pointers only)."""
    perm = np.zeros(8, np.int32)
    out = np.zeros(8, np.float32)
    weight = np.zeros(4, np.float32)

    def gather(n_slots=8, n_edges=4, fmt=native.WEIGHT_F32, pairs=0, w=weight, scales=None,
               slots=out, slot_scales=None, perm_ptr=None):
        rc = lib.ns_gather_slot_weights(perm_ptr or perm.ctypes.data, n_slots, n_edges, fmt, pairs,
                                        w.ctypes.data if w is not None else None,
                                        scales, slots.ctypes.data if slots is not None else None,
                                        slot_scales, None)
        return rc, lib.ns_last_error().decode()

    assert gather(n_slots=7) == (1, "n_slots must be even and in [0, 2^32)")
    assert gather(fmt=7) == (1, "unknown weight format 7")
    assert gather(pairs=1) == (1, "the pair layout applies to NVFP4 only")
    assert gather(slots=None) == (1, "perm and slots are required")
    assert gather(w=None) == (1, "weight is required")
    assert gather(fmt=native.WEIGHT_NVFP4, pairs=1, w=np.zeros(2, np.uint8)) == (
        1, "NVFP4 weights require block scales")
    scales = np.zeros(1, np.uint8)
    assert gather(fmt=native.WEIGHT_NVFP4, w=np.zeros(2, np.uint8), scales=scales.ctypes.data) == (
        1, "NVFP4 slots without pairs need slot_scales")
    assert gather(perm_ptr=perm.ctypes.data + 4) == (1, "perm must be 8-byte aligned")
    assert gather(n_slots=0) == (0, "")


def test_event_flags_are_checked(lib):
    def call(args):
        rc = lib.ns_dendritic_event(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    args, keep = fake_event_args()
    args.flags = 2
    assert call(args) == (1, "unknown event flags 2")
    args.flags = native.EVENT_ADVANCE_ONLY
    args.pending_in, args.pending_out = keep[0][10].ctypes.data, keep[0][11].ctypes.data
    assert call(args) == (1, "the advance-only tick scatters nothing: pending_out must be NULL")
    # The fused advance-only tick: pending_in folds into the current, deltas go to `delta`.
    args.pending_out = None
    args.delta = None
    assert call(args) == (1, "a delta workspace is required")
    args.delta = args.pending_in
    assert "must not overlap outputs or each other" in call(args)[1]


def test_event_activity_counters_are_checked(lib):
    def call(args):
        rc = lib.ns_dendritic_event(ctypes.byref(args), None)
        return rc, lib.ns_last_error().decode()

    counters = np.zeros(native.EVENT_ACTIVITY_SLOTS * native.EVENT_ACTIVITY_STRIDE, np.int64)
    args, keep = fake_event_args()
    args.activity = counters.ctypes.data
    assert call(args) == (1, "activity counts need the one-launch tick (pending_in)")
    args, keep = fake_event_args()
    args.delta = None
    args.pending_in, args.pending_out = keep[0][10].ctypes.data, keep[0][11].ctypes.data
    args.activity = keep[0][11].ctypes.data          # overlaps pending_out
    assert "must not overlap outputs or each other" in call(args)[1]
    args.activity = args.current                     # overlaps an input
    assert "must not overlap" in call(args)[1]


def test_accumulated_spmm_output_must_not_overlap_itself(lib):
    n, batch = 8, 2
    rowptr = np.zeros(n + 1, np.int32)
    bounds = np.array([0, 0, n, 0], np.int32)
    source = np.zeros((batch, n), np.float32)
    out = np.zeros(1, np.float32)
    args = native._SpmmArgs()
    args.n_neurons, args.batch = n, batch
    args.source = native._Plane(source.ctypes.data, n, 1, 0.0)
    args.matrix = native._Csr(n, 0, rowptr.ctypes.data, None, None, native.WEIGHT_F32, None, None)
    args.plan = native._RowPlan(bounds.ctypes.data, 1, lib.ns_block_edges(batch), 0)
    args.out = native._OutPlane(out.ctypes.data, 0, 0)
    args.accumulate = 1
    rc = lib.ns_csr_spmm(ctypes.byref(args), None)
    assert rc == 1 and "must not overlap itself" in lib.ns_last_error().decode()


def test_packed_argument_words_land_in_their_fields():
    """The prepared launches write per-tick words with struct.pack_into at fixed
    offsets; reading the ctypes fields back pins those layouts."""
    import neurosim_gpu.native as nv

    def planes(count, start):
        words = []
        for k in range(count):
            words += [start + 100 * k, -(k + 1), k + 7, float(k) + 0.5]
        return words

    step = nv._StepArgs()
    nv._PLANES5.pack_into(step, nv._STEP_IN, *planes(5, 1000))
    nv._OUTS4.pack_into(step, nv._STEP_OUT, *(v for k in range(4) for v in (2000 + k, 1, k + 3)))
    for k, name in enumerate(nv._IN_NAMES):
        plane = getattr(step, name)
        assert (plane.data, plane.stride_b, plane.stride_n, plane.scalar) == \
            (1000 + 100 * k, -(k + 1), k + 7, k + 0.5)
    for k, name in enumerate(("out_state", "out_dendrite", "out_adaptation", "out_current")):
        plane = getattr(step, name)
        assert (plane.data, plane.stride_b, plane.stride_n) == (2000 + k, 1, k + 3)

    event = nv._EventArgs()
    nv._PLANES5.pack_into(event, nv._EVENT_IN, *planes(5, 3000))
    nv._CURRENT_EMITTED.pack_into(event, nv._EVENT_CURRENT, 4000, 2, 3, 4100, 5, 6, 1.5)
    nv._EVENT_TAIL.pack_into(event, nv._EVENT_TAIL_AT, 11, 12, 13, 14, 1, 0, 15)
    nv._OUTS4.pack_into(event, nv._EVENT_OUT, *(v for k in range(4) for v in (5000 + k, 1, 2)))
    assert event.state.data == 3000 and event.dendritic_drive.scalar == 4.5
    assert (event.current, event.current_stride_b, event.current_stride_n) == (4000, 2, 3)
    assert (event.emitted.data, event.emitted.stride_n, event.emitted.scalar) == (4100, 6, 1.5)
    assert (event.delta, event.pending_in, event.pending_out, event.out_weight) == (11, 12, 13, 14)
    assert (event.flags, event.activity) == (1, 15)
    assert event.out_emitted.data == 5003

    grad = nv._StepGradArgs()
    nv._PLANES5.pack_into(grad, nv._GRAD_IN, *planes(5, 6000))
    nv._PLANES3.pack_into(grad, nv._GRAD_UP, *planes(3, 7000))
    nv._OUTS5.pack_into(grad, nv._GRAD_OUT, *(v for k in range(5) for v in (8000 + k, 1, 9)))
    nv._POINTERS11.pack_into(grad, nv._GRAD_POINTERS, *range(9000, 9011))
    assert grad.adaptation.data == 6200 and grad.grad_adaptation.data == 7200
    assert grad.d_dendritic_drive.data == 8004
    assert grad.d_weight == 9000 and list(grad.d_params) == list(range(9001, 9007))
    assert (grad.workspace, grad.current, grad.out_weight, grad.transposed_panels) == \
        (9007, 9008, 9009, 9010)


def test_row_block_size_follows_the_graph():
    """Small graphs get smaller row blocks (at least two per compute unit where
    the floor allows); large ones keep the kernels' capacity."""
    cap = {b: native.load_library().ns_block_edges(b) for b in (1, 2, 4, 8, 16)}
    assert native.row_block_edges(1, 65_401, 256) == 1024          # floor at batch 1-2
    assert native.row_block_edges(2, 65_401, 256) == 1024
    assert native.row_block_edges(1, 999_828, 256) == 1024
    assert native.row_block_edges(1, 1_999_924, 256) == cap[1]      # 2048
    assert native.row_block_edges(8, 65_401, 256) == 256            # floor from batch 4
    assert native.row_block_edges(16, 16_273, 256) == 256
    assert native.row_block_edges(8, 399_806, 256) == 512
    assert native.row_block_edges(8, 999_828, 256) == cap[8]        # 1024
    assert native.row_block_edges(16, 99_994_973, 256) == cap[16]
    for b in cap:
        for m in (0, 1, 10**3, 10**5, 10**7):
            edges = native.row_block_edges(b, m, 256)
            assert 8 <= edges <= cap[b] and edges % 4 == 0
