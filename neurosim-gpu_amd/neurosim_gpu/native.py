"""Loader and tensor-level shim for the gfx950 C-ABI library libneurosim_hip.so.

``load_native_extension()`` returns an object with the reference extension's
hot-path ops and signatures (csrc/bindings.cpp:3-12,137-143):

    dendritic_step(state, dendrite, adaptation, params, rowptr, source, weight,
                   input, input_scalar, dendritic_input, dendritic_scalar, width,
                   block_scales=None, global_scale=None) -> [state', dendrite', adaptation']
    dendritic_event(state, dendrite, adaptation, params, current, emitted, theta,
                    out_rowptr, dst, weight_index, weight, input, input_scalar,
                    dendritic_input, dendritic_scalar)
                    -> [state', dendrite', adaptation', emitted']   (current updated in place)

plus ``csr_spmm(source, rowptr, col, weight, block_scales=None, global_scale=None)``.
Validation failures raise RuntimeError before anything is launched, like the
reference's TORCH_CHECKs.  Outputs are fresh [B,N] tensors stored neuron-major
(strides (1, B)): the kernels gather s[col, 0:B] as one contiguous run per
edge.  ``width`` is accepted for compatibility (8, 16 or 32) and does not
change the kernels, which size their lane groups per row block.

The library is never built or replaced implicitly: a missing library raises.
"""

from __future__ import annotations

import ctypes
import os
import struct
import threading
import weakref
from collections import OrderedDict
from functools import lru_cache
from operator import is_
from pathlib import Path

import numpy as np
import torch

_LIB_NAME = "libneurosim_hip.so"
ABI_VERSION = 19

WEIGHT_F32, WEIGHT_F16, WEIGHT_E4M3, WEIGHT_NVFP4 = 0, 1, 2, 3
_PLAN_CACHE = 64   # row plans kept per extension (one per live topology and batch width)

_c_i64 = ctypes.c_int64
_c_ptr = ctypes.c_void_p


class _Plane(ctypes.Structure):
    _fields_ = [("data", _c_ptr), ("stride_b", _c_i64), ("stride_n", _c_i64),
                ("scalar", ctypes.c_float)]


class _OutPlane(ctypes.Structure):
    _fields_ = [("data", _c_ptr), ("stride_b", _c_i64), ("stride_n", _c_i64)]


class _Vector(ctypes.Structure):
    _fields_ = [("data", _c_ptr), ("stride", _c_i64)]


class _Csr(ctypes.Structure):
    _fields_ = [("n_rows", _c_i64), ("n_edges", _c_i64), ("rowptr", _c_ptr), ("col", _c_ptr),
                ("weight", _c_ptr), ("format", ctypes.c_int32), ("block_scales", _c_ptr),
                ("global_scale", _c_ptr)]


class _RowPlan(ctypes.Structure):
    _fields_ = [("bounds", _c_ptr), ("n_blocks", _c_i64), ("block_edges", ctypes.c_int32),
                ("reserved", ctypes.c_int32)]


class _PanelPlan(ctypes.Structure):
    _fields_ = [("panel_width", ctypes.c_int32), ("n_panels", ctypes.c_int32),
                ("n_tiles", ctypes.c_int32), ("n_groups", ctypes.c_int32),
                ("waves", ctypes.c_int32), ("flags", ctypes.c_int32),
                ("n_ranges", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("n_slots", _c_i64), ("n_step_words", _c_i64), ("tiles", _c_ptr),
                ("tile_ranges", _c_ptr), ("wave_groups", _c_ptr),
                ("groups", _c_ptr), ("rows", _c_ptr), ("last_steps", _c_ptr), ("col", _c_ptr),
                ("weight", _c_ptr), ("slot_scales", _c_ptr), ("partials", _c_ptr),
                ("range_counters", _c_ptr)]


class _BandPlan(ctypes.Structure):
    _fields_ = [("band_width", ctypes.c_int32), ("n_bands", ctypes.c_int32),
                ("block_rows", ctypes.c_int32), ("n_row_blocks", ctypes.c_int32),
                ("n_blocks", ctypes.c_int32), ("n_groups", ctypes.c_int32),
                ("block_steps", ctypes.c_int32), ("reserved", ctypes.c_int32), ("n_slots", _c_i64),
                ("wave_blocks", _c_ptr), ("blocks", _c_ptr), ("rows", _c_ptr), ("col", _c_ptr),
                ("weight", _c_ptr), ("slot_scales", _c_ptr)]


class _StepArgs(ctypes.Structure):
    _fields_ = [("n_neurons", _c_i64), ("batch", _c_i64),
                ("state", _Plane), ("dendrite", _Plane), ("adaptation", _Plane),
                ("drive", _Plane), ("dendritic_drive", _Plane),
                ("params", _Vector * 6), ("matrix", _Csr), ("plan", _RowPlan),
                ("panels", _c_ptr),
                ("out_state", _OutPlane), ("out_dendrite", _OutPlane),
                ("out_adaptation", _OutPlane), ("out_current", _OutPlane)]


class _EventArgs(ctypes.Structure):
    _fields_ = [("n_neurons", _c_i64), ("batch", _c_i64),
                ("state", _Plane), ("dendrite", _Plane), ("adaptation", _Plane),
                ("drive", _Plane), ("dendritic_drive", _Plane),
                ("params", _Vector * 6),
                ("current", _c_ptr), ("current_stride_b", _c_i64), ("current_stride_n", _c_i64),
                ("emitted", _Plane), ("theta", _Vector),
                ("out_rowptr", _c_ptr), ("dst", _c_ptr), ("weight_index", _c_ptr),
                ("weight", _c_ptr), ("n_edges", _c_i64),
                ("out_state", _OutPlane), ("out_dendrite", _OutPlane),
                ("out_adaptation", _OutPlane), ("out_emitted", _OutPlane),
                ("delta", _c_ptr), ("pending_in", _c_ptr), ("pending_out", _c_ptr),
                ("out_weight", _c_ptr), ("flags", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("activity", _c_ptr)]

EVENT_ADVANCE_ONLY = 1   # NS_EVENT_ADVANCE_ONLY
EVENT_ACTIVITY_SLOTS = 32   # NS_EVENT_ACTIVITY_SLOTS
EVENT_ACTIVITY_STRIDE = 16  # NS_EVENT_ACTIVITY_STRIDE


class _SpmmArgs(ctypes.Structure):
    _fields_ = [("n_neurons", _c_i64), ("batch", _c_i64), ("source", _Plane),
                ("matrix", _Csr), ("plan", _RowPlan), ("out", _OutPlane),
                ("accumulate", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("panels", _c_ptr)]


class _StepGradArgs(ctypes.Structure):
    _fields_ = [("n_neurons", _c_i64), ("batch", _c_i64),
                ("state", _Plane), ("dendrite", _Plane), ("adaptation", _Plane),
                ("drive", _Plane), ("dendritic_drive", _Plane),
                ("params", _Vector * 6), ("matrix", _Csr), ("plan", _RowPlan),
                ("out_rowptr", _c_ptr), ("dst", _c_ptr), ("out_weight_index", _c_ptr),
                ("grad_state", _Plane), ("grad_dendrite", _Plane), ("grad_adaptation", _Plane),
                ("d_state", _OutPlane), ("d_dendrite", _OutPlane), ("d_adaptation", _OutPlane),
                ("d_drive", _OutPlane), ("d_dendritic_drive", _OutPlane),
                ("d_weight", _c_ptr), ("d_params", _c_ptr * 6), ("workspace", _c_ptr),
                ("current", _c_ptr), ("out_weight", _c_ptr), ("transposed_panels", _c_ptr)]


class _EncodeArgs(ctypes.Structure):
    _fields_ = [("weight", _c_ptr), ("n_edges", _c_i64), ("format", ctypes.c_int32),
                ("reserved", ctypes.c_int32), ("codes", _c_ptr), ("block_scales", _c_ptr),
                ("global_scale", _c_ptr), ("workspace", _c_ptr)]


class _TopologyArgs(ctypes.Structure):
    _fields_ = [("n_neurons", _c_i64), ("n_candidates", _c_i64), ("src", _c_ptr),
                ("dst", _c_ptr), ("weight", _c_ptr), ("out_src", _c_ptr), ("out_dst", _c_ptr),
                ("out_weight", _c_ptr), ("out_rowptr", _c_ptr), ("in_rowptr", _c_ptr),
                ("in_col", _c_ptr), ("in_weight", _c_ptr), ("out_weight_index", _c_ptr),
                ("n_edges", _c_ptr), ("workspace", _c_ptr), ("workspace_bytes", _c_i64)]


def library_path() -> Path:
    override = os.environ.get("NEUROSIM_HIP_LIB")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / "_lib" / _LIB_NAME


@lru_cache(maxsize=1)
def load_library() -> ctypes.CDLL:
    """Open the built library once; raise if it is missing or of another ABI."""
    path = library_path()
    if not path.exists():
        raise RuntimeError(
            f"native library {path} is missing; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` or "
            "`make -C neurosim-gpu_amd/csrc`")
    lib = ctypes.CDLL(str(path))
    lib.ns_abi_version.restype = ctypes.c_int
    lib.ns_last_error.restype = ctypes.c_char_p
    lib.ns_block_edges.restype = ctypes.c_int32
    lib.ns_block_edges.argtypes = [_c_i64]
    lib.ns_plan_row_blocks.restype = ctypes.c_int
    lib.ns_plan_row_blocks.argtypes = [_c_ptr, _c_i64, ctypes.c_int32, _c_ptr, _c_i64,
                                       ctypes.POINTER(_c_i64)]
    lib.ns_panel_geometry.restype = ctypes.c_int
    lib.ns_panel_geometry.argtypes = [_c_i64, ctypes.POINTER(ctypes.c_int32),
                                      ctypes.POINTER(ctypes.c_int32)]
    lib.ns_plan_panels.restype = ctypes.c_int
    lib.ns_plan_panels.argtypes = [_c_ptr, _c_ptr, _c_i64, ctypes.c_int32, ctypes.c_int32,
                                   ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                   ctypes.POINTER(_PanelPlan), ctypes.POINTER(_c_i64)] + [_c_ptr] * 8
    lib.ns_gather_slot_weights.restype = ctypes.c_int
    lib.ns_gather_slot_weights.argtypes = [_c_ptr, _c_i64, _c_i64, ctypes.c_int32, ctypes.c_int32,
                                           _c_ptr, _c_ptr, _c_ptr, _c_ptr, _c_ptr]
    lib.ns_plan_bands.restype = ctypes.c_int
    lib.ns_plan_bands.argtypes = [_c_ptr, _c_ptr, _c_i64, ctypes.c_int32, ctypes.c_int32,
                                  ctypes.c_int32, ctypes.POINTER(_BandPlan)] + [_c_ptr] * 5
    lib.ns_band_max_block_rows.restype = ctypes.c_int32
    lib.ns_band_max_block_rows.argtypes = [_c_i64]
    lib.ns_dendritic_step_bands.restype = ctypes.c_int
    lib.ns_dendritic_step_bands.argtypes = [ctypes.POINTER(_StepArgs), ctypes.POINTER(_BandPlan),
                                            _c_ptr]
    lib.ns_encode_workspace_bytes.restype = _c_i64
    lib.ns_encode_workspace_bytes.argtypes = []
    lib.ns_step_backward_workspace_floats.restype = _c_i64
    lib.ns_step_backward_workspace_floats.argtypes = [_c_i64, _c_i64]
    lib.ns_topology_workspace_bytes.restype = _c_i64
    lib.ns_topology_workspace_bytes.argtypes = [_c_i64, _c_i64]
    for name, kind in (("ns_dendritic_step", _StepArgs), ("ns_dendritic_event", _EventArgs),
                       ("ns_csr_spmm", _SpmmArgs), ("ns_encode_weights", _EncodeArgs),
                       ("ns_encode_weights_no_alloc", _EncodeArgs),
                       ("ns_build_topology", _TopologyArgs),
                       ("ns_dendritic_step_backward", _StepGradArgs)):
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = [ctypes.POINTER(kind), _c_ptr]
    version = lib.ns_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    return lib


def _raise_on(code: int, lib: ctypes.CDLL) -> None:
    if code != 0:
        message = lib.ns_last_error().decode("utf-8", "replace")
        raise RuntimeError(message or f"native call failed with code {code}")


def encode_weights(weight: torch.Tensor, precision: str
                   ) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
    """Device encoding of float32 CSR weights (ns_encode_weights).

    Same contract as precision.encode_sparse_weights (reference precision.py:76-90):
    returns (packed codes uint8, block scales uint8 or None, float32 global
    scale, 0-d) on the weights' device, launched on the current stream.
    """
    if weight.ndim != 1 or weight.dtype != torch.float32:
        raise ValueError("encoding requires a vector of FP32 CSR weights")
    if precision not in ("fp8", "nvfp4"):
        raise ValueError("compressed CSR encoding requires fp8 or nvfp4")
    if weight.device.type != "cuda":
        raise ValueError("the device encoder needs the weights on a GPU")
    lib = load_library()
    m = weight.numel()
    source = weight.detach()
    if m and (not source.is_contiguous() or source.data_ptr() % 16):
        source = source.contiguous().clone()
    device = weight.device
    nvfp4 = precision == "nvfp4"
    payload = (m + 1) // 2 if nvfp4 else m
    codes = torch.empty(max(payload, 1), dtype=torch.uint8, device=device)
    scales = torch.empty((m + 15) // 16, dtype=torch.uint8, device=device) if nvfp4 else None
    scale = torch.empty(1, dtype=torch.float32, device=device)
    workspace = torch.empty(int(lib.ns_encode_workspace_bytes()) // 4, dtype=torch.int32,
                            device=device)
    args = _EncodeArgs(source.data_ptr() if m else None, m,
                       WEIGHT_NVFP4 if nvfp4 else WEIGHT_E4M3, 0, codes.data_ptr(),
                       scales.data_ptr() if scales is not None and scales.numel() else None,
                       scale.data_ptr(), workspace.data_ptr())
    stream = torch.cuda.current_stream(device).cuda_stream
    _raise_on(lib.ns_encode_weights(ctypes.byref(args), stream), lib)
    return codes[:payload], scales, scale.view(())


def build_topology(n_neurons: int, src: torch.Tensor, dst: torch.Tensor,
                   weight: torch.Tensor) -> dict:
    """Coalesced graph and both CSR views built on the device (ns_build_topology).

    ``src``/``dst`` are int64 and ``weight`` float32 device vectors of candidate
    edges whose indices the caller has checked to lie in [0, n_neurons).
    Returns the SparseTopology fields, bitwise equal to the CPU build
    (reference topology.py:32-115).  Reads the edge count back (one sync).
    """
    lib = load_library()
    device = weight.device
    m = int(weight.numel())
    src = src.to(torch.int64).contiguous()
    dst = dst.to(torch.int64).contiguous()
    weight = weight.contiguous()
    size = int(lib.ns_topology_workspace_bytes(int(n_neurons), m))
    if size < 0:
        _raise_on(1, lib)
    workspace = torch.empty(size + 256, dtype=torch.uint8, device=device)
    base = workspace.data_ptr()
    aligned = base + (-base) % 256
    cap = max(m, 1)
    out = {name: torch.empty(cap, dtype=dtype, device=device) for name, dtype in (
        ("src", torch.int32), ("dst", torch.int32), ("weight", torch.float32),
        ("in_col", torch.int32), ("in_weight", torch.float32), ("out_weight_index", torch.int32))}
    out["out_rowptr"] = torch.empty(n_neurons + 1, dtype=torch.int32, device=device)
    out["in_rowptr"] = torch.empty(n_neurons + 1, dtype=torch.int32, device=device)
    count = torch.empty(1, dtype=torch.int64, device=device)
    ptr = (lambda t: t.data_ptr() if m else None)
    args = _TopologyArgs(int(n_neurons), m, ptr(src), ptr(dst), ptr(weight), out["src"].data_ptr(),
                         out["dst"].data_ptr(), out["weight"].data_ptr(),
                         out["out_rowptr"].data_ptr(), out["in_rowptr"].data_ptr(),
                         out["in_col"].data_ptr(), out["in_weight"].data_ptr(),
                         out["out_weight_index"].data_ptr(), count.data_ptr(), aligned, size)
    stream = torch.cuda.current_stream(device).cuda_stream
    _raise_on(lib.ns_build_topology(ctypes.byref(args), stream), lib)
    edges = int(count.item())
    for name in ("src", "dst", "weight", "in_col", "in_weight", "out_weight_index"):
        out[name] = out[name][:edges]
    return out


def row_block_edges(batch: int, n_edges: int, units: int) -> int:
    """Edges per row block: the kernels' capacity for ``batch``, halved while the
    graph would give fewer than two blocks per compute unit, down to 1024 edges at
    batch 1 or 2 (one full pass of a workgroup's lanes) and 256 from batch 4.
    Graph-replayed ticks measured with each size (rows kernel, µs): N=4096,
    M=65k: B=1 5.00 at 2048 edges, 4.37 at 1024; B=8 8.85 at 1024, 5.89 at 256;
    N=1024, M=16k, B=16: 16.6 at 1024, 8.4 at 256; N=20k, M=400k, B=8: 9.0 at
    1024, 8.3 at 512; N=50k, M=1M: B=1 7.97 at 2048, 7.88 at 1024, B=8 13.5 at
    1024, 15.2 at 512; N=166k, M=2M, B=1: 13.4 at 2048, 13.7 at 1024."""
    edges = int(load_library().ns_block_edges(int(batch)))
    floor = 1024 if batch <= 2 else 256
    while edges > floor and n_edges < 2 * units * edges:
        edges //= 2
    return edges


def plan_row_blocks(rowptr: torch.Tensor, batch: int, device: torch.device) -> tuple[torch.Tensor, int, int]:
    """Row blocks for the tick kernels, built on the host and placed on ``device``.

    Returns (bounds int32 device tensor [2*(blocks+1)], blocks, edges per block:
    ``row_block_edges`` for the graph, at most ``ns_block_edges(batch)``).
    Reads rowptr once on the host (a synchronisation), so call it at set-up.
    """
    lib = load_library()
    host = np.ascontiguousarray(rowptr.detach().to("cpu", torch.int32).numpy())
    n = host.size - 1
    device = torch.device(device)
    units = (torch.cuda.get_device_properties(device).multi_processor_count
             if device.type == "cuda" else 256)
    block_edges = row_block_edges(batch, int(host[-1]) if n >= 0 else 0, units)
    count = _c_i64(0)
    _raise_on(lib.ns_plan_row_blocks(host.ctypes.data, n, block_edges, None, 0,
                                     ctypes.byref(count)), lib)
    bounds = np.empty(2 * (count.value + 1), dtype=np.int32)
    _raise_on(lib.ns_plan_row_blocks(host.ctypes.data, n, block_edges, bounds.ctypes.data,
                                     bounds.size, ctypes.byref(count)), lib)
    return torch.from_numpy(bounds).to(device), int(count.value), block_edges


def _check_float(value: torch.Tensor, state: torch.Tensor, what: str) -> None:
    if not isinstance(value, torch.Tensor):
        raise RuntimeError(f"{what} must be a tensor")
    if value.device != state.device:
        raise RuntimeError("all tensors must be on the state's CUDA device")
    if value.dtype != torch.float32:
        raise RuntimeError("all values must be float32")


def _plane(value: torch.Tensor, state: torch.Tensor, what: str) -> _Plane:
    _check_float(value, state, what)
    if value.shape != state.shape:
        raise RuntimeError("state/current/drive shape mismatch")
    return _Plane(value.data_ptr(), value.stride(0), value.stride(1), 0.0)


def _drive(value: torch.Tensor | None, scalar: float, state: torch.Tensor) -> _Plane:
    if value is None:
        return _Plane(None, 0, 0, float(scalar))
    return _plane(value, state, "drive")


def _out(value: torch.Tensor) -> _OutPlane:
    return _OutPlane(value.data_ptr(), value.stride(0), value.stride(1))


def _index(value: torch.Tensor, state: torch.Tensor) -> None:
    if (not isinstance(value, torch.Tensor) or value.device != state.device
            or value.dtype != torch.int32 or not value.is_contiguous() or value.dim() != 1):
        raise RuntimeError("indices must be contiguous int32 vectors on the state device")


def _check_state(state: torch.Tensor) -> None:
    if (not isinstance(state, torch.Tensor) or state.device.type != "cuda"
            or state.dtype != torch.float32):
        raise RuntimeError("state must be CUDA float32")
    if state.dim() != 2 or state.size(1) <= 0:
        raise RuntimeError("state must be [B,N], N > 0")


def _params(values, state: torch.Tensor):
    if not isinstance(values, (list, tuple)) or len(values) != 6:
        raise RuntimeError("six neuron parameter vectors are required")
    vectors = (_Vector * 6)()
    for i, value in enumerate(values):
        _check_float(value, state, "parameter")
        if value.dim() != 1 or value.numel() != state.size(1):
            raise RuntimeError("parameters must have one value per neuron")
        vectors[i] = _Vector(value.data_ptr(), value.stride(0))
    return vectors


def _new_outputs(count: int, batch: int, n: int, device) -> tuple:
    """``count`` fresh neuron-major [batch, n] planes from one allocation, and
    that allocation's address.  At batch 1 a neuron-major plane is a row, so the
    planes are the rows of a [count, 1, n] block (no transposed view needed)."""
    if batch == 1:
        storage = torch.empty((count, 1, n), dtype=torch.float32, device=device)
        return storage.unbind(0), storage.data_ptr()
    storage = torch.empty((count, n, batch), dtype=torch.float32, device=device)
    return storage.transpose(1, 2).unbind(0), storage.data_ptr()


def _neuron_major(plane: torch.Tensor) -> bool:
    """Element (b, n) of a [B,N] plane at offset n * B + b (at B=1 any row)."""
    batch = plane.size(0)
    return plane.stride(1) == batch and (batch == 1 or plane.stride(0) == 1)


def new_planes(count: int, batch: int, n: int, like: torch.Tensor) -> list[torch.Tensor]:
    """``count`` fresh [B,N] planes stored neuron-major in one allocation."""
    return list(_new_outputs(count, batch, n, like.device)[0])


def panel_geometry(batch: int) -> tuple[int, int]:
    """(largest panel width, wavefronts per workgroup) of the panel kernel."""
    lib = load_library()
    width, waves = ctypes.c_int32(), ctypes.c_int32()
    _raise_on(lib.ns_panel_geometry(int(batch), ctypes.byref(width), ctypes.byref(waves)), lib)
    return width.value, waves.value


LANE_TARGET = 24   # at most this many edges per lane before a row gets more lanes


PANEL_PAIRS = 1   # NS_PANEL_PAIRS
PANEL_COMBINE_LAUNCH = 2   # NS_PANEL_COMBINE_LAUNCH
PANEL_INDEXED = 4   # NS_PANEL_INDEXED
# Largest row range the tick kernel's last tile finishes by itself when the
# caller leaves the choice to the layout.  The last tile updates its whole
# range on one compute unit, and in every measurement so far the combine
# kernel, spread over the chip, was faster: N=166,000, M=25M, B=1 (3255-row
# ranges) 35.6 against 33.3 us per tick; N=50,000, M=1M (390-row ranges) 9.5
# against 8.8 us at B=1 and 12.1 against 10.4 at B=2.  So one launch is taken
# only on request (combine_launch=False).
ONE_LAUNCH_MAX_RANGE_ROWS = 0


def plan_panels_host(rowptr: torch.Tensor, col: torch.Tensor, batch: int, tiles_per_panel: int,
                     max_panel_width: int | None = None, lane_target: int = LANE_TARGET,
                     pairs: bool = False):
    """Host panel layout of a CSR (numpy arrays): see ns_plan_panels."""
    lib = load_library()
    width, waves = panel_geometry(batch)
    if max_panel_width is not None:
        width = min(width, int(max_panel_width))
    rowptr = np.ascontiguousarray(rowptr.detach().to("cpu", torch.int32).numpy())
    col = np.ascontiguousarray(col.detach().to("cpu", torch.int32).numpy())
    n = rowptr.size - 1
    plan = _PanelPlan()
    entries = _c_i64()
    args = (rowptr.ctypes.data, col.ctypes.data if col.size else None, n, width,
            int(tiles_per_panel), waves, int(lane_target), PANEL_PAIRS if pairs else 0,
            ctypes.byref(plan), ctypes.byref(entries))
    _raise_on(lib.ns_plan_panels(*args, *([None] * 8)), lib)
    tiles = np.empty(4 * plan.n_tiles, np.int32)
    tile_ranges = np.empty(plan.n_tiles, np.int32)
    wave_groups = np.empty(plan.n_tiles * plan.waves + 1, np.int32)
    groups = np.empty(4 * plan.n_groups, np.int32)
    rows = np.empty(entries.value, np.uint16)
    last_steps = np.empty(plan.n_step_words, np.uint32)
    perm = np.empty(plan.n_slots, np.int32)
    cols = np.empty(plan.n_slots, np.uint16)
    _raise_on(lib.ns_plan_panels(*args, tiles.ctypes.data, tile_ranges.ctypes.data,
                                 wave_groups.ctypes.data, groups.ctypes.data, rows.ctypes.data,
                                 last_steps.ctypes.data, perm.ctypes.data, cols.ctypes.data), lib)
    return plan, tiles, tile_ranges, wave_groups, groups, rows, last_steps, perm, cols


def plan_bands_host(rowptr: torch.Tensor, col: torch.Tensor, band_width: int, block_rows: int,
                    block_steps: int = 4):
    """Host band layout of a CSR (numpy arrays): see ns_plan_bands."""
    lib = load_library()
    rowptr = np.ascontiguousarray(rowptr.detach().to("cpu", torch.int32).numpy())
    col = np.ascontiguousarray(col.detach().to("cpu", torch.int32).numpy())
    n = rowptr.size - 1
    plan = _BandPlan()
    args = (rowptr.ctypes.data, col.ctypes.data if col.size else None, n, int(band_width),
            int(block_rows), int(block_steps), ctypes.byref(plan))
    _raise_on(lib.ns_plan_bands(*args, *([None] * 5)), lib)
    wave_blocks = np.empty(BAND_WAVES * plan.n_row_blocks + 1, np.int32)
    blocks = np.empty(4 * (plan.n_blocks + 1), np.int32)
    rows = np.empty(64 * plan.n_groups, np.uint32)
    perm = np.empty(plan.n_slots, np.int32)
    cols = np.empty(plan.n_slots, np.uint16)
    _raise_on(lib.ns_plan_bands(*args, wave_blocks.ctypes.data, blocks.ctypes.data,
                                rows.ctypes.data, perm.ctypes.data, cols.ctypes.data), lib)
    return plan, wave_blocks, blocks, rows, perm, cols


def band_max_block_rows(batch: int = 16) -> int:
    """Most destination rows per band workgroup at this batch (its LDS holds the
    rows' sums over a tile of 16, 8 or 4 columns)."""
    return int(load_library().ns_band_max_block_rows(batch))


def _device_tensor(array: np.ndarray, device) -> torch.Tensor:
    if array.dtype == np.uint16:
        array = array.view(np.int16)
    elif array.dtype == np.uint32:
        array = array.view(np.int32)
    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


class _SlotLayout:
    """Weights of a CSR payload rearranged into a layout's slot order.

    Subclasses set ``n_slots`` and ``perm`` (int32 on the device: the CSR edge
    of each slot, -1 for padding); padding slots get code 0.  The copy is made
    on the device by ns_gather_slot_weights and kept for one weight key.
    """

    n_slots: int
    perm: torch.Tensor
    pairs: bool = False
    _slot_weights: tuple | None = None
    _slot_key = None

    def slot_weights(self, key, weight: torch.Tensor, block_scales: torch.Tensor | None):
        """Weights of the CSR payload (original edge order) rearranged into slot order."""
        if self._slot_key == key and self._slot_weights is not None:
            return self._slot_weights
        device, n = weight.device, self.n_slots
        nvfp4 = block_scales is not None
        if not nvfp4:
            fmt = {torch.float32: WEIGHT_F32, torch.float16: WEIGHT_F16,
                   torch.uint8: WEIGHT_E4M3}[weight.dtype]
            slots = torch.empty(n, dtype=weight.dtype, device=device)
            scales = None
        elif self.pairs:
            fmt, slots, scales = WEIGHT_NVFP4, torch.empty(n // 2, dtype=torch.int16, device=device), None
        else:
            fmt = WEIGHT_NVFP4
            slots = torch.empty(n // 2, dtype=torch.uint8, device=device)
            scales = torch.empty(n, dtype=torch.uint8, device=device)
        edges = weight.numel() * (2 if nvfp4 else 1)
        if nvfp4:
            edges = min(edges, 16 * block_scales.numel())
        lib = load_library()
        payload = weight.detach()
        _raise_on(lib.ns_gather_slot_weights(
            self.perm.data_ptr(), n, edges, fmt, int(self.pairs and nvfp4),
            payload.data_ptr() if payload.numel() else None,
            block_scales.data_ptr() if nvfp4 and block_scales.numel() else None,
            slots.data_ptr(), scales.data_ptr() if scales is not None else None,
            ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)), lib)
        self._slot_weights = (slots, scales)
        self._slot_key = key
        return self._slot_weights


class PanelLayout(_SlotLayout):
    """Column-panel layout of one graph for batch width 1 or 2 (see ns_plan_panels).

    Built once per graph structure on the host from copies of in_rowptr and
    in_col (a synchronisation; set-up only).  Holds the device tables, the
    slot permutation, the partials workspace, the row ranges' counters and,
    per weight version and encoding, the weights rearranged into slot order on
    the device.  Launches sharing a layout must be ordered on one stream.
    With several panels the panels' sums of a row range are added, and the
    range's rows updated, either by the tick kernel's last tile of the range
    (one launch per tick) or by a second kernel (``combine_launch``); the
    results are bitwise the same.  The last tile updates the whole range on
    one compute unit, so the default (``combine_launch=None``) takes one launch
    only for ranges of at most ``ONE_LAUNCH_MAX_RANGE_ROWS`` rows (none, as
    measured so far).
    """

    def __init__(self, topology, batch: int, device, *, tiles_per_panel: int | None = None,
                 max_panel_width: int | None = None, lane_target: int = LANE_TARGET,
                 pairs: bool = False, combine_launch: bool | None = None) -> None:
        n = topology.n_neurons
        width, _ = panel_geometry(batch)
        panels = -(-n // (min(width, max_panel_width or width) & ~3))
        if tiles_per_panel is None:
            # One workgroup per compute unit in total.
            units = torch.cuda.get_device_properties(device).multi_processor_count
            tiles_per_panel = max(1, units // panels)
        plan, tiles, tile_ranges, wave_groups, groups, rows, last_steps, perm, cols = \
            plan_panels_host(topology.in_rowptr, topology.in_col, batch, tiles_per_panel,
                             max_panel_width, lane_target, pairs)
        range_rows = int((tiles.reshape(-1, 4)[:, 2] - tiles.reshape(-1, 4)[:, 1]).max())
        if combine_launch is None:
            combine_launch = plan.n_panels > 1 and range_rows > ONE_LAUNCH_MAX_RANGE_ROWS
        if combine_launch:
            plan.flags |= PANEL_COMBINE_LAUNCH
        self.pairs, self.combine_launch = bool(pairs), bool(combine_launch)
        self.batch, self.n = int(batch), n
        self.n_panels, self.n_tiles, self.n_slots = plan.n_panels, plan.n_tiles, plan.n_slots
        self.n_groups, self.n_ranges = plan.n_groups, plan.n_ranges
        self.panel_width = plan.panel_width
        self.tiles = _device_tensor(tiles, device)
        self.tile_ranges = _device_tensor(tile_ranges, device)
        # every launch leaves the counters zero again
        self.range_counters = torch.zeros(plan.n_ranges, dtype=torch.int32, device=device)
        self.wave_groups = _device_tensor(wave_groups, device)
        self.groups = _device_tensor(groups, device)
        self.rows = _device_tensor(rows if rows.size else np.zeros(1, np.uint16), device)
        self.last_steps = _device_tensor(last_steps.view(np.int32), device)
        self.col = _device_tensor(cols, device)
        self.perm = torch.from_numpy(perm).to(device)
        # per-panel sums by row, then the same sums in row-table order
        self.partials = torch.empty(2 * plan.n_panels * n * batch, dtype=torch.float32,
                                    device=device)
        self._plan = plan
        self._slot_weights: tuple | None = None
        self._slot_key = None

    def plan_struct(self, slot_weight: torch.Tensor, slot_scales: torch.Tensor | None) -> _PanelPlan:
        plan = _PanelPlan()
        ctypes.memmove(ctypes.addressof(plan), ctypes.addressof(self._plan), ctypes.sizeof(plan))
        plan.tiles, plan.wave_groups = self.tiles.data_ptr(), self.wave_groups.data_ptr()
        plan.tile_ranges = self.tile_ranges.data_ptr()
        plan.range_counters = self.range_counters.data_ptr()
        plan.groups, plan.rows = self.groups.data_ptr(), self.rows.data_ptr()
        plan.last_steps = self.last_steps.data_ptr()
        plan.col = self.col.data_ptr()
        plan.weight = slot_weight.data_ptr()
        plan.slot_scales = slot_scales.data_ptr() if slot_scales is not None else None
        plan.partials = self.partials.data_ptr()
        # The struct holds raw pointers: it keeps what they point at alive, so a
        # launch captured with it (a rollout's graph) stays valid after the
        # layout has moved on to other weights.
        plan._tensors = (self, slot_weight, slot_scales)
        return plan

    def indexed_plan_struct(self) -> _PanelPlan:
        """A plan whose slots carry CSR edge numbers (NS_PANEL_INDEXED): the tick
        reads float32 weights from the CSR-order array itself, so it needs no
        slot-order copy of them."""
        plan = self.plan_struct(self.perm, None)
        plan.flags |= PANEL_INDEXED
        return plan


# Sources per band (at most 65535, the most a 16-bit band-local index holds;
# 0xFFFF marks padding): 53248 neurons x 16 columns x 4 bytes = 3.4 MB of
# state, most of an XCD's 4 MB L2, leaving room for the slot stream.  Measured
# at N=1M, M=100M, fp8 (us per tick), B=16: 49152 sources 725.6, 53248 710.7,
# 57344 719.0, 61440 720.2, 65535 726.1 (32768: 736.4); B=8: 609.4, 597.4,
# 600.5, 597.5, 598.7.  Fewer bands mean fewer barriers, groups and flushes.
BAND_WIDTH = 53248
# Wavefronts per band workgroup (kBandWaves): one workgroup per compute unit.
BAND_WAVES = 16


def default_band_rows(n: int, units: int, batch: int = 16) -> int:
    """Destination rows per band workgroup: one workgroup per compute unit, in
    whole rounds (the grid is a multiple of ``units``), as few rounds as fit LDS.
    Workgroups of one round start together and so walk the bands together, and
    each round reads the bands into L2 once more: at N=1M, 8-column tiles fit one
    round of 3907 rows (560 us per tick against 579 for two rounds of 1954)."""
    limit = band_max_block_rows(batch)
    rounds = 1
    while -(-n // (units * rounds)) > limit:
        rounds += 1
    return max(1, -(-n // (units * rounds)))


class BandLayout(_SlotLayout):
    """Source-band layout of one graph for batches that are multiples of 4 (see ns_plan_bands).

    Built once per graph structure on the host from copies of in_rowptr and
    in_col (a synchronisation; set-up only).  Holds the device tables, the
    slot permutation and, per weight version and encoding, the weights
    rearranged into slot order on the device.  ``block_rows`` defaults to
    ``default_band_rows`` for ``batch``.
    """

    def __init__(self, topology, device, *, band_width: int = BAND_WIDTH,
                 block_rows: int | None = None, block_steps: int = 4,
                 batch: int = 16) -> None:
        n = topology.n_neurons
        if block_rows is None:
            units = torch.cuda.get_device_properties(device).multi_processor_count
            block_rows = default_band_rows(n, units, batch)
        plan, wave_blocks, blocks, rows, perm, cols = plan_bands_host(
            topology.in_rowptr, topology.in_col, band_width, block_rows, block_steps)
        self.n = n
        self.band_width, self.n_bands = plan.band_width, plan.n_bands
        self.block_rows, self.n_row_blocks = plan.block_rows, plan.n_row_blocks
        self.n_blocks, self.n_groups, self.n_slots = plan.n_blocks, plan.n_groups, plan.n_slots
        self.wave_blocks = _device_tensor(wave_blocks, device)
        self.blocks = _device_tensor(blocks, device)
        self.rows = _device_tensor(rows, device)
        self.col = _device_tensor(cols, device)
        self.perm = torch.from_numpy(perm).to(device)
        self._plan = plan
        self._slot_weights = None
        self._slot_key = None

    def plan_struct(self, slot_weight: torch.Tensor, slot_scales: torch.Tensor | None) -> _BandPlan:
        plan = _BandPlan()
        ctypes.memmove(ctypes.addressof(plan), ctypes.addressof(self._plan), ctypes.sizeof(plan))
        plan.wave_blocks, plan.blocks = self.wave_blocks.data_ptr(), self.blocks.data_ptr()
        plan.rows, plan.col = self.rows.data_ptr(), self.col.data_ptr()
        plan.weight = slot_weight.data_ptr()
        plan.slot_scales = slot_scales.data_ptr() if slot_scales is not None else None
        plan._tensors = (self, slot_weight, slot_scales)   # kept alive with the pointers
        return plan


class NativeExtension:
    """Drop-in for the reference's compiled extension (hot-path ops only)."""

    def __init__(self) -> None:
        self.lib = load_library()
        # id(rowptr) -> (weakref, version, {capacity: plan}); identity is re-checked on
        # lookup.  A rowptr made under torch.inference_mode has no version counter
        # (PyTorch tracks none for such tensors): its plans follow its identity alone.
        self._plans: "OrderedDict[int, tuple]" = OrderedDict()
        self._lock = threading.Lock()

    # -- row plans ---------------------------------------------------------
    def plan_tensors(self, rowptr: torch.Tensor, batch: int) -> tuple[torch.Tensor, int, int]:
        """Cached (bounds, blocks, edges per block) of ``rowptr`` for batch width
        ``batch`` (cached per kernel capacity, which the batch width sets)."""
        capacity = int(self.lib.ns_block_edges(int(batch)))
        key = id(rowptr)
        with self._lock:
            entry = self._plans.get(key)
            version = None if torch.is_inference(rowptr) else rowptr._version
            if entry is None or entry[0]() is not rowptr or entry[1] != version:
                entry = (weakref.ref(rowptr), version, {})
                self._plans[key] = entry
            self._plans.move_to_end(key)
            while len(self._plans) > _PLAN_CACHE:
                self._plans.popitem(last=False)
            plan = entry[2].get(capacity)
        if plan is None:
            plan = plan_row_blocks(rowptr, batch, rowptr.device)
            with self._lock:
                entry[2][capacity] = plan
        return plan

    def plan_for(self, rowptr: torch.Tensor, batch: int) -> _RowPlan:
        bounds, blocks, block_edges = self.plan_tensors(rowptr, batch)
        return _RowPlan(bounds.data_ptr(), blocks, block_edges, 0)

    # -- weights -----------------------------------------------------------
    @staticmethod
    def _csr(state, rowptr, source, weight, block_scales, global_scale) -> _Csr:
        _index(rowptr, state)
        _index(source, state)
        n = state.size(1)
        edges = source.numel()
        if rowptr.numel() != n + 1:
            raise RuntimeError("invalid CSR geometry")
        if (not isinstance(weight, torch.Tensor) or weight.device != state.device
                or not weight.is_contiguous() or weight.dim() != 1):
            raise RuntimeError("CSR weights must be a contiguous vector on the state device")
        scales_ptr = scale_ptr = None
        if weight.dtype == torch.uint8:
            if global_scale is None:
                raise RuntimeError("quantized CSR weights require a global scale")
            _check_float(global_scale, state, "global scale")
            if global_scale.numel() != 1:
                raise RuntimeError("global scale must have one value")
            expected = (edges + 1) // 2 if block_scales is not None else edges
            if weight.numel() != expected:
                raise RuntimeError("invalid quantized CSR weight count")
            if block_scales is not None:
                if (block_scales.device != state.device or block_scales.dtype != torch.uint8
                        or not block_scales.is_contiguous() or block_scales.dim() != 1
                        or block_scales.numel() != (edges + 15) // 16):
                    raise RuntimeError("invalid NVFP4 block scales")
                fmt = WEIGHT_NVFP4
                scales_ptr = block_scales.data_ptr()
            else:
                fmt = WEIGHT_E4M3
            scale_ptr = global_scale.data_ptr()
        else:
            if (block_scales is not None or global_scale is not None or weight.numel() != edges
                    or weight.dtype not in (torch.float32, torch.float16)):
                raise RuntimeError("invalid floating-point CSR weights")
            fmt = WEIGHT_F32 if weight.dtype == torch.float32 else WEIGHT_F16
        return _Csr(n, edges, rowptr.data_ptr(), source.data_ptr(), weight.data_ptr(), fmt,
                    scales_ptr, scale_ptr)

    # -- ops ----------------------------------------------------------------
    def dendritic_step(self, state, dendrite, adaptation, params, rowptr, source, weight,
                       input, input_scalar, dendritic_input, dendritic_scalar, width,
                       block_scales=None, global_scale=None, panels=None, bands=None,
                       current_out=None):
        _check_state(state)
        args = _StepArgs()
        args.state = _plane(state, state, "state")
        args.dendrite = _plane(dendrite, state, "dendrite")
        args.adaptation = _plane(adaptation, state, "adaptation")
        args.params = _params(params, state)
        args.drive = _drive(input, input_scalar, state)
        args.dendritic_drive = _drive(dendritic_input, dendritic_scalar, state)
        args.matrix = self._csr(state, rowptr, source, weight, block_scales, global_scale)
        if width not in (8, 16, 32):
            raise RuntimeError("width must be 8, 16 or 32")
        batch, n = state.shape
        args.n_neurons, args.batch = n, batch
        panel_struct = None
        if bands is not None:              # a _BandPlan built by BandLayout.plan_struct
            if panels is not None:
                raise RuntimeError("pass a panel or a band layout, not both")
            if not (state.stride(0) == 1 and state.stride(1) >= batch and state.stride(1) % 4 == 0
                    and state.data_ptr() % 16 == 0):
                # The band kernel gathers whole neuron rows of s: a neuron-major copy.
                state = new_planes(1, batch, n, state)[0].copy_(state)
                args.state = _plane(state, state, "state")
        elif panels is not None:
            panel_struct = panels          # a _PanelPlan built by PanelLayout.plan_struct
            args.panels = ctypes.addressof(panel_struct)
        else:
            args.plan = self.plan_for(rowptr, batch)
        outs = new_planes(3, batch, n, state)
        args.out_state, args.out_dendrite, args.out_adaptation = (_out(o) for o in outs)
        if current_out is not None:        # j = W @ s as well, for a recorded tick's backward
            _check_float(current_out, state, "current")
            if current_out.shape != state.shape:
                raise RuntimeError("state/current shape mismatch")
            args.out_current = _out(current_out)
        stream = torch.cuda.current_stream(state.device).cuda_stream
        if bands is not None:
            _raise_on(self.lib.ns_dendritic_step_bands(ctypes.byref(args), ctypes.byref(bands),
                                                       stream), self.lib)
        else:
            _raise_on(self.lib.ns_dendritic_step(ctypes.byref(args), stream), self.lib)
        return outs

    def dendritic_event(self, state, dendrite, adaptation, params, current, emitted, theta,
                        rowptr, dst, weight_index, weight, input, input_scalar,
                        dendritic_input, dendritic_scalar, delta=None, pending=None,
                        out_weight=None, advance_only=False, activity=None):
        """One PELS tick (ns_dendritic_event); returns the four new planes.

        Without ``pending`` the tick is two launches and ``current`` is updated
        in place.  ``pending=(pending_in, pending_out)``, two float32 buffers of
        B*N entries (n*B + b), makes it one launch: ``current`` receives
        current + pending_in, pending_in is zeroed, and this tick's W @ delta
        is added into pending_out (zero on entry), so the persistent current
        afterwards is current + pending_out.  ``out_weight`` optionally gives
        the weights in source-major order (``weight[weight_index]``), which the
        scatter then streams instead of gathering.  ``advance_only`` runs the
        advance and emission only (NS_EVENT_ADVANCE_ONLY): ``delta`` (entry
        n*B + b) receives the emitted deltas, for the caller to propagate, and
        ``current`` is left as it was, or, with ``pending=(pending_in, None)``,
        receives current + pending_in in one launch.  ``activity``, an int64
        tensor of EVENT_ACTIVITY_SLOTS * EVENT_ACTIVITY_STRIDE counters (one-launch
        forms only), has the tick's active out-edges added to it."""
        _check_state(state)
        args = _EventArgs()
        args.state = _plane(state, state, "state")
        args.dendrite = _plane(dendrite, state, "dendrite")
        args.adaptation = _plane(adaptation, state, "adaptation")
        args.params = _params(params, state)
        args.drive = _drive(input, input_scalar, state)
        args.dendritic_drive = _drive(dendritic_input, dendritic_scalar, state)
        _check_float(current, state, "current")
        if current.shape != state.shape:
            raise RuntimeError("state/current/drive shape mismatch")
        args.current = current.data_ptr()
        args.current_stride_b, args.current_stride_n = current.stride(0), current.stride(1)
        args.emitted = _plane(emitted, state, "emitted")
        _check_float(theta, state, "theta")
        if theta.dim() != 1 or theta.numel() != state.size(1):
            raise RuntimeError("theta must have N values")
        args.theta = _Vector(theta.data_ptr(), theta.stride(0))
        for index in (rowptr, dst, weight_index):
            _index(index, state)
        _check_float(weight, state, "weight")
        if (rowptr.numel() != state.size(1) + 1 or dst.numel() != weight.numel()
                or dst.numel() != weight_index.numel() or not weight.is_contiguous()
                or weight.dim() != 1):
            raise RuntimeError("invalid event topology geometry")
        args.out_rowptr, args.dst = rowptr.data_ptr(), dst.data_ptr()
        args.weight_index, args.weight = weight_index.data_ptr(), weight.data_ptr()
        args.n_edges = weight.numel()
        batch, n = state.shape
        args.n_neurons, args.batch = n, batch
        outs = new_planes(4, batch, n, state)
        (args.out_state, args.out_dendrite, args.out_adaptation,
         args.out_emitted) = (_out(o) for o in outs)
        if out_weight is not None:
            if (out_weight.dtype != torch.float32 or not out_weight.is_contiguous()
                    or out_weight.numel() != weight.numel()
                    or out_weight.device != state.device):
                raise RuntimeError("out_weight must be M contiguous float32 on the state's device")
            args.out_weight = out_weight.data_ptr()
        if advance_only:
            args.flags = EVENT_ADVANCE_ONLY
        if pending is not None:
            pending_in, pending_out = pending
            if advance_only and pending_out is not None:
                raise RuntimeError("the advance-only tick scatters nothing: no pending_out")
            for buffer in (pending_in, pending_out):
                if buffer is None:
                    continue
                if (buffer.numel() < batch * n or buffer.dtype != torch.float32
                        or not buffer.is_contiguous() or buffer.device != state.device):
                    raise RuntimeError("pending buffers must hold B*N float32 on the state's device")
            args.pending_in = pending_in.data_ptr()
            args.pending_out = None if pending_out is None else pending_out.data_ptr()
        if delta is None and (pending is None or advance_only):
            delta = torch.empty(batch * n, dtype=torch.float32, device=state.device)
        if activity is not None:
            if (activity.dtype != torch.int64 or not activity.is_contiguous()
                    or activity.numel() < EVENT_ACTIVITY_SLOTS * EVENT_ACTIVITY_STRIDE
                    or activity.device != state.device):
                raise RuntimeError("activity must hold EVENT_ACTIVITY_SLOTS * "
                                   "EVENT_ACTIVITY_STRIDE int64 counters on the state's device")
            args.activity = activity.data_ptr()
        if delta is not None:
            if (delta.numel() < batch * n or delta.dtype != torch.float32
                    or not delta.is_contiguous()):
                raise RuntimeError("delta workspace must hold B*N float32")
            args.delta = delta.data_ptr()
        stream = torch.cuda.current_stream(state.device).cuda_stream
        _raise_on(self.lib.ns_dendritic_event(ctypes.byref(args), stream), self.lib)
        return outs

    def dendritic_step_backward(self, state, dendrite, adaptation, params, rowptr, source,
                                weight, input, input_scalar, dendritic_input, dendritic_scalar,
                                out_rowptr, dst, weight_index, grad_state, grad_dendrite,
                                grad_adaptation, *, need_drive=False, need_dendritic=False,
                                need_weight=False, need_params=(False,) * 6, out_weight=None,
                                current=None, transposed_panels=None):
        """Gradients of one float32 tick (ns_dendritic_step_backward).

        Returns (d_state, d_dendrite, d_adaptation, d_drive, d_dendritic_drive,
        d_weight, [d_param x 6]); entries not asked for are None.  Upstream
        gradients may be None (zero).  ``out_weight`` optionally gives the
        weights in source-major order (``weight[weight_index]``), which the
        transposed product then streams instead of gathering.  ``current``
        optionally gives the forward's j = W @ s as ``dendritic_step`` wrote it
        (``current_out``, a neuron-major [B,N] plane), which spares recomputing it.
        ``transposed_panels`` (a ``_PanelPlan`` of ``TransposedPanels.plan``,
        batch 1 or 2) runs the transposed product on the panel kernel.
        """
        _check_state(state)
        batch, n = state.shape
        args = _StepGradArgs()
        args.n_neurons, args.batch = n, batch
        args.state = _plane(state, state, "state")
        args.dendrite = _plane(dendrite, state, "dendrite")
        args.adaptation = _plane(adaptation, state, "adaptation")
        args.params = _params(params, state)
        args.drive = _drive(input, input_scalar, state)
        args.dendritic_drive = _drive(dendritic_input, dendritic_scalar, state)
        if weight.dtype != torch.float32:
            raise RuntimeError("the tick backward needs float32 weights")
        args.matrix = self._csr(state, rowptr, source, weight, None, None)
        args.plan = self.plan_for(rowptr, batch)
        for index in (out_rowptr, dst, weight_index):
            _index(index, state)
        if out_rowptr.numel() != n + 1 or dst.numel() != weight.numel() or \
                weight_index.numel() != weight.numel():
            raise RuntimeError("invalid source-major topology geometry")
        args.out_rowptr, args.dst = out_rowptr.data_ptr(), dst.data_ptr()
        args.out_weight_index = weight_index.data_ptr()
        if out_weight is not None:
            _check_float(out_weight, state, "source-major weights")
            if out_weight.numel() != weight.numel() or not out_weight.is_contiguous():
                raise RuntimeError("source-major weights must be a contiguous [M] vector")
            args.out_weight = out_weight.data_ptr() if out_weight.numel() else None
        if transposed_panels is not None:
            args.transposed_panels = ctypes.addressof(transposed_panels)
        if current is not None:
            _check_float(current, state, "current")
            if current.shape != state.shape or not _neuron_major(current):
                raise RuntimeError("current must be a neuron-major [B,N] plane")
            args.current = current.data_ptr()
        args.grad_state = _drive(grad_state, 0.0, state)
        args.grad_dendrite = _drive(grad_dendrite, 0.0, state)
        args.grad_adaptation = _drive(grad_adaptation, 0.0, state)
        planes = new_planes(3 + int(need_drive) + int(need_dendritic), batch, n, state)
        args.d_state, args.d_dendrite, args.d_adaptation = (_out(o) for o in planes[:3])
        rest = iter(planes[3:])
        d_drive = next(rest) if need_drive else None
        d_dendritic = next(rest) if need_dendritic else None
        args.d_drive = _out(d_drive) if d_drive is not None else _OutPlane(None, 0, 0)
        args.d_dendritic_drive = (_out(d_dendritic) if d_dendritic is not None
                                  else _OutPlane(None, 0, 0))
        d_weight = torch.empty_like(weight) if need_weight else None
        args.d_weight = d_weight.data_ptr() if d_weight is not None and weight.numel() else None
        # The wanted parameter gradients and the workspace share one allocation.
        wanted = [i for i, want in enumerate(need_params) if want]
        work = int(self.lib.ns_step_backward_workspace_floats(n, batch))
        block = torch.empty(len(wanted) * n + work, dtype=torch.float32, device=state.device)
        d_params = [None] * 6
        for k, i in enumerate(wanted):
            d_params[i] = block[k * n:(k + 1) * n]
            args.d_params[i] = d_params[i].data_ptr()
        workspace = block[len(wanted) * n:]
        args.workspace = workspace.data_ptr() if workspace.numel() else None
        stream = torch.cuda.current_stream(state.device).cuda_stream
        _raise_on(self.lib.ns_dendritic_step_backward(ctypes.byref(args), stream), self.lib)
        return (*planes[:3], d_drive, d_dendritic, d_weight, d_params)

    def csr_spmm(self, source, rowptr, col, weight, block_scales=None, global_scale=None, *,
                 accumulate_into=None, panels=None):
        """W @ source as a new neuron-major [B,N] plane, or, with
        ``accumulate_into`` (a [B,N] float32 tensor on the device whose elements
        are distinct), added into that tensor in place, which is returned.
        ``panels`` (a ``_PanelPlan`` of this CSR, batch 1 or 2) runs the product
        on the column-panel kernel instead of row blocks."""
        _check_state(source)
        args = _SpmmArgs()
        args.source = _plane(source, source, "source")
        args.matrix = self._csr(source, rowptr, col, weight, block_scales, global_scale)
        batch, n = source.shape
        args.n_neurons, args.batch = n, batch
        if panels is not None:
            args.panels = ctypes.addressof(panels)
        else:
            args.plan = self.plan_for(rowptr, batch)
        if accumulate_into is None:
            (out,) = new_planes(1, batch, n, source)
        else:
            out = accumulate_into
            _check_float(out, source, "accumulated output")
            if out.shape != source.shape:
                raise RuntimeError("the accumulated output must be [B,N]")
            args.accumulate = 1
        args.out = _out(out)
        stream = torch.cuda.current_stream(source.device).cuda_stream
        _raise_on(self.lib.ns_csr_spmm(ctypes.byref(args), stream), self.lib)
        return out


def drive_plane(value: torch.Tensor, state_like: torch.Tensor) -> _Plane:
    """The plane of a [B,N]-broadcastable float32 drive tensor (validated)."""
    view = value.expand_as(state_like)
    return _plane(view, state_like, "drive")


class TickLauncher:
    """A prepared fused tick: fixed weights, plan and parameters.

    Only the state planes (and, if given per call, the drive planes) change
    between launches, so a multi-tick loop does no validation or allocation per
    tick and can be captured into one HIP graph.  Keeps every tensor it points
    at alive; drive planes passed per call must be kept alive by the caller.
    """

    def __init__(self, extension: "NativeExtension", state_like: torch.Tensor, params, rowptr,
                 col, weight, drive, dendritic_drive, block_scales=None, global_scale=None,
                 panels=None, bands=None):
        _check_state(state_like)
        self.lib = extension.lib
        args = _StepArgs()
        args.params = _params(params, state_like)
        args.matrix = extension._csr(state_like, rowptr, col, weight, block_scales, global_scale)
        drive_t = drive if isinstance(drive, torch.Tensor) else None
        ddrive_t = dendritic_drive if isinstance(dendritic_drive, torch.Tensor) else None
        if drive_t is not None:
            drive_t = drive_t.expand_as(state_like)
        if ddrive_t is not None:
            ddrive_t = ddrive_t.expand_as(state_like)
        args.drive = _drive(drive_t, 0.0 if drive_t is not None else float(drive), state_like)
        args.dendritic_drive = _drive(ddrive_t, 0.0 if ddrive_t is not None
                                      else float(dendritic_drive), state_like)
        self.fixed_drives = (_Plane.from_buffer_copy(args.drive),
                             _Plane.from_buffer_copy(args.dendritic_drive))
        batch, n = state_like.shape
        args.n_neurons, args.batch = n, batch
        bounds = None
        if bands is not None and panels is not None:
            raise RuntimeError("pass a panel or a band layout, not both")
        if bands is not None:
            pass                            # the band plan goes with each launch
        elif panels is not None:
            args.panels = ctypes.addressof(panels)
        else:
            bounds, blocks, block_edges = extension.plan_tensors(rowptr, batch)
            args.plan = _RowPlan(bounds.data_ptr(), blocks, block_edges, 0)
        self.args = args
        self.bands = bands
        self.batch, self.n = batch, n
        self._keep = (list(params), rowptr, col, weight, drive_t, ddrive_t, block_scales,
                      global_scale, bounds, panels, bands)

    def __call__(self, source: tuple, target: tuple, stream: int | None = None,
                 drives: tuple | None = None) -> None:
        """One tick from planes (s, d, a) into planes (s', d', a') (all [B,N] views).
        ``drives`` optionally replaces the two drive planes for this launch:
        (somatic, dendritic) ``_Plane`` structs (see ``drive_plane``), None for
        the one fixed at construction."""
        args = self.args
        somatic, dendritic = drives if drives is not None else (None, None)
        args.drive = somatic if somatic is not None else self.fixed_drives[0]
        args.dendritic_drive = dendritic if dendritic is not None else self.fixed_drives[1]
        args.state = _Plane(source[0].data_ptr(), source[0].stride(0), source[0].stride(1), 0.0)
        args.dendrite = _Plane(source[1].data_ptr(), source[1].stride(0), source[1].stride(1), 0.0)
        args.adaptation = _Plane(source[2].data_ptr(), source[2].stride(0), source[2].stride(1),
                                 0.0)
        args.out_state, args.out_dendrite, args.out_adaptation = (_out(t) for t in target)
        if stream is None:
            stream = torch.cuda.current_stream(source[0].device).cuda_stream
        if self.bands is not None:
            _raise_on(self.lib.ns_dendritic_step_bands(ctypes.byref(args), ctypes.byref(self.bands),
                                                       stream), self.lib)
        else:
            _raise_on(self.lib.ns_dendritic_step(ctypes.byref(args), stream), self.lib)


def current_stream(device: torch.device) -> int:
    """torch's current HIP stream on ``device`` (an index-carrying CUDA device), as
    the integer handle the C-ABI takes."""
    return _RAW_STREAM(device.index)


def _public_raw_stream(index: int) -> int:
    return torch.cuda.current_stream(index).cuda_stream


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", _public_raw_stream)


def _consecutive(struct_type, names: tuple, size: int) -> int:
    """Byte offset of the first of ``names``, checked to be laid out back to back."""
    offsets = [getattr(struct_type, name).offset for name in names]
    if any(b - a != size for a, b in zip(offsets, offsets[1:])):
        raise RuntimeError(f"{struct_type.__name__}: fields {names} are not consecutive")
    return offsets[0]


# The per-tick words of the step, event and step-backward argument structs are
# written with one struct.pack_into per run of consecutive fields: input planes
# (data, two strides, scalar: 32 bytes), output planes (data, two strides: 24
# bytes) and pointers.  The offsets below are checked against the ctypes layouts.
_PLANES5 = struct.Struct("<" + "Qqqf4x" * 5)
_PLANES3 = struct.Struct("<" + "Qqqf4x" * 3)
_OUTS4 = struct.Struct("<" + "Qqq" * 4)
_OUTS5 = struct.Struct("<" + "Qqq" * 5)
_POINTERS11 = struct.Struct("<" + "Q" * 11)
_CURRENT_EMITTED = struct.Struct("<Qqq" + "Qqqf4x")
_EVENT_TAIL = struct.Struct("<QQQQiiQ")
if ctypes.sizeof(_Plane) != 32 or ctypes.sizeof(_OutPlane) != 24:
    raise RuntimeError("plane structs must be 32 and 24 bytes")
_IN_NAMES = ("state", "dendrite", "adaptation", "drive", "dendritic_drive")
_STEP_IN = _consecutive(_StepArgs, _IN_NAMES, 32)
_STEP_OUT = _consecutive(_StepArgs, ("out_state", "out_dendrite", "out_adaptation",
                                     "out_current"), 24)
_EVENT_IN = _consecutive(_EventArgs, _IN_NAMES, 32)
_EVENT_OUT = _consecutive(_EventArgs, ("out_state", "out_dendrite", "out_adaptation",
                                       "out_emitted"), 24)
_EVENT_CURRENT = _consecutive(_EventArgs, ("current", "current_stride_b", "current_stride_n",
                                           "emitted"), 8)
_EVENT_TAIL_AT = _consecutive(_EventArgs, ("delta", "pending_in", "pending_out", "out_weight"), 8)
if (_EventArgs.flags.offset != _EVENT_TAIL_AT + 32
        or _EventArgs.activity.offset != _EVENT_TAIL_AT + 40):
    raise RuntimeError("_EventArgs: flags and activity must follow out_weight")
_GRAD_IN = _consecutive(_StepGradArgs, _IN_NAMES, 32)
_GRAD_UP = _consecutive(_StepGradArgs, ("grad_state", "grad_dendrite", "grad_adaptation"), 32)
_GRAD_OUT = _consecutive(_StepGradArgs, ("d_state", "d_dendrite", "d_adaptation", "d_drive",
                                         "d_dendritic_drive"), 24)
_GRAD_POINTERS = _StepGradArgs.d_weight.offset
if [getattr(_StepGradArgs, f).offset - _GRAD_POINTERS
        for f in ("d_params", "workspace", "current", "out_weight", "transposed_panels")] \
        != [8, 56, 64, 72, 80]:
    raise RuntimeError("_StepGradArgs: the output pointers must be consecutive")


_data_ptr = torch.Tensor.data_ptr


def _plane_words(value: torch.Tensor, state: torch.Tensor, what: str) -> tuple:
    """(data, stride_b, stride_n) of a validated [B,N] float32 plane."""
    _check_float(value, state, what)
    if value.shape != state.shape:
        raise RuntimeError("state/current/drive shape mismatch")
    return value.data_ptr(), value.stride(0), value.stride(1)


def _drive_words(value: torch.Tensor | None, scalar: float, state: torch.Tensor) -> tuple:
    if value is None:
        return 0, 0, 0, float(scalar)
    return _plane_words(value, state, "drive") + (0.0,)


class PreparedTick:
    """An eager matrix tick with its fixed arguments validated once: the
    parameter vectors, the CSR matrix and its row plan, panel or band layout.

    Each call validates the three state planes unless they are this object's own
    previous outputs, allocates three fresh neuron-major output planes (one
    allocation, as ``new_planes``), writes the per-tick words of the argument
    struct in two packed writes and launches on torch's current stream.  The
    results equal ``NativeExtension.dendritic_step`` on the same inputs.
    ``matches`` says whether the prepared arguments are still the ones given
    (the same tensor objects at the same addresses); the caller builds a new one
    otherwise.  Every fixed tensor is kept alive here."""

    def __init__(self, extension: "NativeExtension", state: torch.Tensor, params, rowptr, col,
                 weight, block_scales=None, global_scale=None, panels=None, bands=None):
        _check_state(state)
        if panels is not None and bands is not None:
            raise RuntimeError("pass a panel or a band layout, not both")
        self.lib = extension.lib
        args = _StepArgs()
        args.params = _params(params, state)
        args.matrix = extension._csr(state, rowptr, col, weight, block_scales, global_scale)
        batch, n = state.shape
        args.n_neurons, args.batch = n, batch
        bounds = None
        if panels is not None:
            args.panels = ctypes.addressof(panels)
        elif bands is None:
            bounds, blocks, block_edges = extension.plan_tensors(rowptr, batch)
            args.plan = _RowPlan(bounds.data_ptr(), blocks, block_edges, 0)
        self.args, self._ref = args, ctypes.byref(args)
        self.bands, self._bands_ref = bands, (ctypes.byref(bands) if bands is not None else None)
        self.batch, self.n, self.shape, self.device = batch, n, state.shape, state.device
        self.params = tuple(params)
        self._fixed = (rowptr, col, weight, block_scales, global_scale, panels, bands,
                       *self.params)
        self._addressed = (*self.params, rowptr, col, weight)
        self._pointers = tuple(map(_data_ptr, self._addressed))
        self._bounds = bounds
        self._last = None     # (s', d', a', their nine words)

    def matches(self, state, params, rowptr, col, weight, block_scales=None, global_scale=None,
                panels=None, bands=None) -> bool:
        """The same tensor objects (and layouts) as prepared, still at the same
        addresses (an assignment to ``.data`` keeps the object, not the address)."""
        given = (rowptr, col, weight, block_scales, global_scale, panels, bands, *params)
        if len(given) != 13 or not all(map(is_, given, self._fixed)):
            return False
        last = self._last
        if (last is None or state is not last[0]) and state.shape != self.shape:
            return False
        return tuple(map(_data_ptr, self._addressed)) == self._pointers

    def __call__(self, state, dendrite, adaptation, drive, drive_scalar, dendritic_drive,
                 dendritic_scalar, current: bool = False) -> tuple:
        """One tick; drives are validated [B,N] views or None with a scalar.
        Returns the three new planes, and with ``current`` a fourth, j = W @ s
        (neuron-major, from the same allocation), as a recorded tick's backward
        reads it."""
        last = self._last
        if (last is not None and state is last[0] and dendrite is last[1]
                and adaptation is last[2] and state.data_ptr() == last[3][0]
                and dendrite.data_ptr() == last[3][4] and adaptation.data_ptr() == last[3][8]):
            words = last[3]
        else:
            _check_state(state)
            if state.device != self.device:
                raise RuntimeError("all tensors must be on the state's CUDA device")
            if state.shape != self.shape:
                raise RuntimeError("state/current/drive shape mismatch")
            if self.bands is not None and not (
                    state.stride(0) == 1 and state.stride(1) >= self.batch
                    and state.stride(1) % 4 == 0 and state.data_ptr() % 16 == 0):
                # The band kernel gathers whole neuron rows of s: a neuron-major copy.
                state = new_planes(1, self.batch, self.n, state)[0].copy_(state)
            words = (_plane_words(state, state, "state") + (0.0,)
                     + _plane_words(dendrite, state, "dendrite") + (0.0,)
                     + _plane_words(adaptation, state, "adaptation") + (0.0,))
        args = self.args
        _PLANES5.pack_into(args, _STEP_IN, *words,
                           *_drive_words(drive, drive_scalar, state),
                           *_drive_words(dendritic_drive, dendritic_scalar, state))
        batch, n = self.batch, self.n
        outs, base = _new_outputs(4 if current else 3, batch, n, self.device)
        size = 4 * n * batch
        out = (base, 1, batch, base + size, 1, batch, base + 2 * size, 1, batch)
        _OUTS4.pack_into(args, _STEP_OUT, *out,
                         *((base + 3 * size, 1, batch) if current else (0, 0, 0)))
        stream = current_stream(self.device)
        if self.bands is not None:
            code = self.lib.ns_dendritic_step_bands(self._ref, self._bands_ref, stream)
        else:
            code = self.lib.ns_dendritic_step(self._ref, stream)
        _raise_on(code, self.lib)
        self._last = (outs[0], outs[1], outs[2],
                      (out[0], 1, batch, 0.0, out[3], 1, batch, 0.0, out[6], 1, batch, 0.0))
        return outs


class PreparedBackward:
    """The backward of a recorded matrix tick (ns_dendritic_step_backward) with
    its fixed arguments validated once: the parameter vectors, the float32 CSR
    with its row plan and the source-major view.  Each call validates the
    forward's state planes, drives, upstream gradients, the forward's current
    and the optional source-major weights, allocates the gradient planes (one
    allocation), the weight gradient and the parameter gradients with the
    workspace (one allocation), writes the per-call words and launches.  The
    results equal ``NativeExtension.dendritic_step_backward`` on the same inputs."""

    def __init__(self, extension: "NativeExtension", state: torch.Tensor, params, rowptr, col,
                 weight, out_rowptr, dst, weight_index):
        _check_state(state)
        batch, n = state.shape
        args = _StepGradArgs()
        args.n_neurons, args.batch = n, batch
        args.params = _params(params, state)
        if weight.dtype != torch.float32:
            raise RuntimeError("the tick backward needs float32 weights")
        args.matrix = extension._csr(state, rowptr, col, weight, None, None)
        bounds, blocks, block_edges = extension.plan_tensors(rowptr, batch)
        args.plan = _RowPlan(bounds.data_ptr(), blocks, block_edges, 0)
        for index in (out_rowptr, dst, weight_index):
            _index(index, state)
        if out_rowptr.numel() != n + 1 or dst.numel() != weight.numel() or \
                weight_index.numel() != weight.numel():
            raise RuntimeError("invalid source-major topology geometry")
        args.out_rowptr, args.dst = out_rowptr.data_ptr(), dst.data_ptr()
        args.out_weight_index = weight_index.data_ptr()
        self.lib, self.args, self._ref = extension.lib, args, ctypes.byref(args)
        self.batch, self.n, self.shape, self.device = batch, n, state.shape, state.device
        self.params = tuple(params)
        self._work = int(extension.lib.ns_step_backward_workspace_floats(n, batch))
        self._tensors = (rowptr, col, weight, out_rowptr, dst, weight_index)
        self._bounds = bounds

    def matches(self, state, params, rowptr, col, weight, out_rowptr, dst, weight_index) -> bool:
        """Whether the given tensors are those prepared: the same objects, or (as
        autograd's saved tensors may be) tensors over the same memory with the same
        layout."""
        given = tuple(params) + (rowptr, col, weight, out_rowptr, dst, weight_index)
        mine = self.params + self._tensors
        if state.shape != self.shape or len(given) != len(mine):
            return False
        return all(a is b or (a.data_ptr() == b.data_ptr() and a.dtype == b.dtype
                              and a.shape == b.shape and a.stride() == b.stride())
                   for a, b in zip(given, mine))

    def __call__(self, state, dendrite, adaptation, drive, drive_scalar, dendritic_drive,
                 dendritic_scalar, grad_state, grad_dendrite, grad_adaptation, *,
                 need_drive=False, need_dendritic=False, need_weight=False,
                 need_params=(False,) * 6, out_weight=None, current=None,
                 transposed_panels=None):
        _check_state(state)
        if state.device != self.device:
            raise RuntimeError("all tensors must be on the state's CUDA device")
        if state.shape != self.shape:
            raise RuntimeError("state/current/drive shape mismatch")
        batch, n, weight = self.batch, self.n, self._tensors[2]
        args = self.args
        _PLANES5.pack_into(args, _GRAD_IN,
                           *_plane_words(state, state, "state"), 0.0,
                           *_plane_words(dendrite, state, "dendrite"), 0.0,
                           *_plane_words(adaptation, state, "adaptation"), 0.0,
                           *_drive_words(drive, drive_scalar, state),
                           *_drive_words(dendritic_drive, dendritic_scalar, state))
        _PLANES3.pack_into(args, _GRAD_UP, *_drive_words(grad_state, 0.0, state),
                           *_drive_words(grad_dendrite, 0.0, state),
                           *_drive_words(grad_adaptation, 0.0, state))
        out_weight_ptr = 0
        if out_weight is not None:
            _check_float(out_weight, state, "source-major weights")
            if out_weight.numel() != weight.numel() or not out_weight.is_contiguous():
                raise RuntimeError("source-major weights must be a contiguous [M] vector")
            out_weight_ptr = out_weight.data_ptr() if out_weight.numel() else 0
        current_ptr = 0
        if current is not None:
            _check_float(current, state, "current")
            if current.shape != state.shape or not _neuron_major(current):
                raise RuntimeError("current must be a neuron-major [B,N] plane")
            current_ptr = current.data_ptr()
        count = 3 + int(need_drive) + int(need_dendritic)
        storage = torch.empty((count, n, batch), dtype=torch.float32, device=self.device)
        base, size = storage.data_ptr(), 4 * n * batch
        words = []
        for k in range(5):
            present = k < 3 or (k == 3 and need_drive) or (k == 4 and need_dendritic)
            index = k if k < 4 else count - 1
            words += (base + index * size, 1, batch) if present else (0, 0, 0)
        _OUTS5.pack_into(args, _GRAD_OUT, *words)
        planes = storage.transpose(1, 2).unbind(0)
        d_weight = torch.empty_like(weight) if need_weight else None
        wanted = [i for i, want in enumerate(need_params) if want]
        block = torch.empty(len(wanted) * n + self._work, dtype=torch.float32,
                            device=self.device)
        d_params = [None] * 6
        param_ptrs = [0] * 6
        for k, i in enumerate(wanted):
            d_params[i] = block[k * n:(k + 1) * n]
            param_ptrs[i] = d_params[i].data_ptr()
        workspace_ptr = block.data_ptr() + 4 * len(wanted) * n if self._work else 0
        _POINTERS11.pack_into(args, _GRAD_POINTERS,
                              d_weight.data_ptr() if d_weight is not None and weight.numel() else 0,
                              *param_ptrs, workspace_ptr, current_ptr, out_weight_ptr,
                              ctypes.addressof(transposed_panels) if transposed_panels is not None
                              else 0)
        _raise_on(self.lib.ns_dendritic_step_backward(self._ref, current_stream(self.device)),
                  self.lib)
        d_drive = planes[3] if need_drive else None
        d_dendritic = planes[count - 1] if need_dendritic else None
        return (planes[0], planes[1], planes[2], d_drive, d_dendritic, d_weight, d_params)


class PreparedEvent:
    """An eager PELS tick with its fixed arguments validated once: parameter
    vectors, thresholds, the source-major topology, the delta workspace (made
    here on first need when none is given), the two pending buffers (n*B + b
    entries each) and the activity counters.

    Per call it validates the state, emitted and current planes unless they are
    the ones it saw (or wrote) last, allocates four fresh neuron-major output
    planes and writes the per-tick words: planes, the pending buffers of
    ``parity`` (0 or 1; None without pending buffers), the source-major weight
    copy, the advance-only flag and the activity counters of a sampled tick.
    The results equal ``NativeExtension.dendritic_event`` on the same inputs."""

    def __init__(self, extension: "NativeExtension", state: torch.Tensor, params, theta, rowptr,
                 dst, weight_index, weight, delta=None, pending=None, activity=None):
        _check_state(state)
        self.lib = extension.lib
        args = _EventArgs()
        args.params = _params(params, state)
        _check_float(theta, state, "theta")
        if theta.dim() != 1 or theta.numel() != state.size(1):
            raise RuntimeError("theta must have N values")
        args.theta = _Vector(theta.data_ptr(), theta.stride(0))
        for index in (rowptr, dst, weight_index):
            _index(index, state)
        _check_float(weight, state, "weight")
        if (rowptr.numel() != state.size(1) + 1 or dst.numel() != weight.numel()
                or dst.numel() != weight_index.numel() or not weight.is_contiguous()
                or weight.dim() != 1):
            raise RuntimeError("invalid event topology geometry")
        args.out_rowptr, args.dst = rowptr.data_ptr(), dst.data_ptr()
        args.weight_index, args.weight = weight_index.data_ptr(), weight.data_ptr()
        args.n_edges = weight.numel()
        batch, n = state.shape
        args.n_neurons, args.batch = n, batch
        if delta is not None and (delta.numel() < batch * n or delta.dtype != torch.float32
                                  or not delta.is_contiguous() or delta.device != state.device):
            raise RuntimeError("delta workspace must hold B*N float32")
        if pending is not None and (
                pending.dim() != 2 or pending.size(0) != 2 or pending.size(1) < batch * n
                or pending.dtype != torch.float32 or not pending.is_contiguous()
                or pending.device != state.device):
            raise RuntimeError("pending buffers must hold B*N float32 on the state's device")
        if activity is not None and (
                activity.dtype != torch.int64 or not activity.is_contiguous()
                or activity.numel() < EVENT_ACTIVITY_SLOTS * EVENT_ACTIVITY_STRIDE
                or activity.device != state.device):
            raise RuntimeError("activity must hold EVENT_ACTIVITY_SLOTS * "
                               "EVENT_ACTIVITY_STRIDE int64 counters on the state's device")
        self.args, self._ref = args, ctypes.byref(args)
        self.batch, self.n, self.shape, self.device = batch, n, state.shape, state.device
        self.params = tuple(params)
        self._fixed = (theta, rowptr, dst, weight_index, weight, pending, activity, *self.params)
        self._addressed = (*self.params, theta, rowptr, dst, weight_index, weight)
        self._pointers = tuple(map(_data_ptr, self._addressed))
        self._delta = delta
        self._pending = ((pending[0].data_ptr(), pending[1].data_ptr())
                         if pending is not None else None)
        self._activity = activity.data_ptr() if activity is not None else 0
        self._out_weight = (None, 0)
        self._current = (None, None)
        self._last = None     # (s', d', a', e', their words)

    def matches(self, state, params, theta, rowptr, dst, weight_index, weight, pending=None,
                activity=None) -> bool:
        given = (theta, rowptr, dst, weight_index, weight, pending, activity, *params)
        if len(given) != 13 or not all(map(is_, given, self._fixed)):
            return False
        last = self._last
        if (last is None or state is not last[0]) and state.shape != self.shape:
            return False
        return tuple(map(_data_ptr, self._addressed)) == self._pointers

    def __call__(self, state, dendrite, adaptation, emitted, current, drive, drive_scalar,
                 dendritic_drive, dendritic_scalar, *, parity=None, advance_only=False,
                 sample=False, out_weight=None) -> tuple:
        """One tick; drives are validated [B,N] views or None with a scalar."""
        last = self._last
        if (last is not None and state is last[0] and dendrite is last[1]
                and adaptation is last[2] and state.data_ptr() == last[4][0]
                and dendrite.data_ptr() == last[4][4] and adaptation.data_ptr() == last[4][8]):
            words = last[4]
        else:
            _check_state(state)
            if state.device != self.device:
                raise RuntimeError("all tensors must be on the state's CUDA device")
            if state.shape != self.shape:
                raise RuntimeError("state/current/drive shape mismatch")
            words = (_plane_words(state, state, "state") + (0.0,)
                     + _plane_words(dendrite, state, "dendrite") + (0.0,)
                     + _plane_words(adaptation, state, "adaptation") + (0.0,))
        if last is not None and emitted is last[3] and emitted.data_ptr() == last[5][0]:
            emitted_words = last[5]
        else:
            emitted_words = _plane_words(emitted, state, "emitted") + (0.0,)
        if current is not self._current[0] or current.data_ptr() != self._current[1][0]:
            _check_float(current, state, "current")
            if current.shape != state.shape:
                raise RuntimeError("state/current/drive shape mismatch")
            self._current = (current, (current.data_ptr(), current.stride(0), current.stride(1)))
        if out_weight is not self._out_weight[0]:
            if out_weight is not None and (
                    out_weight.dtype != torch.float32 or not out_weight.is_contiguous()
                    or out_weight.numel() != self.args.n_edges
                    or out_weight.device != state.device):
                raise RuntimeError("out_weight must be M contiguous float32 on the state's device")
            self._out_weight = (out_weight, out_weight.data_ptr() if out_weight is not None else 0)
        args = self.args
        _PLANES5.pack_into(args, _EVENT_IN, *words,
                           *_drive_words(drive, drive_scalar, state),
                           *_drive_words(dendritic_drive, dendritic_scalar, state))
        _CURRENT_EMITTED.pack_into(args, _EVENT_CURRENT, *self._current[1], *emitted_words)
        if parity is None:
            pending_in = pending_out = 0
        else:
            if self._pending is None:
                raise RuntimeError("this tick was prepared without pending buffers")
            pending_in, pending_out = self._pending[parity], self._pending[1 - parity]
            if advance_only:
                pending_out = 0
        if sample and not self._activity:
            raise RuntimeError("this tick was prepared without activity counters")
        delta = 0
        if parity is None or advance_only:
            if self._delta is None:       # a workspace of its own, made on first need
                self._delta = torch.empty(self.batch * self.n, dtype=torch.float32,
                                          device=self.device)
            delta = self._delta.data_ptr()
        _EVENT_TAIL.pack_into(args, _EVENT_TAIL_AT, delta, pending_in, pending_out,
                              self._out_weight[1], EVENT_ADVANCE_ONLY if advance_only else 0,
                              0, self._activity if sample else 0)
        batch, n = self.batch, self.n
        outs, base = _new_outputs(4, batch, n, self.device)
        size = 4 * n * batch
        out = (base, 1, batch, base + size, 1, batch, base + 2 * size, 1, batch,
               base + 3 * size, 1, batch)
        _OUTS4.pack_into(args, _EVENT_OUT, *out)
        _raise_on(self.lib.ns_dendritic_event(self._ref, current_stream(self.device)), self.lib)
        self._last = (outs[0], outs[1], outs[2], outs[3],
                      (out[0], 1, batch, 0.0, out[3], 1, batch, 0.0, out[6], 1, batch, 0.0),
                      (out[9], 1, batch, 0.0))
        return outs


class PreparedAccumulate:
    """``out += W @ source`` (ns_csr_spmm with accumulate) with every argument
    validated once: a source plane, float32 CSR weights with their row plan (or
    a column-panel plan) and the accumulated output, all fixed tensors (the PELS
    runtime's delta workspace and current).  ``matches`` says whether the given tensors are
    still those objects at those addresses; a call only launches."""

    def __init__(self, extension: "NativeExtension", source: torch.Tensor, rowptr, col, weight,
                 out: torch.Tensor, panels: "_PanelPlan | None" = None):
        _check_state(source)
        args = _SpmmArgs()
        args.source = _plane(source, source, "source")
        args.matrix = extension._csr(source, rowptr, col, weight, None, None)
        batch, n = source.shape
        args.n_neurons, args.batch = n, batch
        bounds = None
        if panels is not None:
            args.panels = ctypes.addressof(panels)
        else:
            bounds, blocks, block_edges = extension.plan_tensors(rowptr, batch)
            args.plan = _RowPlan(bounds.data_ptr(), blocks, block_edges, 0)
        _check_float(out, source, "accumulated output")
        if out.shape != source.shape:
            raise RuntimeError("the accumulated output must be [B,N]")
        args.out = _out(out)
        args.accumulate = 1
        self.lib, self.args, self._ref = extension.lib, args, ctypes.byref(args)
        self.device = source.device
        self._tensors = (source, rowptr, col, weight, out)
        self._pointers = tuple(t.data_ptr() for t in self._tensors)
        self._bounds, self.panels = bounds, panels

    def matches(self, source, rowptr, col, weight, out, panels=None) -> bool:
        given = (source, rowptr, col, weight, out)
        return (panels is self.panels and all(a is b for a, b in zip(given, self._tensors))
                and tuple(t.data_ptr() for t in given) == self._pointers)

    def __call__(self) -> None:
        _raise_on(self.lib.ns_csr_spmm(self._ref, current_stream(self.device)), self.lib)


@lru_cache(maxsize=1)
def load_native_extension(verbose: bool = False) -> NativeExtension:
    """The process-wide native extension (library loaded once, never rebuilt)."""
    return NativeExtension()
