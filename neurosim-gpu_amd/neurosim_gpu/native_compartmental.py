"""Native (gfx950 HIP) dendritic runtimes with explicit reference fallbacks.

API of the reference's native_compartmental module
(src/neurosim_gpu/native_compartmental.py:13-177):

* NativeDendriticMatrixRuntime -- the fused tick: CSR gather-product over the
  B columns plus the three-state update, with fp32 / fp16 / fp8 e4m3 / nvfp4
  weights decoded in-kernel and accumulated in float32 (one launch on row
  blocks or bands; on column panels, a panel launch and a combine launch).
* NativeDendriticPELSRuntime -- advance + emission threshold, then the
  emitters' out-edge scatter into the persistent current: one launch per tick
  (through pending buffers), or the reference's two (``one_launch=False``).

Matrix ticks that need autograd (any tensor with requires_grad under grad
mode) run the same native forward with a native backward
(ns_dendritic_step_backward; ``last_backend`` "native-autograd"), where the
reference falls back to its torch step.  PELS ticks that need autograd or
statistics run the PyTorch reference step and say so in ``last_backend``
("reference-autograd" / "reference-stats"); reduced weight storage is
inference-only.  The native library must be present: a missing
library raises at construction, nothing falls back silently.
"""

from __future__ import annotations

import warnings
from types import SimpleNamespace

import torch

from .compartmental import DendriticDynamics, DendriticMatrixRuntime, DendriticPELSRuntime
from .native import (BAND_WIDTH, EVENT_ACTIVITY_SLOTS, EVENT_ACTIVITY_STRIDE, BandLayout,
                     NativeExtension, PanelLayout, PreparedAccumulate, PreparedBackward,
                     PreparedEvent, PreparedTick, encode_weights,
                     load_native_extension, panel_geometry)
from .topology import SparseTopology


def _capture_error(what: str) -> RuntimeError:
    """A derived weight array missing while the stream is being captured: built
    here, it would be filled only when the graph replays, and the eager ticks
    after the capture would read it unfilled."""
    return RuntimeError(f"the {what} of this weight version is built on an eager tick; "
                        "run one eager tick before capturing ticks into a graph")


def _require_gpu_float32(initial_state: torch.Tensor) -> None:
    if initial_state.device.type != "cuda" or initial_state.dtype != torch.float32:
        raise ValueError("native compartment runtime requires CUDA float32")


class _NativeCompartments:
    def _init_native(self, initial_state: torch.Tensor, extension) -> None:
        _require_gpu_float32(initial_state)
        self.extension = extension if extension is not None else load_native_extension()
        self.last_backend = "unstepped"
        # The eager tick's launch arguments, validated once and reused while the
        # parameters, weights and layout stay the same objects (PreparedTick,
        # PreparedEvent), and those of a tick recorded for autograd.
        self._prepared = self._prepared_recorded = None
        # The backward's prepared launch, shared by the ticks recorded here (a
        # one-element holder, since the backward runs after the forward returns).
        self._prepared_backward = [None]

    def _parameters(self) -> list[torch.Tensor]:
        model = self.compartment_dynamics
        return [model.soma.alpha, model.soma.gain, model.dendrite_decay,
                model.adaptation_decay, model.coupling, model.adaptation_strength]

    def _needs_autograd(self, drive, dendritic_drive) -> bool:
        if not torch.is_grad_enabled():
            return False
        values = [self.state, self.dendritic_state, self.adaptation_state,
                  self.topology.weight, self.topology.in_weight, *self._parameters(),
                  drive, dendritic_drive]
        values += self._event_tensors()
        return any(isinstance(v, torch.Tensor) and v.requires_grad for v in values)

    def _event_tensors(self) -> list[torch.Tensor]:
        return []

    def _drive(self, value) -> tuple[torch.Tensor | None, float]:
        """(broadcast [B,N] view, 0.0) for tensors, (None, value) for numbers."""
        if not isinstance(value, torch.Tensor):
            return None, float(value)
        if value.device != self.state.device or value.dtype != self.state.dtype:
            raise ValueError("drive must match state device and dtype")
        try:
            return value.expand_as(self.state), 0.0
        except RuntimeError as error:
            raise ValueError("drive must broadcast to [batch, n_neurons]") from error

    def _native_spmm(self, source: torch.Tensor) -> torch.Tensor:
        """W @ source on the device (float32 weights), neuron-major output."""
        topology = self.topology
        return self.extension.csr_spmm(source.detach(), topology.in_rowptr, topology.in_col,
                                       topology.in_weight.detach())


def _weight_key(weight: torch.Tensor) -> tuple:
    """Identity and in-place version of a weight tensor, for caches derived from
    it.  A cache that stores this key also holds the tensor, so the identity
    cannot pass to another tensor while the cache refers to it.  A tensor made
    under torch.inference_mode has no version counter (PyTorch tracks none for
    them); its key is its identity alone."""
    return (id(weight), None if torch.is_inference(weight) else weight._version)


class SourceMajorWeights:
    """Source-major copy of the CSR weights (``weight[out_weight_index]``) for
    kernels that walk out-edges: the backward's transposed product and the PELS
    scatter.

    Reading CSR-order weights along out-edges is one random gather per edge.
    The copy costs one such gather and is then streamed, so it is built on the
    ``build_after``-th request for one weight version: the second for the
    backward (backpropagation through several ticks reuses a version; a single
    backward keeps the direct gather), the first for PELS ticks.  A version is
    (tensor, in-place version counter, optional caller key), so an optimizer
    step on the weights, in place or into a new tensor, invalidates the copy.
    ``enabled`` turns the copy off.
    """

    def __init__(self, build_after: int = 2) -> None:
        self.enabled = True
        self.build_after = build_after
        self._key = None
        self._source: torch.Tensor | None = None
        self._seen = 0
        self._values: torch.Tensor | None = None

    def get(self, weight: torch.Tensor, out_weight_index: torch.Tensor,
            version=None) -> torch.Tensor | None:
        """The copy for ``weight``, or None while it is not (yet) built.
        ``version`` adds to the key (e.g. a topology weight version)."""
        if not self.enabled:
            return None
        key = (_weight_key(weight), version)
        if key != self._key or self._source is not weight:
            self._key, self._source, self._seen, self._values = key, weight, 0, None
        self._seen += 1
        if self._seen >= self.build_after and self._values is None:
            if torch.cuda.is_current_stream_capturing():
                return None          # built by an eager request (see _capture_error)
            with torch.no_grad():
                self._values = torch.index_select(weight.detach(), 0, out_weight_index)
        return self._values


class TransposedPanels:
    """Column-panel layout of the transposed matrix, for the backward's W^T @ g.

    Its rows are the sources (``out_rowptr``, ``dst``: the source-major view)
    and its slots name CSR positions through ``out_weight_index``.  On the
    first request for a weight version the plan is indexed (NS_PANEL_INDEXED):
    the kernel reads each slot's weight from the CSR-order weights through
    that position, so a weight version used once (an optimizer step before
    every backward) needs no copy.  The slot-order copy, one random read per
    edge, is made on the second request (backpropagation through several
    ticks, or repeated passes on fixed weights), and streamed after that.
    Built on the host from the source-major view (set-up only, like the
    forward's layout)."""

    def __init__(self, topology, batch: int, device, *, max_panel_width: int | None = None) -> None:
        view = SimpleNamespace(n_neurons=topology.n_neurons, n_edges=topology.n_edges,
                               in_rowptr=topology.out_rowptr, in_col=topology.dst)
        self.layout = PanelLayout(view, batch, device, max_panel_width=max_panel_width,
                                  combine_launch=True)
        perm = self.layout.perm
        owi = topology.out_weight_index.to(device=device, dtype=torch.int32)
        self.layout.perm = torch.where(perm >= 0, owi[perm.clamp(min=0).long()],
                                       perm).to(torch.int32).contiguous()
        self._key, self._source, self._seen = None, None, 0
        self._indexed = None

    def plan(self, weight: torch.Tensor):
        """The plan struct for ``weight`` (float32, CSR order): on the first
        request for a weight version the indexed plan, whose slots carry CSR
        edge numbers so the kernel reads ``weight`` in place; from the second on,
        ``weight`` gathered into slot order once."""
        key = _weight_key(weight)
        if key != self._key or self._source is not weight:
            self._key, self._source, self._seen = key, weight, 0
        self._seen += 1
        if self._seen < 2:
            if self._indexed is None:
                self._indexed = self.layout.indexed_plan_struct()
            return self._indexed
        slots, _ = self.layout.slot_weights(key, weight, None)
        return self.layout.plan_struct(slots, None)


class _NativeTick(torch.autograd.Function):
    """One float32 fused tick (ns_dendritic_step) whose backward is native too
    (ns_dendritic_step_backward): gradients of the states, tensor drives, the
    six parameter vectors and the CSR weights, as autograd through the
    reference's torch step would give them."""

    @staticmethod
    def forward(ctx, info, state, dendrite, adaptation, weight, drive, dendritic_drive, *params):
        _, _, us, vs, tick, _, _, _ = info
        # The launch arguments were prepared (and validated) for this weight, plan
        # and these parameters; j = W @ s is kept for the backward, which then
        # needs no product of its own.
        *outs, current = tick(state, dendrite, adaptation, drive, us, dendritic_drive, vs,
                              current=True)
        ctx.current = current
        ctx.info = info
        ctx.has_drive = (drive is not None, dendritic_drive is not None)
        saved = [state, dendrite, adaptation, weight, *params]
        saved += [t for t in (drive, dendritic_drive) if t is not None]
        ctx.save_for_backward(*saved)
        ctx.set_materialize_grads(False)
        return tuple(outs)

    @staticmethod
    def backward(ctx, grad_state, grad_dendrite, grad_adaptation):
        extension, topology, us, vs, _, source_major, transposed, cache = ctx.info
        saved = list(ctx.saved_tensors)
        state, dendrite, adaptation, weight = saved[:4]
        params = saved[4:10]
        rest = iter(saved[10:])
        drive = next(rest) if ctx.has_drive[0] else None
        dendritic_drive = next(rest) if ctx.has_drive[1] else None
        needs = ctx.needs_input_grad
        panels = transposed.plan(weight) if transposed is not None else None
        out_weight = (None if panels is not None
                      else source_major.get(weight, topology.out_weight_index))
        fixed = (topology.in_rowptr, topology.in_col, weight, topology.out_rowptr,
                 topology.dst, topology.out_weight_index)
        prepared = cache[0]
        if prepared is None or not prepared.matches(state, params, *fixed):
            prepared = cache[0] = PreparedBackward(extension, state, params, *fixed)
        (d_state, d_dendrite, d_adaptation, d_drive, d_dendritic, d_weight,
         d_params) = prepared(
            state, dendrite, adaptation, drive, us, dendritic_drive, vs, grad_state,
            grad_dendrite, grad_adaptation, need_drive=bool(needs[5]),
            need_dendritic=bool(needs[6]), need_weight=bool(needs[4]),
            need_params=tuple(bool(x) for x in needs[7:13]),
            out_weight=out_weight, current=ctx.current, transposed_panels=panels)
        ctx.current = None
        return (None, d_state if needs[1] else None, d_dendrite if needs[2] else None,
                d_adaptation if needs[3] else None, d_weight, d_drive, d_dendritic, *d_params)


# "auto" takes column panels (batch 1-2) when the graph has at least
# PANEL_AUTO_MIN_SEGMENT edges per (row, panel) on average and at least
# PANEL_AUTO_MIN_EDGES edges; sparser or smaller graphs run faster on row
# blocks.  Measured (us per tick, rows / panels): N=50k M=1M B=1 8.2 / 8.8;
# N=166k M=2M B=1 15.0 / 13.0, B=2 20.5 / 22.5; N=400k M=4M B=1 26.8 / 28.6,
# B=2 39.8 / 76.4; N=400k M=16M B=2 121.8 / 82.1; N=166k M=25M B=1 117 / 33.
PANEL_AUTO_MIN_SEGMENT = 2.0
PANEL_AUTO_MIN_EDGES = 2_000_000


def panels_pay_off(topology, batch: int) -> bool:
    """Whether column panels beat row blocks for this graph and batch (see above)."""
    width, _ = panel_geometry(batch)
    n = max(topology.n_neurons, 1)
    panels = -(-n // (width & ~3))
    return (topology.n_edges >= PANEL_AUTO_MIN_EDGES
            and topology.n_edges >= PANEL_AUTO_MIN_SEGMENT * panels * n)


# Fewest bytes of one workgroup's column tile of the state (16 columns when the
# batch is a multiple of 16, else 8 or 4) for which "auto" picks the band kernel,
# one XCD's L2.  Measured, us per tick (rows / bands), 20 edges per neuron, fp32:
# B=8: N=50k (1.6 MB) 14.7 / 17.2, N=131k (4 MB) 36.5 / 29.5, N=262k 75.0 / 46.3,
# N=524k 173.7 / 89.0; B=16: N=65k (4 MB) 46.4 / 29.0, N=131k 81.9 / 41.4,
# N=262k 152.8 / 66.5; N=1M, M=100M, fp8: B=8 1603 / 658, B=16 1933 / 855.
BAND_AUTO_MIN_TILE_BYTES = 4 << 20


def band_tile_columns(batch: int) -> int:
    """State columns per band workgroup: 16, or 8 for an odd multiple of 8, or 4
    for an odd multiple of 4."""
    return 16 if batch % 16 == 0 else 8 if batch % 8 == 0 else 4


def default_band_steps(batch: int) -> int:
    """Steps per register block of the band tick: 8 for 8- and 4-column tiles,
    whose gathers need fewer registers (N=1M, M=100M, fp8, us per tick at 8 / 4
    steps: B=8 579 / 590, B=4 515 / 537), 4 for 16 columns (8 steps exceed the
    registers of 16 wavefronts per compute unit and spill)."""
    return 4 if band_tile_columns(batch) == 16 else 8


def bands_pay_off(n_neurons: int, batch: int) -> bool:
    """Whether "auto" picks the band kernel for this state size."""
    return (batch > 0 and batch % 4 == 0
            and n_neurons * band_tile_columns(batch) * 4 >= BAND_AUTO_MIN_TILE_BYTES)


class NativeDendriticMatrixRuntime(_NativeCompartments, DendriticMatrixRuntime):
    """One HIP launch per tick for CSR propagation plus all three neuron states.

    States, parameters, drives and accumulation are float32 on the GPU.
    ``weight_dtype=torch.float16`` or ``weight_format='fp8'|'nvfp4'`` stores
    the CSR weights compressed (re-encoded whenever topology.weight_version
    changes) and decodes them in-kernel before each float32 multiply.
    Returned states stay valid after later ticks (every tick allocates fresh
    outputs).  ``threads_per_row`` is accepted for compatibility.

    ``kernel`` picks the tick kernel: "panels" stages column panels of the
    state in LDS and streams a panel-sorted copy of the graph (batch 1 or 2;
    built once, at construction), "bands" streams a band-sorted copy of the
    graph whose gathers stay within an L2-sized band of sources at a time
    (batch a multiple of 4; built once), "rows" streams the CSR as is and
    gathers the state from cache.  "auto" uses panels when the batch allows
    and the graph is dense enough for them (``panels_pay_off``), bands when
    the batch is a multiple of 4 and a workgroup's column tile of the state
    (16, 8 or 4 columns) is at least ``BAND_AUTO_MIN_TILE_BYTES`` (``bands_pay_off``),
    rows otherwise.  ``panel_width`` caps
    the neurons per panel (default: what LDS holds) and ``panel_tiles`` sets
    the workgroups per panel (default: compute units / panels).
    ``panel_pairs`` builds the pair layout (``NS_PANEL_PAIRS``: every row at least
    two lanes, edges of one 16-edge weight block in slot pairs), whose NVFP4
    slots carry one block-scale byte per pair instead of per slot; the default
    uses it for NVFP4 weights only.
    ``band_width`` sets the sources per band (default ``BAND_WIDTH``),
    ``band_rows`` the destination rows per band workgroup (default: one
    workgroup per compute unit, ``default_band_rows``) and ``band_steps`` the
    register block (2, 4 or 8 steps; default ``default_band_steps``; 8 steps
    with 16 columns per workgroup spill registers and run about 3x slower).
    """

    def __init__(self, topology: SparseTopology, dynamics: DendriticDynamics,
                 initial_state: torch.Tensor, *, threads_per_row: int | None = None,
                 extension=None, weight_dtype: torch.dtype = torch.float32,
                 weight_format: str | None = None, kernel: str = "auto",
                 panel_width: int | None = None, panel_tiles: int | None = None,
                 band_width: int | None = None, band_rows: int | None = None,
                 band_steps: int | None = None, panel_pairs: bool | None = None) -> None:
        if kernel not in ("auto", "rows", "panels", "bands"):
            raise ValueError("kernel must be 'auto', 'rows', 'panels' or 'bands'")
        if threads_per_row not in (None, 8, 16, 32):
            raise ValueError("threads_per_row must be 8, 16, 32 or None")
        _require_gpu_float32(initial_state)
        if weight_dtype not in (torch.float32, torch.float16):
            raise ValueError("weight_dtype must be torch.float32 or torch.float16")
        if weight_format not in (None, "fp8", "nvfp4"):
            raise ValueError("weight_format must be None, 'fp8' or 'nvfp4'")
        if weight_format is not None and weight_dtype != torch.float32:
            raise ValueError("weight_format and non-default weight_dtype conflict")
        super().__init__(topology, dynamics, initial_state)
        degree = topology.n_edges / max(topology.n_neurons, 1)
        self.threads_per_row = threads_per_row or (8 if degree <= 16 else 16 if degree <= 48 else 32)
        self._init_native(initial_state, extension)
        self.weight_dtype = weight_dtype
        self.weight_format = weight_format
        self._invalidate_precision_cache()
        batch = initial_state.shape[0]
        native = isinstance(self.extension, NativeExtension)
        if kernel == "panels" and (batch not in (1, 2) or not native):
            raise ValueError("the panel kernel needs batch 1 or 2 and the native extension")
        if kernel == "bands" and (batch % 4 or batch == 0 or not native):
            raise ValueError("the band kernel needs a batch that is a multiple of 4 and the "
                             "native extension")
        use_panels = kernel == "panels" or (kernel == "auto" and batch in (1, 2) and native
                                            and panels_pay_off(topology, batch))
        use_bands = kernel == "bands" or (
            kernel == "auto" and native and bands_pay_off(topology.n_neurons, batch))
        self.kernel = "panels" if use_panels else "bands" if use_bands else "rows"
        if self.kernel == "rows" and native and batch > 0:
            # A row plan reads rowptr on the host (a synchronisation): made now, not on
            # a tick that may be captured into a graph.
            self.extension.plan_tensors(topology.in_rowptr, batch)
        if panel_pairs is None:
            panel_pairs = weight_format == "nvfp4"
        self._panels = (PanelLayout(topology, batch, initial_state.device,
                                    tiles_per_panel=panel_tiles, max_panel_width=panel_width,
                                    pairs=panel_pairs)
                        if use_panels else None)
        self.source_major_weights = SourceMajorWeights()
        self._unversioned_warned = False
        # The first panel tick of a float32 weight version reads in_weight in place.
        self.indexed_first_tick = True
        self._indexed_key = self._indexed_source = self._indexed_struct = None
        self._recorded_key, self._recorded_source, self._recorded_seen = None, None, 0
        # The backward's transposed product on panels (False: the out-edge walk).
        self.transposed_panels_enabled = True
        self._transposed: TransposedPanels | None = None
        self._panel_width = panel_width
        self._bands = (BandLayout(topology, initial_state.device,
                                  band_width=band_width or BAND_WIDTH, block_rows=band_rows,
                                  block_steps=band_steps or default_band_steps(batch),
                                  batch=batch)
                       if use_bands else None)

    def _invalidate_precision_cache(self) -> None:
        self._packed_weight = None
        self._packed_weight_version = -1
        self._panel_struct = None
        self._panel_struct_key = None
        self._panel_struct_source = None

    def _recorded_panel_plan(self, weight: torch.Tensor):
        """Panel plan for a tick recorded for autograd, or None for the row kernel.

        The first recorded tick of a weight version runs the indexed panel plan,
        which reads ``weight`` (CSR order) itself, so a weight version seen once
        (an optimizer step every tick) costs no slot-order copy.  From the
        second recorded tick of one version on (backpropagation through time,
        repeated evaluation) the panel kernel runs on a slot-order copy of that
        version, built once.  A version is (tensor, in-place version counter),
        so an update of the weights is never missed.
        """
        if self._panels is None:
            return None
        key = ("recorded",) + _weight_key(weight)
        if key != self._recorded_key or self._recorded_source is not weight:
            self._recorded_key, self._recorded_source, self._recorded_seen = key, weight, 0
        self._recorded_seen += 1
        if self._recorded_seen < 2:
            return self._panels.indexed_plan_struct()
        return self._slot_plan(self._panels, key, weight.detach(), ())

    def _slot_plan(self, layout, key: tuple, weight: torch.Tensor, scales: tuple):
        """ctypes plan of ``layout`` over ``weight`` in slot order, rebuilt when
        ``key`` changes.  The weight payload is held with the plan, so the
        identity in the key stays its own."""
        if self._panel_struct_key != key:
            if torch.cuda.is_current_stream_capturing():
                if layout is self._panels and self.checkpoint_precision == "fp32":
                    # Float32 panels read in_weight in place until an eager tick copies it.
                    if self._indexed_struct is None:
                        self._indexed_struct = self._panels.indexed_plan_struct()
                    return self._indexed_struct
                raise _capture_error("slot-order weight copy")
            block = scales[0] if len(scales) == 2 else None
            slots, slot_scales = layout.slot_weights(key, weight, block)
            self._panel_struct = layout.plan_struct(slots, slot_scales)
            self._panel_struct_key = key
            self._panel_struct_source = weight
        return self._panel_struct

    def _band_plan(self, weight: torch.Tensor, scales: tuple):
        """ctypes band plan for this tick's weights (rebuilt when the weights change)."""
        self._warn_if_unversioned(weight)
        key = (self.topology.weight_version, self.checkpoint_precision) + _weight_key(weight)
        return self._slot_plan(self._bands, key, weight, scales)

    def _panel_plan(self, weight: torch.Tensor, scales: tuple, *, reuse: bool = False):
        """ctypes panel plan for this tick's weights (rebuilt when the weights
        change: a new topology weight version, or the payload replaced or
        modified in place).

        Float32 weights: the first tick of a weight version runs the indexed
        plan (NS_PANEL_INDEXED), which reads ``in_weight`` in CSR order, and the
        slot-order copy is built when the same version ticks again, so weights
        that change every tick (plasticity, training) never pay for a copy.
        ``reuse=True`` (a captured rollout, which replays one version many
        times) builds the copy at once.  ``indexed_first_tick = False`` turns
        the indexed first tick off."""
        self._warn_if_unversioned(weight)
        key = (self.topology.weight_version, self.checkpoint_precision) + _weight_key(weight)
        if (not reuse and self.indexed_first_tick and self.checkpoint_precision == "fp32"
                and self._panel_struct_key != key
                and (key != self._indexed_key or self._indexed_source is not weight)):
            self._indexed_key, self._indexed_source = key, weight
            if self._indexed_struct is None:
                self._indexed_struct = self._panels.indexed_plan_struct()
            return self._indexed_struct
        return self._slot_plan(self._panels, key, weight, scales)

    def _warn_if_unversioned(self, weight: torch.Tensor) -> None:
        """Warn once per runtime when float32 panel or band ticks run over an
        ``in_weight`` made under torch.inference_mode: PyTorch keeps no version
        counter for such a tensor, so an in-place edit of it is not seen by the
        slot-order copy these kernels read, while the reference's float32 tick
        reads ``in_weight`` afresh every tick.  (Reduced encodings follow the
        topology's weight version, as the reference's do.)"""
        if (self._unversioned_warned or self.checkpoint_precision != "fp32"
                or not torch.is_inference(weight)):
            return
        self._unversioned_warned = True
        warnings.warn(
            "in_weight was created under torch.inference_mode and has no version counter: "
            f"the {self.kernel} tick reads a slot-order copy of it, so after editing "
            "in_weight in place call topology.mark_weights_mutated_() (or "
            "apply_source_weights_) before the next step", RuntimeWarning, stacklevel=4)

    @property
    def checkpoint_precision(self) -> str:
        if self.weight_format is not None:
            return self.weight_format
        return "fp16" if self.weight_dtype == torch.float16 else "fp32"

    @property
    def precision_execution(self) -> str:
        return f"cuda-fused-{self.checkpoint_precision}-weights-fp32-fma"

    @property
    def weight_storage_bytes(self) -> int:
        """Logical inference payload in bytes, excluding the original topology."""
        edges = self.topology.n_edges
        if self.weight_format == "nvfp4":
            return (edges + 1) // 2 + (edges + 15) // 16 + 4
        if self.weight_format == "fp8":
            return edges + 4
        return edges * (2 if self.weight_dtype == torch.float16 else 4)

    def _weights(self) -> tuple[torch.Tensor, tuple, str]:
        """(weight payload, scale arguments, backend label) for this tick."""
        weight = self.topology.in_weight
        if self.weight_format is None and self.weight_dtype == torch.float32:
            return weight, (), "native"
        if self._packed_weight_version != self.topology.weight_version:
            if torch.cuda.is_current_stream_capturing():
                raise _capture_error(f"{self.weight_format or 'fp16'} weight payload")
            with torch.no_grad():
                if self.weight_format is None:
                    self._packed_weight = (weight.detach().to(torch.float16),)
                elif isinstance(self.extension, NativeExtension):
                    # On the device in two launches (ns_encode_weights), bit-exact
                    # with precision.encode_sparse_weights.
                    self._packed_weight = encode_weights(weight.detach(), self.weight_format)
                else:
                    from .precision import encode_sparse_weights
                    self._packed_weight = encode_sparse_weights(weight.detach(), self.weight_format)
            self._packed_weight_version = self.topology.weight_version
        payload, *scales = self._packed_weight
        return payload, tuple(scales), f"native-{self.weight_format or 'fp16'}-weight"

    def step(self, drive: torch.Tensor | float = 0.0, *,
             dendritic_drive: torch.Tensor | float = 0.0) -> torch.Tensor:
        if self._needs_autograd(drive, dendritic_drive):
            if self.weight_format is not None or self.weight_dtype == torch.float16:
                raise RuntimeError("native reduced-precision weight storage is inference-only")
            if not isinstance(self.extension, NativeExtension):
                self.last_backend = "reference-autograd"
                return super().step(drive, dendritic_drive=dendritic_drive)
            return self._autograd_step(drive, dendritic_drive)
        u, us = self._drive(drive)
        v, vs = self._drive(dendritic_drive)
        weight, scales, backend = self._weights()
        extra = {}
        if self._panels is not None:
            extra["panels"] = self._panel_plan(weight, scales)
        elif self._bands is not None:
            extra["bands"] = self._band_plan(weight, scales)
        topology, params = self.topology, self._parameters()
        if isinstance(self.extension, NativeExtension):
            tick = self._prepared
            if tick is None or not tick.matches(self.state, params, topology.in_rowptr,
                                                topology.in_col, weight, *scales, **extra):
                tick = self._prepared = PreparedTick(self.extension, self.state, params,
                                                     topology.in_rowptr, topology.in_col,
                                                     weight, *scales, **extra)
            outs = tick(self.state, self.dendritic_state, self.adaptation_state, u, us, v, vs)
        else:
            outs = self.extension.dendritic_step(
                self.state, self.dendritic_state, self.adaptation_state, params,
                topology.in_rowptr, topology.in_col, weight, u, us, v, vs,
                self.threads_per_row, *scales, **extra)
        self.state, self.dendritic_state, self.adaptation_state = outs
        self.last_backend = backend
        return self.state


    def _transposed_layout(self) -> TransposedPanels | None:
        """The transposed matrix's panel layout for the backward, built on the
        first recorded tick when the forward runs on panels (the graph is dense
        enough for them); None otherwise."""
        if self._panels is None or not self.transposed_panels_enabled:
            return None
        if self._transposed is None:
            self._transposed = TransposedPanels(self.topology, self.state.shape[0],
                                                self.state.device,
                                                max_panel_width=self._panel_width)
        return self._transposed

    def _autograd_step(self, drive, dendritic_drive) -> torch.Tensor:
        """A float32 tick recorded for autograd, native forward and backward."""
        u, us = self._drive(drive)
        v, vs = self._drive(dendritic_drive)
        topology, weight, params = self.topology, self.topology.in_weight, self._parameters()
        extra = {}
        plan = self._recorded_panel_plan(weight)
        if plan is not None:
            extra["panels"] = plan
        tick = self._prepared_recorded
        if tick is None or not tick.matches(self.state, params, topology.in_rowptr,
                                            topology.in_col, weight, **extra):
            tick = self._prepared_recorded = PreparedTick(
                self.extension, self.state, params, topology.in_rowptr, topology.in_col,
                weight, **extra)
        info = (self.extension, topology, us, vs, tick, self.source_major_weights,
                self._transposed_layout(), self._prepared_backward)
        self.state, self.dendritic_state, self.adaptation_state = _NativeTick.apply(
            info, self.state, self.dendritic_state, self.adaptation_state, weight, u, v,
            *params)
        self.last_backend = "native-autograd"
        return self.state


class NativeDendriticPELSRuntime(_NativeCompartments, DendriticPELSRuntime):
    """The PELS event tick on the device, by default in one HIP launch.

    The scan covers all B*N (neuron, column) pairs; only pairs with a nonzero
    delta walk their out-edges.  In the one-launch tick a wavefront advances
    its pairs and scatters their deltas itself.  Its scatter cannot add into
    the current that other wavefronts of the launch still read, so it adds
    into one of two pending buffers, and the next tick folds that buffer into
    the current as it reads it (j = current + pending, the same float32 sum
    either way).  Reading ``persistent_current`` folds the outstanding buffer
    first, so the attribute always holds W @ emitted as in the reference;
    assigning it discards the outstanding buffer.  The scatter streams a
    source-major copy of the weights (M floats, rebuilt when the weights
    change; ``source_major_weights.enabled = False`` gathers through
    ``out_weight_index`` instead).  Ticks captured in a HIP
    graph use fixed buffers: replays of an even number of ticks chain as they
    are, after an odd number read ``persistent_current`` (which folds) before
    the next replay.  ``one_launch=False`` runs
    the two-launch tick (advance, then scatter into the current).

    ``propagation="matrix"`` propagates the emitted deltas as the reference's
    matrix path does (runtime.py:233-235), current += W @ delta over the
    destination-major CSR, after an advance-only launch: no atomics, so it is
    the faster choice when many sources emit (theta = 0, driven onsets).
    ``propagation="auto"`` chooses between the two as the reference's PELS
    policy does (runtime.py:129-165): at every ``policy_interval``-th tick it
    compares the active out-edges (those of pairs with |s' - emitted| >= theta)
    with ``event_edge_fraction`` of all B*M edges, scattering below it and
    multiplying at or above it.  The count is taken on the device by the tick
    itself and read back without waiting for the GPU: a sampled tick's counters
    are copied to pinned host memory behind it on the stream, and a later policy
    tick whose copy has completed by then applies the decision (the reference
    counts on the host at the policy tick itself).  Until a first sample is in,
    the tick scatters; inside a HIP graph capture the path in force is kept.
    Float32 atomics make the scatter's summation order, and therefore the last
    bits of the current, run-dependent.  Statistics and autograd requests use
    the reference step.

    ``kernel`` picks the kernel of the matrix propagation's product: "rows"
    (CSR row blocks), "panels" (the column-panel kernel in product mode, batch
    1 or 2; its layout is built at construction) or "auto" (panels where they
    pay off, as for NativeDendriticMatrixRuntime).  The panel product reads the
    float32 weights through the slots' CSR edge numbers on the first matrix
    tick of a weight version and from a slot-order copy after that.
    """

    @property
    def precision_execution(self) -> str:
        return "cuda-fused-pels-fp32"

    def __init__(self, topology: SparseTopology, dynamics: DendriticDynamics,
                 initial_state: torch.Tensor, *, theta: float | torch.Tensor,
                 extension=None, one_launch: bool = True, propagation: str = "event",
                 event_edge_fraction: float = 0.12, policy_interval: int = 16,
                 kernel: str = "auto") -> None:
        _require_gpu_float32(initial_state)
        if propagation not in ("event", "matrix", "auto"):
            raise ValueError("native PELS propagation must be 'event', 'matrix' or 'auto'")
        if kernel not in ("auto", "rows", "panels"):
            raise ValueError("kernel must be 'auto', 'rows' or 'panels'")
        self._pending = None
        self.extension = extension if extension is not None else load_native_extension()
        native = isinstance(self.extension, NativeExtension)
        if propagation == "auto" and not (native and one_launch):
            raise ValueError("propagation='auto' needs the native extension and the "
                             "one-launch tick")
        super().__init__(topology, dynamics, initial_state, theta=theta, propagation=propagation,
                         event_edge_fraction=event_edge_fraction,
                         policy_interval=policy_interval)
        self._init_native(initial_state, self.extension)
        batch, n = initial_state.shape
        device = initial_state.device
        self.source_major_weights = SourceMajorWeights(build_after=1)
        self._delta = None
        self._accumulate = None     # the prepared current += W @ delta (matrix propagation)
        if native and one_launch:
            self._pending = torch.zeros(2, batch * n, dtype=torch.float32, device=device)
            self._parity = 0
        if not (native and one_launch) or propagation != "event":
            self._delta = torch.empty(batch * n, dtype=torch.float32, device=device)
        # The path the next tick takes; "auto" changes it from sampled activity.
        self._path = "matrix" if propagation == "matrix" else "event"
        self._activity = self._activity_host = self._sample = None
        if propagation == "auto":
            slots = EVENT_ACTIVITY_SLOTS * EVENT_ACTIVITY_STRIDE
            self._activity = torch.zeros(slots, dtype=torch.int64, device=device)
            self._activity_host = torch.zeros(slots, dtype=torch.int64, pin_memory=True)
        # The matrix propagation's product kernel and, for panels, its layout.
        if kernel == "panels" and (batch not in (1, 2) or not native):
            raise ValueError("the panel kernel needs batch 1 or 2 and the native extension")
        use_panels = native and propagation != "event" and (
            kernel == "panels" or (kernel == "auto" and batch in (1, 2)
                                   and panels_pay_off(topology, batch)))
        self.kernel = "panels" if use_panels else "rows"
        self._product_panels = PanelLayout(topology, batch, device) if use_panels else None
        self._product_key = self._product_source = None
        self._product_seen, self._product_struct, self._product_indexed = 0, None, None

    @property
    def selected_path(self) -> str:
        """The propagation the next native tick takes ("event" or "matrix")."""
        return self._path

    def _product_plan(self):
        """Panel plan of ``in_weight`` for the matrix propagation: the indexed plan
        (CSR edge numbers in the slots) on the first matrix tick of a weight
        version and inside graph captures until the copy exists, the slot-order
        copy from the second eager tick on.  A version is the topology's weight
        version and the tensor's identity and in-place version."""
        layout, weight = self._product_panels, self.topology.in_weight
        key = (self.topology.weight_version,) + _weight_key(weight)
        if key != self._product_key or self._product_source is not weight:
            self._product_key, self._product_source = key, weight
            self._product_seen, self._product_struct = 0, None
        self._product_seen += 1
        if self._product_struct is None:
            # Under graph capture the copy is not built: its gather would only run
            # at replay, while the eager ticks after the capture would read it.
            if self._product_seen < 2 or torch.cuda.is_current_stream_capturing():
                if self._product_indexed is None:
                    self._product_indexed = layout.indexed_plan_struct()
                return self._product_indexed
            slots, _ = layout.slot_weights(("pels",) + key, weight.detach(), None)
            self._product_struct = layout.plan_struct(slots, None)
        return self._product_struct

    def _policy_tick(self) -> bool:
        """For "auto": apply a finished sample at a policy tick and say whether
        this tick samples (counts its active out-edges)."""
        if self.propagation != "auto" or self._tick % self.policy_interval:
            return False
        if torch.cuda.is_current_stream_capturing():
            return False
        if self._sample is not None:
            if not self._sample.query():
                return False                 # the last sample is still on its way
            counts = self._activity_host.view(EVENT_ACTIVITY_SLOTS, EVENT_ACTIVITY_STRIDE)
            edges = int(counts[:, 0].sum())
            slots = max(self.topology.n_edges * self.state.shape[0], 1)
            self._path = "event" if edges / slots < self.event_edge_fraction else "matrix"
            self._sample = None
        return True

    @property
    def persistent_current(self) -> torch.Tensor:
        pending = self._pending
        if pending is not None and not self._current.requires_grad:
            # Between ticks at most one buffer is nonzero, so adding both adds it
            # exactly.  No host flag tracks which: replays of captured ticks
            # change the buffers without the host seeing them.
            batch, n = self._current.shape
            with torch.inference_mode():
                self._current.add_(pending.sum(0).view(n, batch).t())
                pending.zero_()
        return self._current

    @persistent_current.setter
    def persistent_current(self, value: torch.Tensor) -> None:
        if self._pending is not None:
            with torch.inference_mode():
                self._pending.zero_()
        self._current = value

    def _event_tensors(self) -> list[torch.Tensor]:
        return [self._current, self.emitted_state]

    def _source_major(self) -> torch.Tensor | None:
        """in_weight[out_weight_index], rebuilt when the weights change (a new
        tensor, an in-place edit, or a new topology weight version)."""
        if not isinstance(self.extension, NativeExtension):
            return None
        topology = self.topology
        return self.source_major_weights.get(topology.in_weight, topology.out_weight_index,
                                             topology.weight_version)

    def _initial_current(self) -> torch.Tensor:
        if torch.is_grad_enabled() and (self.emitted_state.requires_grad
                                        or self.topology.in_weight.requires_grad):
            return super()._initial_current()
        return self._native_spmm(self.emitted_state)

    def _refresh_current(self) -> None:
        if self._weight_version != self.topology.weight_version:
            if torch.is_grad_enabled() and (self.emitted_state.requires_grad
                                            or self.topology.in_weight.requires_grad):
                self.persistent_current = self._propagate(self.emitted_state).contiguous()
            else:
                self.persistent_current = self._native_spmm(self.emitted_state)
            self._weight_version = self.topology.weight_version

    def step(self, drive: torch.Tensor | float = 0.0, *,
             dendritic_drive: torch.Tensor | float = 0.0, collect_stats: bool = False):
        if collect_stats or self._needs_autograd(drive, dendritic_drive):
            self.last_backend = "reference-stats" if collect_stats else "reference-autograd"
            return super().step(drive, dendritic_drive=dendritic_drive,
                                collect_stats=collect_stats)
        u, us = self._drive(drive)
        v, vs = self._drive(dendritic_drive)
        self._refresh_current()
        # The tick updates the current in place, one element per (column,
        # neuron): an assigned view (expanded, strided) is replaced by a dense
        # copy first, as in the reference (native_compartmental.py:164).  The
        # pending buffers are separate, so nothing outstanding is lost.
        if not self._current.is_contiguous():
            self._current = self._current.contiguous()
        native = isinstance(self.extension, NativeExtension)
        sample = self._policy_tick()
        matrix = native and self._path == "matrix"
        out_weight = self._source_major() if not matrix else None
        topology, params = self.topology, self._parameters()
        if native:
            # One launch with pending buffers: pending[parity] holds the last tick's
            # scatter (or zeros) and the other is zero; the advance-only form (matrix
            # propagation) folds pending[parity] and writes the deltas instead.
            tick = self._prepared
            fixed = (self.theta, topology.out_rowptr, topology.dst, topology.out_weight_index,
                     topology.in_weight)
            if tick is None or not tick.matches(self.state, params, *fixed,
                                                pending=self._pending, activity=self._activity):
                tick = self._prepared = PreparedEvent(self.extension, self.state, params, *fixed,
                                                      delta=self._delta, pending=self._pending,
                                                      activity=self._activity)
            outs = tick(self.state, self.dendritic_state, self.adaptation_state,
                        self.emitted_state, self._current, u, us, v, vs,
                        parity=self._parity if self._pending is not None else None,
                        advance_only=matrix, sample=sample, out_weight=out_weight)
        else:
            extra = {"out_weight": out_weight} if out_weight is not None else {}
            outs = self.extension.dendritic_event(
                self.state, self.dendritic_state, self.adaptation_state, params,
                self._current, self.emitted_state, self.theta, topology.out_rowptr,
                topology.dst, topology.out_weight_index, topology.in_weight, u, us, v, vs,
                **extra)
        self.state, self.dendritic_state, self.adaptation_state, self.emitted_state = outs
        if matrix:
            # current += W @ delta over the destination-major CSR: the matrix
            # propagation of the emitted deltas (entry n*B + b of the workspace).
            panels = self._product_plan() if self._product_panels is not None else None
            product = self._accumulate
            if product is None or not product.matches(product._tensors[0], topology.in_rowptr,
                                                      topology.in_col, topology.in_weight,
                                                      self._current, panels):
                batch, n = self.state.shape
                delta = torch.as_strided(self._delta, (batch, n), (1, batch))
                product = self._accumulate = PreparedAccumulate(
                    self.extension, delta, topology.in_rowptr, topology.in_col,
                    topology.in_weight, self._current, panels)
            product()
        if sample:
            # The counters reach the host behind this tick; a later policy tick
            # reads them once the copy is done, then they start again from zero.
            self._activity_host.copy_(self._activity, non_blocking=True)
            self._sample = torch.cuda.Event()
            self._sample.record()
            self._activity.zero_()
        if self._pending is not None:
            self._parity ^= 1
        self._tick += 1
        self.last_backend = "native-matrix" if matrix else "native"
        return self.state
