"""Closed-loop multi-tick rollouts of the native matrix tick in one HIP graph.

A rollout owns two sets of neuron-major state planes and alternates between
them: tick i reads set i % 2 and writes set (i+1) % 2, so an even number of
ticks ends where it started and the captured graph can be replayed back to
back with no copy, no allocation and no host work per tick.

Inputs can be staged per tick, as in the reference's CUDA-graph rollout of its
drift benchmark (benchmarks/precision_drift.py:74-143): a drive given as a
[ticks, b, n] tensor (b in {1, B}, n in {1, N}) is read one slice per tick,
slice t by tick t of every replay, straight from that tensor's memory.  The
caller refills it in place between replays (``stage``), so new inputs need no
new capture.
"""

from __future__ import annotations

import torch

from .native import NativeExtension, TickLauncher, drive_plane, new_planes


def _per_tick(value, ticks: int, batch: int, n: int, state: torch.Tensor, what: str):
    """None for a fixed drive, else the [ticks, B, N] broadcast view of a staged one."""
    if not isinstance(value, torch.Tensor) or value.dim() != 3:
        return None
    if value.device != state.device or value.dtype != torch.float32:
        raise ValueError(f"{what} must be float32 on the state's device")
    if value.shape[0] != ticks:
        raise ValueError(f"a per-tick {what} needs one slice per tick: [{ticks}, B|1, N|1]")
    try:
        return value.expand(ticks, batch, n)
    except RuntimeError as error:
        raise ValueError(f"each tick's {what} must broadcast to [batch, n_neurons]") from error


class MatrixRollout:
    """``ticks`` fused ticks of a NativeDendriticMatrixRuntime per ``run()``.

    ``drive`` and ``dendritic_drive`` are each a number, a tensor broadcastable
    to [B, N] (the same input every tick), or a [ticks, B|1, N|1] float32
    tensor on the state's device whose slice t drives tick t of each replay.
    A staged tensor is read in place: ``stage()`` (or any in-place write
    ordered before the replay on the stream) changes the next replay's inputs.
    The weights are those of construction time: the captured ticks read that
    weight payload (or its slot-order copy), which the rollout keeps alive, so
    build a new rollout to follow a weight change.  The runtime's current
    states seed the rollout; ``write_back()`` hands the rolled-out states back.
    ``trace=True`` also copies each tick's new somatic state into ``trace``
    ([ticks, B, N], overwritten by every replay or ``advance``), one device
    copy per tick inside the graph.
    """

    def __init__(self, runtime, ticks: int, *, drive=0.0, dendritic_drive=0.0,
                 use_graph: bool = True, trace: bool = False) -> None:
        if ticks <= 0 or ticks % 2:
            raise ValueError("ticks must be a positive even number")
        extension = runtime.extension
        if not isinstance(extension, NativeExtension):
            raise ValueError("rollouts need the native extension")
        batch, n = runtime.state.shape
        if batch == 0:
            raise ValueError("rollouts need at least one column")
        self.runtime = runtime
        self.ticks = ticks
        state = runtime.state
        staged = (_per_tick(drive, ticks, batch, n, state, "drive"),
                  _per_tick(dendritic_drive, ticks, batch, n, state, "dendritic drive"))
        # The tensors a staged drive is read from (kept alive with the graph).
        self.inputs = (drive if staged[0] is not None else None,
                       dendritic_drive if staged[1] is not None else None)
        fixed = [0.0 if s is not None else v for s, v in zip(staged, (drive, dendritic_drive))]
        weight, scales, self.backend = runtime._weights()
        topology = runtime.topology
        panels = (runtime._panel_plan(weight, scales, reuse=True)
                  if runtime._panels is not None else None)
        bands = runtime._band_plan(weight, scales) if runtime._bands is not None else None
        self._launch = TickLauncher(extension, state, runtime._parameters(),
                                    topology.in_rowptr, topology.in_col, weight, fixed[0],
                                    fixed[1], *scales, panels=panels, bands=bands)
        # Per tick: the drive planes it reads (None: the fixed one).
        self._drives = [tuple(drive_plane(s[t], state) if s is not None else None for s in staged)
                        for t in range(ticks)]
        if staged == (None, None):
            self._drives = [None] * ticks
        self._sets = (tuple(new_planes(3, batch, n, state)),
                      tuple(new_planes(3, batch, n, state)))
        self.trace = (torch.empty(ticks, batch, n, dtype=torch.float32, device=state.device)
                      if trace else None)
        self.reset_from_runtime()
        self.graph = None
        if use_graph:
            self._capture()

    def _eager(self, count: int | None = None) -> None:
        count = self.ticks if count is None else count
        for tick in range(count):
            self._launch(self._sets[tick % 2], self._sets[(tick + 1) % 2],
                         drives=self._drives[tick])
            if self.trace is not None:
                self.trace[tick].copy_(self._sets[(tick + 1) % 2][0])

    def _capture(self) -> None:
        saved = [p.clone() for p in self._sets[0]]
        side = torch.cuda.Stream(device=self._sets[0][0].device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._eager(2)                       # warm-up outside capture
        torch.cuda.current_stream().wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self._eager()
        for plane, value in zip(self._sets[0], saved):
            plane.copy_(value)

    def reset_from_runtime(self) -> None:
        """Seed the rollout with the runtime's current three states."""
        rt = self.runtime
        for plane, value in zip(self._sets[0], (rt.state, rt.dendritic_state, rt.adaptation_state)):
            plane.copy_(value)

    def stage(self, drive: torch.Tensor | None = None,
              dendritic_drive: torch.Tensor | None = None) -> None:
        """Copy new per-tick inputs into the staged drive tensors (on the
        current stream, so the next replay reads them)."""
        for value, target, what in ((drive, self.inputs[0], "drive"),
                                    (dendritic_drive, self.inputs[1], "dendritic drive")):
            if value is None:
                continue
            if target is None:
                raise ValueError(f"this rollout's {what} is not staged per tick")
            target.copy_(value)

    def run(self, repeats: int = 1) -> None:
        """Advance ``repeats * ticks`` ticks (asynchronous on the current stream)."""
        for _ in range(repeats):
            if self.graph is not None:
                self.graph.replay()
            else:
                self._eager()

    def advance(self, count: int) -> None:
        """Advance ``count`` ticks: a replay for a whole chunk, else ``count``
        eager ticks reading the first ``count`` staged slices."""
        if not 0 <= count <= self.ticks:
            raise ValueError(f"count must be in [0, {self.ticks}]")
        if count == self.ticks:
            self.run()
            return
        self._eager(count)
        if count % 2:                            # an odd count ends in the other set
            for plane, value in zip(self._sets[0], self._sets[1]):
                plane.copy_(value)

    @property
    def state(self) -> torch.Tensor:
        return self._sets[0][0]

    @property
    def dendritic_state(self) -> torch.Tensor:
        return self._sets[0][1]

    @property
    def adaptation_state(self) -> torch.Tensor:
        return self._sets[0][2]

    def write_back(self) -> None:
        """Give the runtime fresh copies of the rolled-out states."""
        rt = self.runtime
        rt.state, rt.dendritic_state, rt.adaptation_state = (p.clone() for p in self._sets[0])
        rt.last_backend = self.backend
