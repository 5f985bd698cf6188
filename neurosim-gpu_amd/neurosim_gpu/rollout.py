"""Closed-loop multi-tick rollouts of the native matrix tick in one HIP graph.

A rollout owns two sets of neuron-major state planes and alternates between
them: tick i reads set i % 2 and writes set (i+1) % 2, so an even number of
ticks ends where it started and the captured graph can be replayed back to
back with no copy, no allocation and no host work per tick.  This is the
native counterpart of the reference's CUDA-graph rollout used by its drift
benchmark (benchmarks/precision_drift.py:74-143).
"""

from __future__ import annotations

import torch

from .native import NativeExtension, TickLauncher, new_planes


class MatrixRollout:
    """``ticks`` fused ticks of a NativeDendriticMatrixRuntime per ``run()``.

    Drives are fixed for the rollout (numbers or tensors broadcastable to
    [B, N]), and so are the weights: the captured ticks read the weight payload
    (or its slot-order copy) of construction time, so build a new rollout after
    changing the weights.  The runtime's current states seed the rollout;
    ``write_back()`` hands the rolled-out states back to the runtime.
    """

    def __init__(self, runtime, ticks: int, *, drive=0.0, dendritic_drive=0.0,
                 use_graph: bool = True) -> None:
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
        weight, scales, self.backend = runtime._weights()
        topology = runtime.topology
        panels = runtime._panel_plan(weight, scales) if runtime._panels is not None else None
        bands = runtime._band_plan(weight, scales) if runtime._bands is not None else None
        self._launch = TickLauncher(extension, runtime.state, runtime._parameters(),
                                    topology.in_rowptr, topology.in_col, weight, drive,
                                    dendritic_drive, *scales, panels=panels, bands=bands)
        self._sets = (tuple(new_planes(3, batch, n, runtime.state)),
                      tuple(new_planes(3, batch, n, runtime.state)))
        self.reset_from_runtime()
        self.graph = None
        if use_graph:
            self._capture()

    def _eager(self) -> None:
        for tick in range(self.ticks):
            self._launch(self._sets[tick % 2], self._sets[(tick + 1) % 2])

    def _capture(self) -> None:
        saved = [p.clone() for p in self._sets[0]]
        side = torch.cuda.Stream(device=self._sets[0][0].device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            self._launch(self._sets[0], self._sets[1])   # warm-up outside capture
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

    def run(self, repeats: int = 1) -> None:
        """Advance ``repeats * ticks`` ticks (asynchronous on the current stream)."""
        for _ in range(repeats):
            if self.graph is not None:
                self.graph.replay()
            else:
                self._eager()

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
