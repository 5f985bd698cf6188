"""Long-horizon drift of the native matrix tick under each weight encoding.

The reference measures how far fixed-weight rollouts with fp16, fp8 and NVFP4
weights move away from the FP32 rollout of the same graph, model and inputs
over 100,000 ticks (benchmarks/precision_drift.py:23-71,231-282): three
scenarios, three seeds, inputs that change every tick, graph-replayed 32-tick
chunks and error statistics at a fixed schedule of sample ticks.

Here one ``DriftCase`` holds a native runtime and a ``MatrixRollout`` per weight
mode on one graph.  All of them read one pair of staged input buffers, which is
refilled before each chunk, so every mode sees the same inputs tick for tick.

    python -m neurosim_gpu.drift [--steps 100000] [--seeds 11 23 47] \\
        [--scenarios stable_drive slow_adaptation recurrent_stress] [--output drift.json]

As in the reference, the graph is drawn with the GPU's generator by default
(``--draw-device``).  At the protocol's size (1024 neurons, 16,384 candidate
edges) that generator draws the reference's own graphs (seeds 11, 23 and 47:
16,243, 16,273 and 16,267 edges), so the figures compare with its published
ones sample for sample.  ``--draw-device cpu`` draws with the CPU generator
instead, a graph that every machine reproduces.
"""

from __future__ import annotations

import argparse
import json
import math
import time
from pathlib import Path

import torch

from .compartmental import DendriticDynamics
from .dynamics import Dynamics
from .native_compartmental import NativeDendriticMatrixRuntime
from .rollout import MatrixRollout
from .topology import random_topology, topology_to

FIELDS = ("state", "dendritic_state", "adaptation_state")
MODES = ("fp32", "fp16", "fp8", "nvfp4")
# NativeDendriticMatrixRuntime keywords that store each mode's weights.
MODE_OPTIONS = {"fp32": {}, "fp16": {"weight_dtype": torch.float16},
                "fp8": {"weight_format": "fp8"}, "nvfp4": {"weight_format": "nvfp4"}}

_CONTRACTIVE = dict(weight_scale=0.15, alpha=0.72, gain=0.8, tau_dendrite=4.0,
                    tau_adaptation=20.0, coupling=0.45, adaptation_strength=0.15)
# Scenario parameters (reference precision_drift.py:27-37).  recurrent_stress
# has strong recurrent weights and gain: there the dynamics are chaotic and any
# rounding difference grows until the rollouts decorrelate.
SCENARIOS = {
    "stable_drive": dict(_CONTRACTIVE),
    "slow_adaptation": {**_CONTRACTIVE, "tau_adaptation": 5000.0, "adaptation_strength": 0.6},
    "recurrent_stress": {**_CONTRACTIVE, "weight_scale": 1.7, "alpha": 0.9, "gain": 1.3,
                         "tau_dendrite": 8.0, "tau_adaptation": 500.0, "coupling": 0.3,
                         "adaptation_strength": 0.6},
}
# slow_adaptation switches its inputs on for the first GATE_ON ticks of every GATE_PERIOD.
GATE_PERIOD, GATE_ON = 24_000, 8_000
THRESHOLDS = (1e-4, 1e-3, 1e-2, 1e-1)


def scenario_parameters(name: str) -> dict:
    if name not in SCENARIOS:
        raise ValueError(f"Unknown scenario: {name}")
    return dict(SCENARIOS[name])


def scenario_drives(name: str, first_tick: int, count: int, neurons: int, batch: int,
                    device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """Somatic and dendritic drives of ticks first_tick .. first_tick+count-1.

    Both are contiguous float32 [count, batch, neurons] tensors (reference
    precision_drift.py:51-65).  With phase = 0.039 n + 0.7 b:
    recurrent_stress drives the soma with the constant 0.13 + 0.08 sin(phase)
    and the dendrite with nothing; the other scenarios use
    0.20 + 0.05 sin(2 pi t / 257 + phase) and 0.025 + 0.015 sin(2 pi t / 503 + phase),
    and slow_adaptation adds 0.15 to the somatic drive and gates both inputs.
    """
    if name not in SCENARIOS:
        raise ValueError(f"Unknown scenario: {name}")
    f32 = dict(dtype=torch.float32, device=device)
    phase = (0.039 * torch.arange(neurons, **f32).view(1, 1, neurons)
             + 0.7 * torch.arange(batch, **f32).view(1, batch, 1))
    if name == "recurrent_stress":
        soma = (0.13 + 0.08 * torch.sin(phase)).expand(count, batch, neurons)
        return soma.contiguous(), torch.zeros(count, batch, neurons, **f32)
    t = torch.arange(first_tick, first_tick + count, **f32).view(count, 1, 1)
    soma = 0.20 + 0.05 * torch.sin(t * (2 * math.pi / 257) + phase)
    dendritic = 0.025 + 0.015 * torch.sin(t * (2 * math.pi / 503) + phase)
    if name == "slow_adaptation":
        on = ((t % GATE_PERIOD) < GATE_ON).to(torch.float32)
        soma, dendritic = on * (soma + 0.15), on * dendritic
    return soma.contiguous(), dendritic.contiguous()


def sample_ticks(steps: int, interval: int) -> list[int]:
    """Ticks at which the rollouts are compared (reference precision_drift.py:40-48).

    Every multiple of ``interval``, the first and last tick, 1, 2 and 5 times
    each power of ten, and the tick before, at and after every switch of the
    slow_adaptation input gate.
    """
    if steps < 1 or interval < 1:
        raise ValueError("steps and sample interval must be positive")
    ticks = {0, steps}
    ticks.update(range(interval, steps + 1, interval))
    scale = 1
    while scale <= steps:
        ticks.update(k * scale for k in (1, 2, 5) if k * scale <= steps)
        scale *= 10
    for start in range(0, steps + 1, GATE_PERIOD):
        for edge in (start, start + GATE_ON):
            ticks.update(t for t in (edge - 1, edge, edge + 1) if 0 <= t <= steps)
    return sorted(ticks)


def scenario_model(name: str, neurons: int, device="cpu") -> DendriticDynamics:
    p = scenario_parameters(name)
    soma = Dynamics(torch.full((neurons,), p["alpha"], device=device),
                    torch.full((neurons,), p["gain"], device=device))
    return DendriticDynamics.from_time_constants(
        soma, dt=1.0, tau_dendrite=p["tau_dendrite"], tau_adaptation=p["tau_adaptation"],
        coupling=p["coupling"], adaptation_strength=p["adaptation_strength"])


class DriftCase:
    """Native rollouts of one scenario and seed, one per weight mode.

    ``advance(count)`` stages the inputs of the next ``count`` ticks (at most
    ``chunk``) and advances every mode by that many ticks: one graph replay for
    a whole chunk, eager ticks otherwise.  ``states(mode)`` gives the mode's
    three [batch, neurons] states after ``tick`` ticks.  Unless ``topology`` is
    given, the graph is drawn with the generator of ``draw_device`` (default:
    ``device``).
    """

    def __init__(self, scenario: str, seed: int, *, neurons: int = 1024, edges: int = 16_384,
                 batch: int = 4, chunk: int = 32, device="cuda", draw_device=None,
                 modes=MODES, initial_state: float = 0.25, topology=None) -> None:
        if chunk < 2 or chunk % 2:
            raise ValueError("chunk must be an even number of ticks, at least 2")
        unknown = [mode for mode in modes if mode not in MODE_OPTIONS]
        if unknown or not modes:
            raise ValueError(f"modes must be drawn from {MODES}")
        params = scenario_parameters(scenario)
        self.scenario, self.seed, self.chunk = scenario, seed, chunk
        self.neurons, self.batch, self.modes = neurons, batch, tuple(modes)
        if topology is None:
            topology = random_topology(neurons, edges, seed=seed,
                                       device=device if draw_device is None else draw_device,
                                       weight_scale=params["weight_scale"])
        self.topology = topology_to(topology, device)
        self.device = self.topology.in_col.device
        model = scenario_model(scenario, neurons, self.device)
        initial = torch.full((batch, neurons), initial_state, device=self.device)
        self.inputs = tuple(torch.zeros(chunk, batch, neurons, device=self.device)
                            for _ in range(2))
        self.runtimes, self.rollouts = {}, {}
        for mode in self.modes:
            runtime = NativeDendriticMatrixRuntime(self.topology, model, initial.clone(),
                                                   **MODE_OPTIONS[mode])
            self.runtimes[mode] = runtime
            self.rollouts[mode] = MatrixRollout(runtime, chunk, drive=self.inputs[0],
                                                dendritic_drive=self.inputs[1])
        self.tick = 0

    def drives(self, count: int | None = None, device=None):
        """The inputs of the next ``count`` ticks (default: a chunk), float32 on ``device``."""
        return scenario_drives(self.scenario, self.tick, self.chunk if count is None else count,
                               self.neurons, self.batch, self.device if device is None else device)

    def advance(self, count: int, drives=None) -> None:
        """Advance every mode by ``count`` ticks.  ``drives`` overrides the staged
        inputs (a pair of [chunk, batch, neurons] tensors for ticks tick..)."""
        if not 0 < count <= self.chunk:
            raise ValueError(f"count must be in [1, {self.chunk}]")
        soma, dendritic = self.drives() if drives is None else drives
        self.inputs[0].copy_(soma)
        self.inputs[1].copy_(dendritic)
        for mode in self.modes:
            self.rollouts[mode].advance(count)
        self.tick += count

    def states(self, mode: str) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        rollout = self.rollouts[mode]
        return rollout.state, rollout.dendritic_state, rollout.adaptation_state

    def edges(self) -> int:
        return self.topology.n_edges


def error_statistics(candidate: torch.Tensor, baseline: torch.Tensor) -> dict:
    """Mean and RMS absolute error, max-abs error and bias of one state plane."""
    error = (candidate - baseline).double()
    return dict(mae=float(error.abs().mean()), rmse=float(error.square().mean().sqrt()),
                max_abs=float(error.abs().max()), bias=float(error.mean()))


def _window_rms(ticks: list[int], rmse: list[float], start: float, end: float) -> float:
    """RMS over [start, end] of the RMSE curve, its square taken linear between samples."""
    total = 0.0
    for (t0, e0), (t1, e1) in zip(zip(ticks, rmse), zip(ticks[1:], rmse[1:])):
        lo, hi = max(start, t0), min(end, t1)
        if hi <= lo:
            continue
        at = lambda t: e0 * e0 + (e1 * e1 - e0 * e0) * (t - t0) / (t1 - t0)
        total += 0.5 * (at(lo) + at(hi)) * (hi - lo)
    return math.sqrt(total / (end - start)) if end > start else 0.0


def summarize(ticks: list[int], samples: list[dict], steps: int) -> dict:
    """Per mode and state: peaks, early/late windows and first threshold crossings.

    ``samples[i][mode][field]`` holds the error statistics at ``ticks[i]``
    (reference precision_drift.py:202-227).
    """
    summary = {}
    for mode in samples[0]:
        summary[mode] = {}
        for field in FIELDS:
            rows = [sample[mode][field] for sample in samples]
            rmse = [row["rmse"] for row in rows]
            early = _window_rms(ticks, rmse, 0, 0.2 * steps)
            late = _window_rms(ticks, rmse, 0.8 * steps, steps)
            summary[mode][field] = dict(
                final=rows[-1], peak_sampled_rmse=max(rmse),
                peak_sampled_max_abs=max(row["max_abs"] for row in rows),
                early_20_percent_time_weighted_rmse=early,
                late_20_percent_time_weighted_rmse=late,
                late_to_early_rmse_ratio=late / early if early else None,
                first_sampled_rmse_threshold_tick={
                    str(level): next((t for t, e in zip(ticks, rmse) if e >= level), None)
                    for level in THRESHOLDS},
                first_sampled_max_abs_threshold_tick={
                    str(level): next((t for t, row in zip(ticks, rows)
                                      if row["max_abs"] >= level), None)
                    for level in THRESHOLDS})
    return summary


def state_bounds_hold(state, dendrite, adaptation) -> bool:
    """Finite states inside the model's ranges: soma and adaptation in [0, 1],
    dendrite in [-1, 1] (each is a convex mix of values in those ranges)."""
    planes = torch.stack((state, dendrite, adaptation))
    if not bool(torch.isfinite(planes).all()):
        return False
    return bool((state.min() >= 0) & (state.max() <= 1) & (adaptation.min() >= 0)
                & (adaptation.max() <= 1) & (dendrite.abs().max() <= 1))


def run_case(scenario: str, seed: int, *, steps: int = 100_000, sample_interval: int = 256,
             neurons: int = 1024, edges: int = 16_384, batch: int = 4, chunk: int = 32,
             device="cuda", draw_device=None, progress=None) -> dict:
    """One scenario and seed: every mode against the FP32 rollout, at the sample ticks."""
    case = DriftCase(scenario, seed, neurons=neurons, edges=edges, batch=batch, chunk=chunk,
                     device=device, draw_device=draw_device)
    ticks = sample_ticks(steps, sample_interval)
    samples = []
    started = time.perf_counter()
    for target in ticks:
        while case.tick < target:
            case.advance(min(chunk, target - case.tick))
        baseline = case.states("fp32")
        for mode in MODES:
            if not state_bounds_hold(*case.states(mode)):
                raise RuntimeError(f"{mode} state left its bounds or went non-finite at "
                                   f"tick {case.tick} ({scenario}, seed {seed})")
        samples.append({mode: {field: error_statistics(value, base) for field, value, base
                               in zip(FIELDS, case.states(mode), baseline)}
                        for mode in MODES[1:]})
        if progress and case.tick and case.tick % 10_000 == 0:
            progress(f"{scenario} seed={seed} tick={case.tick}/{steps}")
    torch.cuda.synchronize(case.device)
    return dict(scenario=scenario, seed=seed, parameters=scenario_parameters(scenario),
                neurons=neurons, candidate_edges=edges, edges=case.edges(), batch=batch,
                chunk=chunk, execution={mode: rt.precision_execution
                                        for mode, rt in case.runtimes.items()},
                backends={mode: case.rollouts[mode].backend for mode in MODES},
                summary=summarize(ticks, samples, steps),
                wall_seconds=time.perf_counter() - started)


def parser() -> argparse.ArgumentParser:
    cli = argparse.ArgumentParser(description=__doc__,
                                  formatter_class=argparse.RawDescriptionHelpFormatter)
    cli.add_argument("--steps", type=int, default=100_000)
    cli.add_argument("--neurons", type=int, default=1024)
    cli.add_argument("--edges", type=int, default=16_384)
    cli.add_argument("--batch", type=int, default=4)
    cli.add_argument("--chunk", type=int, default=32)
    cli.add_argument("--sample-interval", type=int, default=256)
    cli.add_argument("--seeds", type=int, nargs="+", default=[11, 23, 47])
    cli.add_argument("--scenarios", choices=tuple(SCENARIOS), nargs="+",
                     default=list(SCENARIOS))
    cli.add_argument("--draw-device", default=None,
                     help="device whose generator draws the graph (default: the GPU, as the "
                          "reference does; cpu: repeatable on any machine)")
    cli.add_argument("--output", type=Path, help="where to write the JSON results")
    return cli


def main(argv=None) -> dict:
    args = parser().parse_args(argv)
    if min(args.steps, args.neurons, args.batch, args.sample_interval) < 1 or args.edges < 0:
        raise SystemExit("sizes must be positive and edges non-negative")
    if not torch.cuda.is_available():
        raise SystemExit("the drift probe runs the native tick and needs a GPU")
    cases = [run_case(scenario, seed, steps=args.steps, sample_interval=args.sample_interval,
                      neurons=args.neurons, edges=args.edges, batch=args.batch,
                      chunk=args.chunk, draw_device=args.draw_device,
                      progress=lambda line: print(line, flush=True))
             for scenario in args.scenarios for seed in args.seeds]
    result = dict(protocol=dict(steps=args.steps, seeds=args.seeds, scenarios=args.scenarios,
                                sample_interval=args.sample_interval, chunk=args.chunk,
                                comparison="each weight mode against the native FP32 rollout "
                                           "of the same graph, initial state and inputs",
                                gpu=torch.cuda.get_device_name()),
                  cases=cases)
    if args.output is not None:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(json.dumps(result, indent=1) + "\n")
    for case in cases:
        peaks = ", ".join(
            f"{mode} {max(case['summary'][mode][f]['peak_sampled_max_abs'] for f in FIELDS):.2e}"
            for mode in MODES[1:])
        print(f"{case['scenario']} seed {case['seed']} ({case['edges']} edges): "
              f"peak max-abs vs fp32: {peaks}", flush=True)
    return result


if __name__ == "__main__":
    main()
