"""Soma / dendrite / adaptation simulation from the command line.

    python -m neurosim_gpu.simulate [--backend native --device cuda] ...

Flags, defaults, validation errors and the JSON summary follow the
reference runner (src/neurosim_gpu/simulate.py:23-146), so scripts written
for it run unchanged.  ``--backend native --device cuda`` runs the gfx950 HIP
kernels.  Backend and propagation are taken as given: a missing native
library is an error, never a quiet switch to another path.
"""
from __future__ import annotations

import argparse
import json
import math
from pathlib import Path

import torch

from .checkpoint import load_runtime_checkpoint, save_runtime_checkpoint
from .compartmental import DendriticDynamics, DendriticMatrixRuntime, DendriticPELSRuntime
from .dynamics import Dynamics
from .native_compartmental import NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime
from .precision import PRECISIONS
from .topology import random_topology

# (flag, keyword arguments of add_argument): the runner's whole interface.
_OPTIONS = (
    ("--device", dict(choices=("cpu", "cuda"), default="cpu")),
    ("--backend", dict(choices=("reference", "native"), default="reference")),
    ("--precision", dict(choices=PRECISIONS, default="fp32",
                         help="torch propagation precision, or the native weight storage")),
    ("--propagation", dict(choices=("matrix", "pels"), default="matrix")),
    ("--neurons", dict(type=int, default=1000)),
    ("--edges", dict(type=int, default=20_000,
                     help="random candidate edges; duplicates are merged")),
    ("--batch", dict(type=int, default=1)),
    ("--steps", dict(type=int, default=100, help="ticks run by this invocation")),
    ("--seed", dict(type=int, default=0)),
    ("--theta", dict(type=float, default=0.0,
                     help="PELS emission threshold (0 is exact, above 0 approximate)")),
    ("--drive", dict(type=float, default=0.2)),
    ("--dendritic-drive", dict(type=float, default=0.1)),
    ("--dt", dict(type=float, default=1.0)),
    ("--tau-dendrite", dict(type=float, default=4.0)),
    ("--tau-adaptation", dict(type=float, default=25.0)),
    ("--coupling", dict(type=float, default=0.5)),
    ("--adaptation-strength", dict(type=float, default=0.2)),
    ("--resume", dict(type=Path, help="checkpoint to continue from (same graph, model "
                                      "and runtime)")),
    ("--checkpoint", dict(type=Path, help="where to save every runtime state at the end")),
    ("--output", dict(type=Path, help="where to write the JSON summary")),
)

# Soma parameters of the runner's model: one rate and one gain for every neuron.
SOMA_RATE, SOMA_GAIN = 0.72, 0.8


def parser() -> argparse.ArgumentParser:
    cli = argparse.ArgumentParser(description=__doc__,
                                  formatter_class=argparse.RawDescriptionHelpFormatter)
    for flag, options in _OPTIONS:
        cli.add_argument(flag, **options)
    return cli


def _problems(args: argparse.Namespace):
    """The runner's argument errors, in the order they are reported."""
    yield (min(args.neurons, args.batch, args.steps) <= 0 or args.edges < 0,
           "neurons, batch and steps must be positive; edges must be non-negative")
    yield (not all(map(math.isfinite, (args.theta, args.drive, args.dendritic_drive))),
           "theta and external drives must be finite")
    yield args.theta < 0, "theta must be non-negative"
    yield (args.propagation == "matrix" and args.theta != 0,
           "theta applies only to --propagation pels")
    native = args.backend == "native"
    yield (native and args.device != "cuda",
           "--backend native requires --device cuda and the HIP library")
    yield (native and args.propagation == "pels" and args.precision != "fp32",
           "native PELS supports FP32 only; use native matrix or reference PELS")
    yield (args.precision == "fp16" and args.device != "cuda",
           "--precision fp16 requires --device cuda")
    yield (args.device == "cuda" and not torch.cuda.is_available(),
           "no GPU is available; use --device cpu --backend reference")


def _model(args: argparse.Namespace) -> DendriticDynamics:
    def constant(value: float) -> torch.Tensor:
        return torch.full((args.neurons,), value, device=args.device)

    return DendriticDynamics.from_time_constants(
        Dynamics(constant(SOMA_RATE), constant(SOMA_GAIN)), dt=args.dt,
        tau_dendrite=args.tau_dendrite, tau_adaptation=args.tau_adaptation,
        coupling=args.coupling, adaptation_strength=args.adaptation_strength)


def _native_matrix(graph, model, initial, args):
    storage = {"fp16": dict(weight_dtype=torch.float16), "fp8": dict(weight_format="fp8"),
               "nvfp4": dict(weight_format="nvfp4")}.get(args.precision, {})
    return NativeDendriticMatrixRuntime(graph, model, initial, **storage)


# (propagation, backend) -> runtime.  Reference PELS propagates by matrix.
_BUILDERS = {
    ("matrix", "native"): _native_matrix,
    ("matrix", "reference"): lambda graph, model, initial, args: DendriticMatrixRuntime(
        graph, model, initial, precision=args.precision),
    ("pels", "native"): lambda graph, model, initial, args: NativeDendriticPELSRuntime(
        graph, model, initial, theta=args.theta),
    ("pels", "reference"): lambda graph, model, initial, args: DendriticPELSRuntime(
        graph, model, initial, theta=args.theta, propagation="matrix",
        precision=args.precision),
}


def build_runtime(args: argparse.Namespace):
    for failed, message in _problems(args):
        if failed:
            raise ValueError(message)
    graph = random_topology(args.neurons, args.edges, device=args.device, seed=args.seed)
    initial = torch.zeros(args.batch, args.neurons, device=args.device)
    return _BUILDERS[args.propagation, args.backend](graph, _model(args), initial, args)


def _same_file(a: Path, b: Path) -> bool:
    if a.resolve() == b.resolve():
        return True
    return a.exists() and b.exists() and a.samefile(b)


def _summary_of(value: torch.Tensor, name: str) -> dict:
    if not bool(torch.isfinite(value).all()):
        raise RuntimeError(f"non-finite final {name}")
    return {"shape": list(value.shape), "mean": float(value.mean()),
            "min": float(value.min()), "max": float(value.max())}


def run(args: argparse.Namespace) -> dict:
    if args.output is not None:
        for option in ("checkpoint", "resume"):
            other = getattr(args, option)
            if other is not None and _same_file(args.output, other):
                raise ValueError(f"--output must use a different file from --{option}")
    runtime = build_runtime(args)
    if args.resume is not None:
        load_runtime_checkpoint(args.resume, runtime)
    with torch.inference_mode():
        for _ in range(args.steps):
            runtime.step(args.drive, dendritic_drive=args.dendritic_drive)
    # One host synchronisation, after the whole rollout.
    states = {name: _summary_of(getattr(runtime, name), name)
              for name in ("state", "dendritic_state", "adaptation_state")}
    if args.checkpoint is not None:
        args.checkpoint.parent.mkdir(parents=True, exist_ok=True)
        save_runtime_checkpoint(runtime, args.checkpoint)
    approximate = args.precision != "fp32" or (args.propagation == "pels" and args.theta > 0)
    summary = {
        "model": "soma-dendrite-adaptation", "runtime": type(runtime).__name__,
        "backend": getattr(runtime, "last_backend", "reference"),
        "device": str(runtime.state.device), "dtype": str(runtime.state.dtype),
        "precision": args.precision, "precision_execution": runtime.precision_execution,
        "torch": torch.__version__, "propagation": args.propagation,
        "neurons": runtime.topology.n_neurons, "actual_edges": runtime.topology.n_edges,
        "steps_this_run": args.steps, "theta": args.theta, "approximate": approximate,
        "resumed": args.resume is not None,
        "config": {key: str(value) if isinstance(value, Path) else value
                   for key, value in vars(args).items()},
        "states": states,
    }
    if args.output is not None:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(json.dumps(summary, indent=2) + "\n", encoding="utf-8")
    return summary


def main() -> None:
    cli = parser()
    args = cli.parse_args()
    try:
        summary = run(args)
    except ValueError as error:
        cli.error(str(error))
    print(json.dumps(summary, indent=2))


if __name__ == "__main__":
    main()
