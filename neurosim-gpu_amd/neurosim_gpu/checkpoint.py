"""Checkpoint and restore of runtime states (CPU payload, torch.save container).

Same payload schema as the reference (src/neurosim_gpu/checkpoint.py:23-330)
so checkpoints move between the native and the reference runtimes:
format "neurosim_gpu.runtime_checkpoint", version 1, runtime_type, precision,
a SHA-256 runtime_signature over the immutable parameters, the topology
payload, and CPU copies of the state tensors and scalar counters.  For the
dendritic runtimes that is state, dendritic_state, adaptation_state and, for
PELS, emitted_state, persistent_current, theta, _tick and _weight_version.

Restore rejects a different runtime type, missing states, other parameters or
another topology structure before anything is modified; weights are restored
through the topology mutation API so every runtime sharing the graph sees the
new weight_version.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Any, BinaryIO, Mapping

import torch

from .topology import SparseTopology
from .topology_io import topology_from_dict, topology_to_dict

FORMAT = "neurosim_gpu.runtime_checkpoint"
VERSION = 1

# Field names of the shared schema (the chemistry fields are only carried by
# runtimes that own them; none of this package's runtimes do).
_TENSOR_FIELDS = ("state", "dendritic_state", "adaptation_state", "emitted_state",
                  "persistent_current", "concentration", "pre_trace", "post_trace",
                  "eligibility", "_rpe_accumulator", "_source_release_accumulator",
                  "_rpe_delay", "_drive_shift", "_gain_scale", "theta")
_SCALAR_FIELDS = ("_tick", "_chemistry_tick", "_weight_version", "_cursor",
                  "_has_source_release", "_chemistry_applied")


def _cpu_clone(value: torch.Tensor) -> torch.Tensor:
    return value.detach().to(device="cpu").clone()


def _precision(runtime: Any) -> str:
    return getattr(runtime, "checkpoint_precision", getattr(runtime, "precision", "fp32"))


def _runtime_signature(runtime: Any) -> str:
    """SHA-256 over the immutable parameters, in the schema's hashing order.

    Tensors contribute str(dtype), repr(shape) and their contiguous CPU bytes;
    dataclasses contribute each field name then its value; JSON scalars their
    json.dumps text.  Order: soma alpha, gain; compartment dynamics; theta;
    "precision=..." when not fp32.
    """
    digest = hashlib.sha256()

    def add(value: Any) -> None:
        if isinstance(value, torch.Tensor):
            cpu = value.detach().to(device="cpu").contiguous().clone()
            digest.update(str(cpu.dtype).encode())
            digest.update(repr(tuple(cpu.shape)).encode())
            digest.update(bytes(cpu.untyped_storage()))
        elif isinstance(value, (str, int, float, bool)) or value is None:
            digest.update(json.dumps(value, sort_keys=True).encode())
        elif isinstance(value, (tuple, list)):
            for item in value:
                add(item)
        elif hasattr(value, "__dataclass_fields__"):
            for name in value.__dataclass_fields__:
                digest.update(name.encode())
                add(getattr(value, name))

    dynamics = getattr(runtime, "dynamics", None)
    if dynamics is not None:
        add(dynamics.alpha)
        add(dynamics.gain)
    if hasattr(runtime, "compartment_dynamics"):
        add(runtime.compartment_dynamics)
    if hasattr(runtime, "theta"):
        add(runtime.theta)
    precision = _precision(runtime)
    if precision != "fp32":
        digest.update(f"precision={precision}".encode())
    return digest.hexdigest()


def capture_runtime(runtime: Any, *, communication: Any = None) -> dict[str, Any]:
    """CPU payload of a runtime's states (no device memory is retained)."""
    if communication is not None:
        raise ValueError("delay-line communication state is not supported by this package")
    topology = getattr(runtime, "topology", None)
    if not isinstance(topology, SparseTopology):
        raise ValueError("runtime must own a SparseTopology")
    tensors = {name: _cpu_clone(value) for name in _TENSOR_FIELDS
               if isinstance(value := getattr(runtime, name, None), torch.Tensor)}
    scalars = {name: value for name in _SCALAR_FIELDS if hasattr(runtime, name)
               and isinstance(value := getattr(runtime, name), (bool, int, float))}
    return {"format": FORMAT, "version": VERSION, "runtime_type": type(runtime).__name__,
            "precision": _precision(runtime), "runtime_signature": _runtime_signature(runtime),
            "topology": topology_to_dict(topology), "tensors": tensors, "scalars": scalars}


def _check_payload(payload: Mapping[str, Any]) -> None:
    if payload.get("format") != FORMAT or payload.get("version") != VERSION:
        raise ValueError("unsupported runtime checkpoint format or version")
    for key, what in (("topology", "topology"), ("tensors", "tensor"), ("scalars", "scalar")):
        if not isinstance(payload.get(key), Mapping):
            raise ValueError(f"checkpoint is missing {what} payload")


def restore_runtime(runtime: Any, payload: Mapping[str, Any], *, communication: Any = None,
                    strict_runtime_type: bool = False) -> None:
    """Restore a captured payload into an already-constructed runtime."""
    if communication is not None:
        raise ValueError("delay-line communication state is not supported by this package")
    _check_payload(payload)
    if payload.get("precision", "fp32") != _precision(runtime):
        raise ValueError("checkpoint precision does not match target runtime")
    if hasattr(runtime, "compartment_dynamics"):
        if payload.get("runtime_type") != type(runtime).__name__:
            raise ValueError("compartment checkpoint runtime type must match target runtime")
        for name in ("state", "dendritic_state", "adaptation_state"):
            value = payload["tensors"].get(name)
            target = getattr(runtime, name)
            if not isinstance(value, torch.Tensor):
                raise ValueError(f"checkpoint is missing tensor {name}")
            if value.shape != target.shape or value.dtype != target.dtype:
                raise ValueError(f"checkpoint tensor {name} shape or dtype mismatch")
    if strict_runtime_type and payload.get("runtime_type") != type(runtime).__name__:
        raise ValueError("checkpoint runtime type does not match target runtime")
    signature = payload.get("runtime_signature")
    if signature is not None and signature != _runtime_signature(runtime):
        raise ValueError("checkpoint runtime parameters differ from target runtime")
    saved = topology_from_dict(payload["topology"], device="cpu", reset_weight_version=False)
    target = getattr(runtime, "topology", None)
    if not isinstance(target, SparseTopology):
        raise ValueError("runtime must own a SparseTopology")
    if saved.n_neurons != target.n_neurons or saved.n_edges != target.n_edges:
        raise ValueError("checkpoint topology shape does not match runtime")
    for name in ("src", "dst", "out_rowptr", "in_rowptr", "in_col", "out_weight_index"):
        if not torch.equal(getattr(saved, name).cpu(), getattr(target, name).cpu()):
            raise ValueError(f"checkpoint topology structure differs in {name}")
    for name, value in payload["tensors"].items():
        current = getattr(runtime, name, None)
        if not isinstance(current, torch.Tensor):
            raise ValueError(f"runtime does not expose checkpoint tensor {name}")
        if current.shape != value.shape:
            raise ValueError(f"checkpoint tensor {name} shape {tuple(value.shape)} does not "
                             f"match runtime shape {tuple(current.shape)}")
        if current.dtype != value.dtype:
            raise ValueError(f"checkpoint tensor {name} dtype does not match runtime")

    weight = saved.weight.to(device=target.weight.device)
    if weight.dtype != target.weight.dtype:
        raise ValueError("checkpoint topology weight dtype does not match runtime")
    # A no-op restore must not force peers sharing the graph to rebuild their currents.
    if not torch.equal(target.weight, weight):
        target.apply_source_weights_(weight)
    invalidate = getattr(runtime, "_invalidate_precision_cache", None)
    if invalidate is not None:
        invalidate()
    with torch.no_grad():
        for name, value in payload["tensors"].items():
            # Rebinding (not copy_) also works for expanded zero-stride targets.
            setattr(runtime, name, value.to(device=getattr(runtime, name).device).clone())
    for name, value in payload["scalars"].items():
        if hasattr(runtime, name):
            if name == "_weight_version":
                stale = value != saved.weight_version
                value = target.weight_version - int(stale)
            setattr(runtime, name, value)


def save_runtime_checkpoint(runtime: Any, destination: str | Path | BinaryIO, *,
                            communication: Any = None) -> None:
    torch.save(capture_runtime(runtime, communication=communication), destination)


def load_runtime_checkpoint(source: str | Path | BinaryIO, runtime: Any, *,
                            communication: Any = None, strict_runtime_type: bool = False) -> None:
    payload = torch.load(source, map_location="cpu", weights_only=True)
    if not isinstance(payload, Mapping):
        raise ValueError("runtime checkpoint must contain a mapping")
    restore_runtime(runtime, payload, communication=communication,
                    strict_runtime_type=strict_runtime_type)


__all__ = ["FORMAT", "VERSION", "capture_runtime", "load_runtime_checkpoint",
           "restore_runtime", "save_runtime_checkpoint"]
