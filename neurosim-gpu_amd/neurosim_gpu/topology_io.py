"""Portable CPU serialization of SparseTopology (the checkpoint's topology part).

Same on-disk schema as the reference (src/neurosim_gpu/topology_io.py:27-380):
a mapping with format "neurosim_gpu.sparse_topology", version/schema_version 1,
n_neurons, weight_version, the int32 index arrays src, dst, out_rowptr,
in_rowptr, in_col, out_weight_index and one source-major weight vector
(in_weight optional and redundant).  The destination-major weights are rebuilt
from out_weight_index on load.  Loading validates the whole structure.
"""

from __future__ import annotations

from pathlib import Path
from typing import Any, BinaryIO, Mapping

import torch

from .topology import SparseTopology

FORMAT = "neurosim_gpu.sparse_topology"
SCHEMA_VERSION = 1
_INDEX_FIELDS = ("src", "dst", "out_rowptr", "in_rowptr", "in_col", "out_weight_index")


def _int(value: Any, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int):
        raise ValueError(f"{name} must be a Python integer")
    return int(value)


def _counts_to_offsets(rows: torch.Tensor, n: int) -> torch.Tensor:
    offsets = torch.zeros(n + 1, dtype=torch.int64, device=rows.device)
    offsets[1:] = torch.cumsum(torch.bincount(rows.to(torch.int64), minlength=n), dim=0)
    return offsets


def _validate(payload: Mapping[str, Any]) -> tuple[int, int]:
    """Check schema and structure; return (n_neurons, saved weight_version)."""
    if not isinstance(payload, Mapping):
        raise ValueError("topology payload must be a mapping")
    if payload.get("format") != FORMAT:
        raise ValueError("unsupported topology payload format")
    versions = [_int(payload[k], k) for k in ("version", "schema_version") if k in payload]
    if not versions or any(v != SCHEMA_VERSION for v in versions):
        raise ValueError(f"unsupported topology schema version (expected {SCHEMA_VERSION})")
    n = _int(payload.get("n_neurons"), "n_neurons")
    if n <= 0 or n >= 2**31:
        raise ValueError("n_neurons must be positive and less than 2^31")
    saved_version = _int(payload.get("weight_version", 0), "weight_version")
    if saved_version < 0:
        raise ValueError("weight_version must be non-negative")
    for name in _INDEX_FIELDS + ("weight",):
        value = payload.get(name)
        if not isinstance(value, torch.Tensor) or value.ndim != 1:
            raise ValueError(f"topology payload field {name!r} must be a rank-1 tensor")
    for name in _INDEX_FIELDS:
        if payload[name].dtype != torch.int32:
            raise ValueError(f"topology payload field {name!r} must use torch.int32")
    weight = payload["weight"]
    if not weight.is_floating_point():
        raise ValueError("topology weights must use a floating-point dtype")
    if weight.numel() and not bool(torch.isfinite(weight).all()):
        raise ValueError("topology weights must be finite")
    m = weight.numel()
    if m >= 2**31:
        raise ValueError("this compact topology supports fewer than 2^31 edges")
    devices = {payload[name].device for name in _INDEX_FIELDS + ("weight",)}
    if len(devices) != 1:
        raise ValueError("topology payload tensors must share one device")
    src = payload["src"].to(torch.int64)
    dst = payload["dst"].to(torch.int64)
    for name in ("src", "dst", "in_col", "out_weight_index"):
        if payload[name].numel() != m:
            raise ValueError(f"{name} length does not match weight length")
    for name, rows in (("out_rowptr", src), ("in_rowptr", dst)):
        rowptr = payload[name].to(torch.int64)
        if rowptr.shape != (n + 1,):
            raise ValueError(f"{name} must have shape [{n + 1}]")
        if m and (int(rows.min()) < 0 or int(rows.max()) >= n):
            raise ValueError("edge index out of range")
        if not torch.equal(rowptr, _counts_to_offsets(rows, n)):
            raise ValueError(f"{name} does not match the edge list")
    if m:
        if int(src.min()) < 0 or int(dst.min()) < 0 or int(src.max()) >= n or int(dst.max()) >= n:
            raise ValueError("edge index out of range")
        keys = src * n + dst
        if m > 1:
            step = keys[1:] - keys[:-1]
            if bool((step < 0).any()):
                raise ValueError("source/destination edges are not source-major ordered")
            if bool((step == 0).any()):
                raise ValueError("duplicate source/destination edge")
        slot = payload["out_weight_index"].to(torch.int64)
        if int(slot.min()) < 0 or int(slot.max()) >= m:
            raise ValueError("out_weight_index is out of range")
        inverse = torch.full((m,), -1, dtype=torch.int64, device=slot.device)
        inverse[slot] = torch.arange(m, dtype=torch.int64, device=slot.device)
        if bool((inverse < 0).any()):
            raise ValueError("out_weight_index must be a permutation")
        in_rowptr = payload["in_rowptr"].to(torch.int64)
        rows = torch.repeat_interleave(torch.arange(n, device=slot.device),
                                       in_rowptr[1:] - in_rowptr[:-1])
        if not torch.equal(dst[inverse], rows):
            raise ValueError("out_weight_index does not match in_rowptr")
        if not torch.equal(payload["in_col"].to(torch.int64), src[inverse]):
            raise ValueError("in_col does not match out_weight_index")
    if "in_weight" in payload:
        in_weight = payload["in_weight"]
        if not isinstance(in_weight, torch.Tensor) or in_weight.shape != weight.shape:
            raise ValueError("in_weight length does not match weight length")
        if m and not torch.equal(in_weight[payload["out_weight_index"].long()], weight):
            raise ValueError("in_weight does not match weight and out_weight_index")
    return n, saved_version


def topology_to_dict(topology: SparseTopology, *, include_destination_weights: bool = False
                     ) -> dict[str, Any]:
    """Validated CPU payload of a topology."""
    def cpu(t: torch.Tensor) -> torch.Tensor:
        return t.detach().to("cpu").contiguous()

    payload: dict[str, Any] = {
        "format": FORMAT, "version": SCHEMA_VERSION, "schema_version": SCHEMA_VERSION,
        "n_neurons": int(topology.n_neurons),
        "weight_version": int(topology.weight_version),
        "weight_version_reset_on_load": True,
        "weight": cpu(topology.weight),
    }
    for name in _INDEX_FIELDS:
        payload[name] = cpu(getattr(topology, name))
    if include_destination_weights:
        payload["in_weight"] = cpu(topology.in_weight)
    _validate(payload)
    return payload


def topology_from_dict(payload: Mapping[str, Any], *, device: torch.device | str | None = None,
                       reset_weight_version: bool = True) -> SparseTopology:
    """Rebuild a topology from a payload without sorting or random draws."""
    n, saved_version = _validate(payload)
    target = torch.device("cpu" if device is None else device)
    fields = {name: payload[name].detach().to(target).contiguous()
              for name in _INDEX_FIELDS + ("weight",)}
    slot = fields["out_weight_index"].to(torch.int64)
    in_weight = torch.empty_like(fields["weight"])
    in_weight[slot] = fields["weight"]
    return SparseTopology(n_neurons=n, in_weight=in_weight,
                          weight_version=0 if reset_weight_version else saved_version,
                          **fields)


def save_topology(topology: SparseTopology, destination: str | Path | BinaryIO, *,
                  include_destination_weights: bool = False) -> None:
    torch.save(topology_to_dict(topology, include_destination_weights=include_destination_weights),
               destination)


def load_topology(source: str | Path | BinaryIO, *, device: torch.device | str | None = None,
                  reset_weight_version: bool = True) -> SparseTopology:
    payload = torch.load(source, map_location="cpu", weights_only=True)
    if not isinstance(payload, Mapping):
        raise ValueError("serialized topology must contain a mapping")
    return topology_from_dict(payload, device=device, reset_weight_version=reset_weight_version)
