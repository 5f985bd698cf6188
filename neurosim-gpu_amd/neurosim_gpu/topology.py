"""Fixed sparse graphs: source-major canonical edges plus a destination CSR view.

API of the reference's SparseTopology / random_topology
(src/neurosim_gpu/topology.py:16-247).  The destination-major view
(in_rowptr, in_col, in_weight) feeds the fused matrix tick; the source-major
view (out_rowptr, dst) and out_weight_index feed the PELS scatter, which reads
in_weight[out_weight_index[e]] for canonical edge e.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


def _offsets(rows: torch.Tensor, n_rows: int) -> torch.Tensor:
    """int32 CSR offsets of a sorted (or unsorted) row-id vector."""
    counts = torch.bincount(rows, minlength=n_rows)
    offsets = torch.zeros(n_rows + 1, dtype=torch.int64, device=rows.device)
    offsets[1:] = torch.cumsum(counts, dim=0)
    return offsets.to(torch.int32)


@dataclass(frozen=True)
class SparseTopology:
    """A fixed graph with source-major canonical edges and a destination CSR view."""

    n_neurons: int
    src: torch.Tensor
    dst: torch.Tensor
    weight: torch.Tensor
    out_rowptr: torch.Tensor
    in_rowptr: torch.Tensor
    in_col: torch.Tensor
    out_weight_index: torch.Tensor
    in_weight: torch.Tensor
    weight_version: int = 0

    @classmethod
    def from_edges(cls, n_neurons: int, src: torch.Tensor, dst: torch.Tensor,
                   weight: torch.Tensor) -> "SparseTopology":
        """Coalesce parallel edges (summed) and build both views.

        Canonical edges are ordered by (src, dst); duplicates are summed in
        their input order starting from zero (reference topology.py:62-80).
        """
        if src.ndim != 1 or dst.ndim != 1 or weight.ndim != 1:
            raise ValueError("src, dst and weight must be rank-1 tensors")
        if not (src.numel() == dst.numel() == weight.numel()):
            raise ValueError("src, dst and weight must have equal length")
        index_types = (torch.int32, torch.int64)
        if src.dtype not in index_types or dst.dtype not in index_types:
            raise ValueError("edge indices must use torch.int32 or torch.int64")
        if src.device != dst.device or src.device != weight.device:
            raise ValueError("all edge tensors must be on the same device")
        source = src.to(torch.int64)
        target = dst.to(torch.int64)
        if source.numel():
            low = min(int(source.min()), int(target.min()))
            high = max(int(source.max()), int(target.max()))
            if low < 0 or high >= n_neurons:
                raise ValueError("edge index out of range")
        if source.numel() >= 2**31:
            raise ValueError("this compact topology supports fewer than 2^31 edges")

        if weight.device.type == "cuda" and weight.dtype == torch.float32:
            # On the GPU: ns_build_topology (stable sorts, each run of duplicates
            # summed in order by one lane), bitwise equal to the CPU build below.
            # Other weight dtypes take the torch ops below, as in the reference.
            from .native import build_topology

            return cls(n_neurons=n_neurons, **build_topology(n_neurons, source, target, weight))

        key = source * n_neurons + target
        # unique(sorted) + index_add in input order == stable sort then ordered sum.
        unique_key, inverse = torch.unique(key, sorted=True, return_inverse=True)
        canonical_weight = torch.zeros(unique_key.numel(), dtype=weight.dtype,
                                       device=weight.device).index_add(0, inverse, weight)
        canonical_src = torch.div(unique_key, n_neurons, rounding_mode="floor")
        canonical_dst = unique_key - canonical_src * n_neurons

        # Destination-major order (keys are unique, so any sort is stable here).
        in_order = torch.argsort(canonical_dst * n_neurons + canonical_src)
        slot = torch.empty(unique_key.numel(), dtype=torch.int32, device=weight.device)
        slot[in_order] = torch.arange(unique_key.numel(), dtype=torch.int32,
                                      device=weight.device)
        return cls(
            n_neurons=n_neurons,
            src=canonical_src.to(torch.int32),
            dst=canonical_dst.to(torch.int32),
            weight=canonical_weight,
            out_rowptr=_offsets(canonical_src, n_neurons),
            in_rowptr=_offsets(canonical_dst, n_neurons),
            in_col=canonical_src[in_order].to(torch.int32),
            out_weight_index=slot,
            in_weight=canonical_weight[in_order],
        )

    @property
    def n_edges(self) -> int:
        return self.weight.numel()

    @property
    def out_degree(self) -> torch.Tensor:
        return self.out_rowptr[1:] - self.out_rowptr[:-1]

    def sparse_matrix(self) -> torch.Tensor:
        """W[dst, src] as a torch CSR tensor over the destination-major view."""
        return torch.sparse_csr_tensor(
            self.in_rowptr, self.in_col, self.in_weight,
            size=(self.n_neurons, self.n_neurons), dtype=self.weight.dtype,
            device=self.weight.device, check_invariants=False)

    def dense_matrix(self) -> torch.Tensor:
        matrix = torch.zeros((self.n_neurons, self.n_neurons), dtype=self.weight.dtype,
                             device=self.weight.device)
        matrix.index_put_((self.dst.to(torch.int64), self.src.to(torch.int64)),
                          self.weight, accumulate=True)
        return matrix

    @staticmethod
    def _bytes(*tensors: torch.Tensor) -> int:
        return sum(t.numel() * t.element_size() for t in tensors)

    def storage_bytes(self) -> int:
        return self._bytes(self.src, self.dst, self.weight, self.out_rowptr, self.in_rowptr,
                           self.in_col, self.out_weight_index, self.in_weight)

    def torch_hybrid_storage_bytes(self) -> int:
        """Logical storage of the PyTorch matrix plus event representation."""
        return self._bytes(self.src, self.dst, self.weight, self.out_rowptr, self.in_rowptr,
                           self.in_col, self.in_weight)

    def native_storage_bytes(self) -> int:
        """Storage read by the native matrix and event kernels."""
        return self._bytes(self.dst, self.out_weight_index, self.out_rowptr, self.in_rowptr,
                           self.in_col, self.in_weight)

    @torch.no_grad()
    def apply_source_weights_(self, source_major_weight: torch.Tensor) -> None:
        """Update both weight views from one source-major vector (bumps weight_version)."""
        if source_major_weight.shape != self.weight.shape:
            raise ValueError("source_major_weight shape does not match topology")
        if source_major_weight.device != self.weight.device:
            raise ValueError("source_major_weight must be on the topology device")
        if source_major_weight.dtype != self.weight.dtype:
            raise ValueError("source_major_weight dtype does not match topology")
        self.weight.copy_(source_major_weight)
        self.in_weight[self.out_weight_index.to(torch.int64)] = source_major_weight
        self.mark_weights_mutated_()

    def mark_weights_mutated_(self) -> None:
        """Invalidate persistent-current and packed-weight caches."""
        object.__setattr__(self, "weight_version", self.weight_version + 1)


def random_topology(n_neurons: int, n_edges: int, *, device: torch.device | str,
                    dtype: torch.dtype = torch.float32, seed: int = 0,
                    weight_scale: float = 0.15,
                    build_device: torch.device | str | None = None) -> SparseTopology:
    """Uniform random sources/targets and N(0, (scale/sqrt(mean degree))^2) weights.

    Draw order on one generator seeded with ``seed``: src, dst, weights
    (reference topology.py:224-246).  The generator lives on ``device``, so a
    CPU graph and a GPU graph from the same seed differ; build on the CPU and
    move the tensors for cross-device comparisons.  ``build_device`` (an
    addition to the reference's signature) moves the drawn candidates there
    before coalescing: device="cpu", build_device="cuda" gives the CPU graph's
    exact bits, built by the GPU.
    """
    if n_neurons <= 0 or n_edges < 0:
        raise ValueError("n_neurons must be positive and n_edges non-negative")
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)
    draw = dict(dtype=torch.int64, device=device, generator=generator)
    src = torch.randint(n_neurons, (n_edges,), **draw)
    dst = torch.randint(n_neurons, (n_edges,), **draw)
    scale = weight_scale / max(n_edges / n_neurons, 1.0) ** 0.5
    weight = torch.randn(n_edges, dtype=dtype, device=device, generator=generator) * scale
    if build_device is not None:
        src, dst, weight = src.to(build_device), dst.to(build_device), weight.to(build_device)
    return SparseTopology.from_edges(n_neurons, src, dst, weight)


def topology_to(topology: SparseTopology, device: torch.device | str) -> SparseTopology:
    """The same graph (same bits, same version) with every tensor on ``device``."""
    fields = {name: getattr(topology, name).to(device)
              for name in ("src", "dst", "weight", "out_rowptr", "in_rowptr", "in_col",
                           "out_weight_index", "in_weight")}
    return SparseTopology(n_neurons=topology.n_neurons, weight_version=topology.weight_version,
                          **fields)
