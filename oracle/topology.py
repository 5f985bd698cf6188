"""Oracle graph generator and CSR builder (test infrastructure only).

Restates the reference's ``random_topology`` (topology.py:213-247) and
``SparseTopology.from_edges`` (topology.py:32-115).  Random draws use torch's
CPU generator in the reference's draw order (the stream is the library's, not
something to re-derive); coalescing and both CSR views are rebuilt here in
numpy.

Pins: ``tests/test_oracle_topology.py`` checks the reference-held edge count of
random_topology(1024, 20480, seed=23) (results/compartmental_brainwaves.json:
actual_edges 20295), the canonical-order / permutation invariants the
reference's tests assert (test_topology_io.py:92-113), and a dictionary-based
brute-force coalescer on small graphs.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch


@dataclass
class Graph:
    """Both CSR views of a coalesced graph, as numpy arrays (CPU)."""

    n: int
    src: np.ndarray          # int32 [M], source-major canonical order
    dst: np.ndarray          # int32 [M]
    weight: np.ndarray       # [M], canonical order
    out_rowptr: np.ndarray   # int32 [N+1], source-major
    in_rowptr: np.ndarray    # int32 [N+1], destination-major
    in_col: np.ndarray       # int32 [M], source of each destination-major edge
    in_weight: np.ndarray    # [M], destination-major order
    out_weight_index: np.ndarray  # int32 [M], canonical edge -> destination-major slot

    @property
    def n_edges(self) -> int:
        return int(self.weight.size)

    def dense(self, dtype=np.float64) -> np.ndarray:
        """Dense W[dst, src] (reference topology.py:136-147)."""
        matrix = np.zeros((self.n, self.n), dtype=dtype)
        np.add.at(matrix, (self.dst.astype(np.int64), self.src.astype(np.int64)),
                  self.weight.astype(dtype))
        return matrix


def random_edges(n: int, m: int, *, seed: int = 0, weight_scale: float = 0.15,
                 dtype: torch.dtype = torch.float32):
    """Candidate edges in the reference's draw order (topology.py:224-246).

    src and dst are two int64 randint draws, then one normal draw scaled by
    weight_scale / sqrt(max(m/n, 1)), all from one CPU generator seeded with
    ``seed``.  Returns numpy arrays.
    """
    if n <= 0 or m < 0:
        raise ValueError("n_neurons must be positive and n_edges non-negative")
    generator = torch.Generator(device="cpu")
    generator.manual_seed(seed)
    src = torch.randint(n, (m,), dtype=torch.int64, generator=generator)
    dst = torch.randint(n, (m,), dtype=torch.int64, generator=generator)
    spread = weight_scale / max(m / n, 1.0) ** 0.5
    weight = torch.randn(m, dtype=dtype, generator=generator) * spread
    return src.numpy(), dst.numpy(), weight.numpy()


def _rowptr(rows: np.ndarray, n: int) -> np.ndarray:
    counts = np.bincount(rows, minlength=n) if rows.size else np.zeros(n, np.int64)
    out = np.zeros(n + 1, dtype=np.int64)
    np.cumsum(counts, out=out[1:])
    return out.astype(np.int32)


def build(n: int, src: np.ndarray, dst: np.ndarray, weight: np.ndarray) -> Graph:
    """Coalesce duplicate (src, dst) pairs by summation and build both views.

    Reference topology.py:62-115: stable sort by src*n+dst, duplicates summed
    in that order starting from zero, destination-major view by a stable sort
    on dst*n+src, out_weight_index = inverse of that permutation.
    """
    src = np.asarray(src, dtype=np.int64)
    dst = np.asarray(dst, dtype=np.int64)
    weight = np.asarray(weight)
    key = src * n + dst
    order = np.argsort(key, kind="stable")
    sorted_key = key[order]
    sorted_weight = weight[order]
    first = np.ones(sorted_key.size, dtype=bool)
    first[1:] = sorted_key[1:] != sorted_key[:-1]
    unique_key = sorted_key[first]
    starts = np.flatnonzero(first)
    sizes = np.diff(np.append(starts, sorted_key.size))
    # Strictly sequential sums from zero per run of equal keys (the reference's
    # zeros(...).index_add: a lone -0.0 weight becomes +0.0): the j-th element
    # of every run with more than j elements is added in round j.
    canonical_weight = np.zeros(starts.size, dtype=sorted_weight.dtype) + sorted_weight[starts]
    for j in range(1, int(sizes.max()) if sizes.size else 0):
        runs = np.flatnonzero(sizes > j)
        canonical_weight[runs] = canonical_weight[runs] + sorted_weight[starts[runs] + j]
    c_src = unique_key // n
    c_dst = unique_key % n
    in_order = np.argsort(c_dst * n + c_src)   # keys are unique: any sort is stable
    out_weight_index = np.empty(unique_key.size, dtype=np.int32)
    out_weight_index[in_order] = np.arange(unique_key.size, dtype=np.int32)
    return Graph(
        n=n,
        src=c_src.astype(np.int32),
        dst=c_dst.astype(np.int32),
        weight=canonical_weight,
        out_rowptr=_rowptr(c_src, n),
        in_rowptr=_rowptr(c_dst[in_order], n),
        in_col=c_src[in_order].astype(np.int32),
        in_weight=canonical_weight[in_order],
        out_weight_index=out_weight_index,
    )


def random_graph(n: int, m: int, *, seed: int = 0, weight_scale: float = 0.15,
                 dtype: torch.dtype = torch.float32) -> Graph:
    """random_topology(n, m, device="cpu", seed=seed) restated."""
    return build(n, *random_edges(n, m, seed=seed, weight_scale=weight_scale, dtype=dtype))


def with_weights(graph: Graph, canonical_weight: np.ndarray) -> Graph:
    """The same structure with new canonical weights (reference topology.py:194-205)."""
    canonical_weight = np.asarray(canonical_weight)
    in_weight = np.empty_like(canonical_weight)
    in_weight[graph.out_weight_index] = canonical_weight
    return Graph(graph.n, graph.src, graph.dst, canonical_weight.copy(), graph.out_rowptr,
                 graph.in_rowptr, graph.in_col, in_weight, graph.out_weight_index)


def with_in_weight(graph: Graph, in_weight: np.ndarray) -> Graph:
    """The same structure with new destination-major weights (e.g. decoded ones)."""
    in_weight = np.asarray(in_weight)
    return Graph(graph.n, graph.src, graph.dst, in_weight[graph.out_weight_index].copy(),
                 graph.out_rowptr, graph.in_rowptr, graph.in_col, in_weight.copy(),
                 graph.out_weight_index)


def block_diagonal(graphs: list[Graph]) -> Graph:
    """The disjoint union of graphs: graph k's neurons are numbered after those
    of graphs 0..k-1, so W is block diagonal and both CSR views keep every
    row's edges in their original order.  A CSR product's row sum reads only
    its own row, so each block of a tick over the union evolves exactly as its
    graph would alone (tests/test_oracle_runtime.py checks this bitwise)."""
    offsets = np.cumsum([0] + [g.n for g in graphs])
    edge_offsets = np.cumsum([0] + [g.n_edges for g in graphs])

    def cat(name, shift=None):
        if shift is None:
            return np.concatenate([getattr(g, name) for g in graphs])
        return np.concatenate([getattr(g, name).astype(np.int64) + shift[k]
                               for k, g in enumerate(graphs)])

    def rowptr(name):
        parts = [np.zeros(1, np.int64)] + [getattr(g, name)[1:].astype(np.int64) + edge_offsets[k]
                                           for k, g in enumerate(graphs)]
        return np.concatenate(parts).astype(np.int32)

    return Graph(
        n=int(offsets[-1]),
        src=cat("src", offsets).astype(np.int32),
        dst=cat("dst", offsets).astype(np.int32),
        weight=cat("weight"),
        out_rowptr=rowptr("out_rowptr"),
        in_rowptr=rowptr("in_rowptr"),
        in_col=cat("in_col", offsets).astype(np.int32),
        in_weight=cat("in_weight"),
        out_weight_index=cat("out_weight_index", edge_offsets).astype(np.int32),
    )
