"""The device graph builder (ns_build_topology) against the oracle's CPU build.

Every field of the coalesced graph (canonical src/dst/weight, out_rowptr,
in_rowptr, in_col, in_weight, out_weight_index) must be bitwise equal to
oracle.topology.build on the same candidate edges, which restates the
reference's CPU from_edges (topology.py:32-115) and is pinned by the
reference-held edge count of the brainwaves graph and a brute-force
coalescer.  Covers no candidates, one neuron, duplicate-heavy graphs whose
sums depend on the summation order, lone -0.0 weights, a power-of-two N with
the largest key present, the reference's seed-23 graph (20,295 edges), the
batched workload's graph and the 25M-edge headline graph.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import topology as otop
from neurosim_gpu import SparseTopology, random_topology

pytestmark = pytest.mark.gpu
FIELDS = ("src", "dst", "weight", "out_rowptr", "in_rowptr", "in_col", "in_weight",
          "out_weight_index")


def device_build(n, src, dst, weight, gpu) -> SparseTopology:
    return SparseTopology.from_edges(n, torch.from_numpy(np.asarray(src, np.int64)).to(gpu),
                                     torch.from_numpy(np.asarray(dst, np.int64)).to(gpu),
                                     torch.from_numpy(np.asarray(weight, np.float32)).to(gpu))


def assert_same(topology: SparseTopology, graph: otop.Graph) -> None:
    assert topology.n_edges == graph.n_edges
    for name in FIELDS:
        got = getattr(topology, name).cpu().numpy()
        want = np.asarray(getattr(graph, name))
        assert got.dtype == want.dtype or name in ("weight", "in_weight"), name
        assert got.tobytes() == want.astype(got.dtype).tobytes(), name


@pytest.mark.parametrize("n,m,seed", [(1, 0, 0), (50, 0, 0), (1, 5, 1), (7, 200, 2),
                                      (97, 600, 83), (1000, 20_000, 0), (1024, 20_480, 23),
                                      (3000, 60_000, 1), (50_000, 1_000_000, 0)])
def test_random_candidates(gpu, n, m, seed):
    print(f"case topology random n={n} m={m} seed={seed}", flush=True)
    src, dst, weight = otop.random_edges(n, m, seed=seed)
    topology = device_build(n, src, dst, weight, gpu)
    assert_same(topology, otop.build(n, src, dst, weight))
    if (n, m, seed) == (1024, 20_480, 23):
        assert topology.n_edges == 20_295      # results/compartmental_brainwaves.json


def test_order_dependent_duplicate_sums(gpu):
    print("case topology duplicates", flush=True)
    rng = np.random.default_rng(5)
    n = 4
    src = rng.integers(0, n, 5000)
    dst = rng.integers(0, n, 5000)
    weight = (rng.standard_normal(5000) * 10.0 ** rng.integers(-3, 8, 5000)).astype(np.float32)
    assert_same(device_build(n, src, dst, weight, gpu), otop.build(n, src, dst, weight))
    values = np.array([1e8, 1.0, -1e8, 1.0, 3.0, -2.0, 1e-3, 5.0, 1e8, -1e8, 0.5], np.float32)
    zeros, ones = np.zeros(values.size, np.int64), np.ones(values.size, np.int64)
    assert_same(device_build(2, zeros, ones, values, gpu), otop.build(2, zeros, ones, values))


def test_negative_zero_and_largest_key(gpu):
    print("case topology -0.0 and key n*n-1", flush=True)
    n = 1024                                   # n*n is a power of two
    src = np.array([n - 1, 0, 5, 5, n - 1], np.int64)
    dst = np.array([n - 1, 0, 6, 6, 0], np.int64)
    weight = np.array([-0.0, -0.0, -0.0, -0.0, 2.5], np.float32)
    topology = device_build(n, src, dst, weight, gpu)
    assert_same(topology, otop.build(n, src, dst, weight))
    assert not torch.signbit(topology.weight).any()


def test_headline_graph_25m(gpu, large_case):
    """random_topology(166000, 25M candidates, seed 0): the device build of the same
    candidates equals the host build every other test uses."""
    print("case topology headline N=166000 M=25M", flush=True)
    src, dst, weight = otop.random_edges(166_000, 25_000_000, seed=0)
    topology = device_build(166_000, src, dst, weight, gpu)
    assert_same(topology, large_case.graph)


def test_random_topology_on_the_gpu_is_consistent(gpu):
    """random_topology(device='cuda') draws on the GPU generator, as the reference
    does, and builds on the device: the result equals the oracle's build of
    those same draws."""
    print("case topology random_topology cuda", flush=True)
    topology = random_topology(2000, 50_000, device=gpu, seed=4)
    generator = torch.Generator(device=gpu)
    generator.manual_seed(4)
    draw = dict(dtype=torch.int64, device=gpu, generator=generator)
    src = torch.randint(2000, (50_000,), **draw)
    dst = torch.randint(2000, (50_000,), **draw)
    weight = torch.randn(50_000, dtype=torch.float32, device=gpu, generator=generator) * (0.15 / 5.0)
    assert_same(topology, otop.build(2000, src.cpu().numpy(), dst.cpu().numpy(),
                                     weight.cpu().numpy()))
