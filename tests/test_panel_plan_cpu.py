"""The column-panel layout (ns_plan_panels) on the host: invariants, and a numpy
emulation of the panel kernel's decomposition against the plain CSR product.

Covers several panels (small panel widths), rows longer than one chunk (hub
rows split with continuation flags), rows without edges, empty graphs and
stripes of unequal size.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import topology as otop
from neurosim_gpu.native import panel_geometry, plan_panels_host


def hub_graph(n: int, seed: int) -> otop.Graph:
    rng = np.random.default_rng(seed)
    hubs = min(n, 9000)
    dst = np.concatenate([np.zeros(hubs, np.int64), np.full(n // 2, 3), rng.integers(0, n, 8 * n)])
    src = np.concatenate([np.arange(hubs), rng.permutation(n)[: n // 2], rng.integers(0, n, 8 * n)])
    return otop.build(n, src, dst, rng.standard_normal(dst.size).astype(np.float32))


GRAPHS = {
    "random": lambda: otop.random_graph(3000, 60_000, seed=1),
    "hubs": lambda: hub_graph(12_000, 2),
    "sparse": lambda: otop.random_graph(700, 300, seed=3),
    "empty": lambda: otop.build(50, np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(0, np.float32)),
    "single": lambda: otop.random_graph(1, 0, seed=0),
}


def emulate(graph: otop.Graph, batch: int, n_stripes: int, width: int | None, source: np.ndarray,
            n_groups: int | None = None):
    plan, tiles, chunks, offsets, lanes, stripes, perm, cols = plan_panels_host(
        torch.from_numpy(graph.in_rowptr), torch.from_numpy(graph.in_col), batch, n_stripes, width,
        n_groups)
    n, m = graph.n, graph.n_edges
    cap, chunk_edges, pad = panel_geometry(batch)
    assert plan.chunk_edges == chunk_edges and plan.pad == pad
    assert plan.panel_width % 4 == 0 and plan.panel_width <= min(cap, width or cap)
    assert plan.n_panels * plan.panel_width >= n > (plan.n_panels - 1) * plan.panel_width
    assert stripes[0] == 0 and stripes[-1] == n and np.all(np.diff(stripes) > 0)
    rows_of_edge = np.repeat(np.arange(n), np.diff(graph.in_rowptr))
    partial = np.zeros((plan.n_panels, n, batch))
    written = np.zeros((plan.n_panels, n), dtype=np.int64)
    stripe_done = np.zeros((plan.n_panels, plan.n_stripes), dtype=np.int64)
    seen = np.zeros(m, dtype=np.int64)
    tiles = tiles.reshape(-1, 4)
    chunks = chunks.reshape(-1, 8)
    lanes = lanes.reshape(-1, 512)
    assert np.array_equal(np.sort(tiles[:, 1]), tiles[:, 1]) and tiles[0, 1] == 0
    assert np.all(tiles[1:, 1] == tiles[:-1, 2]) and tiles[-1, 2] == plan.n_chunks
    for panel, c0, c1, _group in tiles:
        carry = np.zeros(batch)
        current = None                 # stripe in progress and the next row expected
        for c in range(c0, c1):
            slot0, nedge, row0, nrows, off0, flags, lane_index, stripe = chunks[c]
            assert slot0 % pad == 0 and 0 < nrows <= 511 and nedge <= chunk_edges
            if current is None:
                current, expected_row = stripe, stripes[stripe]
            assert stripe == current and row0 == expected_row
            offs = offsets[off0: off0 + nrows + 1].astype(np.int64)
            assert offs[0] == 0 and offs[-1] == nedge and np.all(np.diff(offs) >= 0)
            tail = perm[slot0 + nedge: slot0 + -(-nedge // pad) * pad]
            assert np.all(tail == -1)
            for lane in range(512):
                first = lane * pad
                if first < nedge:
                    r = lanes[lane_index, lane]
                    assert offs[r] <= first < offs[r + 1]
                else:
                    assert lanes[lane_index, lane] == nrows
            for r in range(nrows):
                slots = np.arange(slot0 + offs[r], slot0 + offs[r + 1])
                edges = perm[slots]
                assert np.all(edges >= 0)
                seen[edges] += 1
                row = row0 + r
                assert np.all(rows_of_edge[edges] == row)
                sources = graph.in_col[edges].astype(np.int64)
                assert np.array_equal(sources - panel * plan.panel_width, cols[slots].astype(np.int64))
                assert np.all(sources // plan.panel_width == panel)
                value = (graph.in_weight[edges].astype(np.float64)[:, None] * source[sources]).sum(0)
                if r == 0 and flags & 1:
                    value = carry + value
                if r == nrows - 1 and flags & 2:
                    carry = value
                    expected_row = row
                    continue
                partial[panel, row] = value
                written[panel, row] += 1
                expected_row = row + 1
            if flags & 4:
                assert expected_row == stripes[stripe + 1]
                stripe_done[panel, stripe] += 1
                current = None
        assert current is None, "a tile ends at a stripe boundary"
    assert np.all(seen == 1), "every edge lands in exactly one slot"
    assert np.all(written == 1), "every (panel, row) is finished exactly once"
    assert np.all(stripe_done == 1), "every (panel, stripe) completes exactly once"
    return plan, partial.sum(0)


@pytest.mark.parametrize("name", list(GRAPHS))
@pytest.mark.parametrize("batch,stripes,width,groups", [(1, 7, None, 3), (1, 3, 256, 3),
                                                         (2, 5, 1000, 2), (2, 1, 64, 1)])
def test_panel_layout_reproduces_the_csr_product(name, batch, stripes, width, groups):
    graph = GRAPHS[name]()
    if width is not None and graph.n // width > 24:
        width = -(-graph.n // 24)          # keep the python emulation to <= 24 panels
    rng = np.random.default_rng(11)
    source = rng.random((graph.n, batch))
    plan, result = emulate(graph, batch, stripes, width, source, groups)
    from scipy.sparse import csr_matrix

    matrix = csr_matrix((graph.in_weight.astype(np.float64), graph.in_col, graph.in_rowptr),
                        shape=(graph.n, graph.n))
    expected = matrix @ source
    np.testing.assert_allclose(result, expected, rtol=1e-12, atol=1e-12)


def test_hub_rows_are_split_across_chunks():
    graph = hub_graph(12_000, 2)
    plan, tiles, chunks, *_ = plan_panels_host(torch.from_numpy(graph.in_rowptr),
                                               torch.from_numpy(graph.in_col), 1, 4, None, 2)
    flags = chunks.reshape(-1, 8)[:, 5]
    assert (flags & 1).any() and (flags & 2).any()


def test_planner_rejects_bad_geometry():
    from neurosim_gpu import native

    lib = native.load_library()
    rowptr = np.array([0, 1, 2], np.int32)
    col = np.array([0, 5], np.int32)      # column out of range
    plan = native._PanelPlan()
    rows = native._c_i64()
    import ctypes

    rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, 2, 64, 1, 1, 8192, 16,
                            ctypes.byref(plan), ctypes.byref(rows), *([None] * 7))
    assert rc != 0 and b"out of range" in lib.ns_last_error()
    col = np.array([0, 1], np.int32)
    rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, 2, 64, 1, 1, 4096, 16,
                            ctypes.byref(plan), ctypes.byref(rows), *([None] * 7))
    assert rc != 0 and b"chunk_edges" in lib.ns_last_error()
