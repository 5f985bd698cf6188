"""The column-panel layout (ns_plan_panels) on the host: invariants, and a numpy
emulation of the panel kernel's decomposition against the plain CSR product.

The emulation walks every wavefront's stream as the kernel does (register
blocks of up to 16 steps, prefetch of the next block) and checks
that every slot the kernel reads lies inside the slot arrays, that every edge
lands in exactly one slot of its row and panel, that each (panel, row) is
finished exactly once, and that the per-lane sums plus the lane butterfly
reproduce the CSR product.  Covers several panels (small panel widths), hub
rows that take all 64 lanes, rows without edges, empty graphs and tiny graphs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import topology as otop
from neurosim_gpu.native import panel_geometry, plan_panels_host

MAX_BLOCK_STEPS = 16
TAIL_SLOTS = 2 * MAX_BLOCK_STEPS * 64


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


def emulate(graph: otop.Graph, batch: int, tiles_per_panel: int, width: int | None,
            source: np.ndarray, lane_target: int = 24, pairs: bool = False):
    plan, tiles, tile_ranges, wave_groups, groups, rows, last_steps, perm, cols = plan_panels_host(
        torch.from_numpy(graph.in_rowptr), torch.from_numpy(graph.in_col), batch, tiles_per_panel,
        width, lane_target, pairs)
    assert plan.flags == (1 if pairs else 0)
    if pairs:
        # slots 2i and 2i+1 hold edges of one 16-edge weight block, or padding
        pair = perm.reshape(-1, 2)
        both = (pair >= 0).all(1)
        assert np.array_equal(pair[both, 0] >> 4, pair[both, 1] >> 4)
        assert (groups.reshape(-1, 4)[:, 2] & 255).min(initial=1) >= 1, "every row has two lanes"
    n, m = graph.n, graph.n_edges
    cap, waves = panel_geometry(batch)
    W, P = plan.panel_width, plan.n_panels
    assert plan.waves == waves == 16
    assert W % 4 == 0 and W <= min(cap, width or cap)
    assert P * W >= n > (P - 1) * W
    assert perm.size == cols.size == plan.n_slots
    assert last_steps.size == plan.n_slots // 64 // 32 + 2
    step_ends = np.unpackbits(last_steps.view(np.uint8), bitorder="little").astype(bool)
    marked = np.zeros_like(step_ends)
    tiles = tiles.reshape(-1, 4)
    groups = groups.reshape(-1, 4)
    assert wave_groups.size == plan.n_tiles * waves + 1 and wave_groups[0] == 0
    assert wave_groups[-1] == plan.n_groups and np.all(np.diff(wave_groups) >= 0)
    covered = np.zeros((P, n), dtype=np.int64)
    for panel, r0, r1, entry0 in tiles:
        assert 0 <= r0 < r1 <= n and r1 - r0 <= 65536
        covered[panel, r0:r1] += 1
        # the tile's row-table entries are contiguous and list each of its rows once
        assert np.array_equal(np.sort(rows[entry0:entry0 + r1 - r0].astype(np.int64)),
                              np.arange(r1 - r0))
    assert np.all(covered == 1), "each panel's tiles partition the rows"
    # Row ranges shared by all panels: the tiles of range k are one per panel
    # and cover the same rows, and the ranges cut the rows in order.
    R = plan.n_ranges
    assert R >= 1 and plan.n_tiles == P * R and tile_ranges.size == plan.n_tiles
    assert tile_ranges.min() == 0 and tile_ranges.max() == R - 1
    bounds = []
    for k in range(R):
        mine = tiles[tile_ranges == k]
        assert np.array_equal(np.sort(mine[:, 0]), np.arange(P)), "one tile per panel"
        assert np.all(mine[:, 1] == mine[0, 1]) and np.all(mine[:, 2] == mine[0, 2])
        bounds.append((mine[0, 1], mine[0, 2]))
    assert bounds[0][0] == 0 and bounds[-1][1] == n
    assert all(bounds[k][1] == bounds[k + 1][0] for k in range(R - 1))

    rows_of_edge = np.repeat(np.arange(n), np.diff(graph.in_rowptr))
    partial = np.zeros((P, n, batch))
    written = np.zeros((P, n), dtype=np.int64)
    seen = np.zeros(m, dtype=np.int64)
    last_stream_end = 0
    for t, (panel, r0, r1, _) in enumerate(tiles):   # _: the tile's first row-table entry
        for w in range(waves):
            g0, g1 = wave_groups[t * waves + w], wave_groups[t * waves + w + 1]
            if g0 == g1:
                continue
            first = groups[g0, 0]
            total = (groups[g1 - 1, 0] - first) // 64 + groups[g1 - 1, 1]
            # furthest slot any lane reads: one block of prefetch past the last consumed block
            blocks = -(-total // MAX_BLOCK_STEPS)
            assert first + (blocks + 1) * MAX_BLOCK_STEPS * 64 <= plan.n_slots
            last_stream_end = max(last_stream_end, first + 64 * total)
            slot = first
            for g in range(g0, g1):
                slot0, steps, packed, rowtab = groups[g]
                lg, nrows = packed & 255, packed >> 8
                lanes = 1 << lg
                assert slot0 == slot and slot0 % 64 == 0, "a wave's groups are contiguous"
                assert 0 <= lg <= 6 and 1 <= nrows <= 64 >> lg and steps >= 1
                marked[slot0 // 64 + steps - 1] = True
                block = np.arange(slot0, slot0 + 64 * steps).reshape(steps, 64)
                edges = perm[block]
                srcs = cols[block].astype(np.int64)
                pad = edges < 0
                assert np.all(srcs[pad] == W), "padding reads the sentinel zero"
                for k in range(64 >> lg):
                    lane_edges = edges[:, k * lanes:(k + 1) * lanes]
                    if k >= nrows:
                        assert np.all(lane_edges < 0)
                        continue
                    row = r0 + int(rows[rowtab + k])
                    assert r0 <= row < r1 and _ <= rowtab + k < _ + r1 - r0
                    mine = lane_edges.T          # [lane j, step]: edges j, j+lanes, ...
                    order = lane_edges.reshape(-1)
                    real = order[order >= 0]
                    assert np.all(rows_of_edge[real] == row)
                    assert np.all(graph.in_col[real] // W == panel)
                    seen[real] += 1
                    lane_sums = []
                    for j in range(lanes):
                        e = mine[j][mine[j] >= 0]
                        assert np.array_equal(cols[block[:, k * lanes + j]][mine[j] >= 0].astype(np.int64),
                                              graph.in_col[e] - panel * W)
                        lane_sums.append((graph.in_weight[e].astype(np.float64)[:, None]
                                          * source[graph.in_col[e]]).sum(0))
                    while len(lane_sums) > 1:        # the xor butterfly pairs neighbours first
                        lane_sums = [lane_sums[i] + lane_sums[i + 1] for i in range(0, len(lane_sums), 2)]
                    partial[panel, row] = lane_sums[0]
                    written[panel, row] += 1
                slot += 64 * steps
    assert np.array_equal(marked, step_ends), "the bitmap marks exactly each group's last step"
    assert np.all(seen == 1), "every edge lands in exactly one slot"
    assert np.all(written == 1), "every (panel, row) is finished exactly once"
    tail = perm[last_stream_end:]
    assert tail.size >= TAIL_SLOTS and np.all(tail == -1) and np.all(cols[last_stream_end:] == W)
    return plan, partial.sum(0)


@pytest.mark.parametrize("pairs", [False, True])
@pytest.mark.parametrize("name", list(GRAPHS))
@pytest.mark.parametrize("batch,tiles,width", [(1, 3, None), (1, 5, 256), (2, 2, 1000), (2, 1, 64)])
def test_panel_layout_reproduces_the_csr_product(name, batch, tiles, width, pairs):
    graph = GRAPHS[name]()
    if width is not None and graph.n // width > 24:
        width = -(-graph.n // 24)          # keep the python emulation to <= 24 panels
    rng = np.random.default_rng(11)
    source = rng.random((graph.n, batch))
    plan, result = emulate(graph, batch, tiles, width, source, pairs=pairs)
    from scipy.sparse import csr_matrix

    matrix = csr_matrix((graph.in_weight.astype(np.float64), graph.in_col, graph.in_rowptr),
                        shape=(graph.n, graph.n))
    expected = matrix @ source
    np.testing.assert_allclose(result, expected, rtol=1e-12, atol=1e-12)


def test_lane_widths_follow_segment_length():
    graph = hub_graph(12_000, 2)
    plan, tiles, tile_ranges, wave_groups, groups, rows, last_steps, perm, cols = plan_panels_host(
        torch.from_numpy(graph.in_rowptr), torch.from_numpy(graph.in_col), 1, 4)
    lg = groups.reshape(-1, 4)[:, 2] & 255
    assert lg.max() == 6, "the 9000-edge hub row takes a whole wavefront"
    assert (lg == 0).any()


def test_waves_are_balanced_within_a_tile():
    graph = otop.random_graph(20_000, 1_000_000, seed=4)
    plan, tiles, tile_ranges, wave_groups, groups, rows, last_steps, perm, cols = plan_panels_host(
        torch.from_numpy(graph.in_rowptr), torch.from_numpy(graph.in_col), 1, 8)
    cost = groups.reshape(-1, 4)[:, 1] + 1
    for t in range(plan.n_tiles):
        loads = [cost[wave_groups[t * 16 + w]: wave_groups[t * 16 + w + 1]].sum() for w in range(16)]
        assert max(loads) <= 1.1 * np.mean(loads) + max(cost)


def test_planner_rejects_bad_geometry():
    from neurosim_gpu import native

    lib = native.load_library()
    rowptr = np.array([0, 1, 2], np.int32)
    col = np.array([0, 5], np.int32)      # column out of range
    plan = native._PanelPlan()
    entries = native._c_i64()
    import ctypes

    rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, 2, 64, 1, 16, 12, 0,
                            ctypes.byref(plan), ctypes.byref(entries), *([None] * 8))
    assert rc != 0 and b"out of range" in lib.ns_last_error()
    col = np.array([0, 1], np.int32)
    rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, 2, 64, 1, 8, 12, 0,
                            ctypes.byref(plan), ctypes.byref(entries), *([None] * 8))
    assert rc != 0 and b"wavefronts" in lib.ns_last_error()
    # NS_PANEL_COMBINE_LAUNCH (2) is the caller's to set on a plan, not a layout flag
    for flags in (2, 4):
        rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, 2, 64, 1, 16, 12, flags,
                                ctypes.byref(plan), ctypes.byref(entries), *([None] * 8))
        assert rc != 0 and b"flags" in lib.ns_last_error()


@pytest.mark.parametrize("flags", [0, 1])
@pytest.mark.parametrize("rowptr,col,bad", [
    ([0, 1, 2], [0, -1], -1),                                  # -1: no longer a 'no error' value
    ([0, 1, 2], [-7, 1], -7),
    ([0] + list(range(5, 5 * 13, 5)), [4, 4, 4, 8, -1] * 12, -1),   # 12 rows, several panels
])
def test_planner_rejects_negative_and_large_columns(flags, rowptr, col, bad):
    import ctypes

    from neurosim_gpu import native

    lib = native.load_library()
    rowptr = np.asarray(rowptr, np.int32)
    n = rowptr.size - 1
    col = np.asarray(col, np.int32)
    plan = native._PanelPlan()
    entries = native._c_i64()
    rc = lib.ns_plan_panels(rowptr.ctypes.data, col.ctypes.data, n, 4, 1, 16, 12, flags,
                            ctypes.byref(plan), ctypes.byref(entries), *([None] * 8))
    message = lib.ns_last_error()
    assert rc != 0 and b"out of range" in message
    first = int(np.flatnonzero((col < 0) | (col >= n))[0])
    assert f"column {bad} out of range (edge {first})".encode() in message


@pytest.mark.parametrize("pairs", [False, True])
def test_panel_plan_does_not_depend_on_thread_count(monkeypatch, pairs):
    """Rows are laid out in chunks of 4096 on up to 16 host threads; a graph of
    many chunks must give the same plan as a one-thread build."""
    graph = hub_graph(70_000, 5)
    plans = []
    for threads in ("1", "16"):
        monkeypatch.setenv("NEUROSIM_PLAN_THREADS", threads)
        plans.append(plan_panels_host(torch.from_numpy(graph.in_rowptr),
                                      torch.from_numpy(graph.in_col), 1, 37, 4000, pairs=pairs))
    one, many = plans
    for field in ("panel_width", "n_panels", "n_tiles", "n_groups", "n_ranges", "n_slots",
                  "n_step_words"):
        assert getattr(one[0], field) == getattr(many[0], field)
    for x, y in zip(one[1:], many[1:]):
        assert np.array_equal(x, y)
