"""The source-band layout (ns_plan_bands) on the host: invariants, and a numpy
emulation of the band kernel's decomposition against the plain CSR product.

The invariants: every edge lands in exactly one slot, with its band-local
source index; a wavefront's register blocks walk the bands in order, their
slots contiguous, each block spanning `block_steps` steps with its slots
lane-major (lane l's steps consecutive) and padding past its step count, each
record carrying its first step within the group; a
group's lane takes its first row's segment of the band in CSR order and, from
its switch step on, possibly a second row's; the group lasts as long as its
longest first segment, and its last block is marked; each row of a block
meets each band in one group (of one wavefront) at most; the wavefronts' steps
in a band differ by no more than one group's; the tables end with the sentinel
block, the sentinel group and the tail padding.  The emulation follows the
kernel's summation order (per row: bands in order, the workgroup passing a
barrier after each; within a band the segment's edges one at a time) and must
reproduce the CSR product.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from neurosim_gpu import native
from neurosim_gpu.native import band_max_block_rows, plan_bands_host

PAD = 0xFFFF
NO_ROW = 0xFFF
WAVES = native.BAND_WAVES
TAIL = 8 * 64


def lane_rows(word):
    """(first row, second row, switch step) of a lane word."""
    word = int(word)
    return word & NO_ROW, (word >> 12) & NO_ROW, word >> 24


def random_csr(n, m, seed, hubs=()):
    rng = np.random.default_rng(seed)
    dst = [rng.integers(0, n, m)]
    src = [rng.integers(0, n, m)]
    for row, length in hubs:
        dst.append(np.full(length, row))
        src.append(rng.integers(0, n, length))
    dst, src = np.concatenate(dst), np.concatenate(src)
    order = np.argsort(dst, kind="stable")
    dst, src = dst[order], src[order]
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=n))
    return rowptr.astype(np.int32), src.astype(np.int32)


def layout(rowptr, col, width, rows, steps):
    plan, wave_blocks, blocks, group_rows, perm, cols = plan_bands_host(
        torch.from_numpy(rowptr), torch.from_numpy(col), width, rows, steps)
    return plan, wave_blocks, blocks.reshape(-1, 4), group_rows.reshape(-1, 64), perm, cols


CASES = [
    (500, 6000, 3, (), 64, 100, 8),
    (3000, 40000, 4, ((7, 900), (2999, 2500)), 333, 257, 4),
    (2000, 30000, 5, ((0, 4000),), 2000, 2000, 8),      # one band, one block
    (1000, 0, 6, (), 100, 64, 8),                       # no edges
    (4000, 20000, 7, (), 50, 1, 8),                     # one row per block
    (12000, 96000, 8, ((0, 9000), (3, 6000)), 2000, 4095, 8),  # 12-bit row limit
]


@pytest.mark.parametrize("n,m,seed,hubs,width,rows,steps", CASES)
def test_band_layout_invariants(n, m, seed, hubs, width, rows, steps):
    rowptr, col = random_csr(n, m, seed, hubs)
    edges = int(rowptr[-1])
    plan, wave_blocks, blocks, group_rows, perm, cols = layout(rowptr, col, width, rows, steps)
    n_bands = -(-n // width)
    n_row_blocks = -(-n // rows)
    assert (plan.n_bands, plan.n_row_blocks, plan.block_rows, plan.band_width) == (
        n_bands, n_row_blocks, rows, width)
    assert wave_blocks.size == WAVES * n_row_blocks + 1 and wave_blocks[0] == 0
    assert wave_blocks[-1] == plan.n_blocks and np.all(np.diff(wave_blocks) >= 0)
    assert blocks.shape == (plan.n_blocks + 1, 4) and group_rows.shape == (plan.n_groups, 64)
    assert perm.size == cols.size == plan.n_slots

    # every edge in exactly one slot, with its band-local source index
    real = perm >= 0
    assert np.array_equal(np.sort(perm[real]), np.arange(edges))
    assert np.all(cols[~real] == PAD)

    # sentinel block, sentinel group, tail padding
    assert tuple(blocks[-1]) == (0, 0, 0, plan.n_groups - 1)
    assert np.all(group_rows[-1] == NO_ROW | NO_ROW << 12)
    assert np.all(perm[-TAIL:] == -1)

    row_of_edge = np.repeat(np.arange(n), np.diff(rowptr))
    segments = {}
    for e in range(edges):
        segments.setdefault((int(row_of_edge[e]), int(col[e]) // width), []).append(e)
    step = 0
    for q in range(n_row_blocks):
        r0 = q * rows
        seen_bands = {}
        band_steps = np.zeros((n_bands, WAVES), np.int64)
        group_steps = np.zeros(n_bands, np.int64)
        for w in range(WAVES):
            prev_band = -1
            b = wave_blocks[WAVES * q + w]
            while b < wave_blocks[WAVES * q + w + 1]:
                # one group: consecutive blocks of one group and band, the last marked
                group, band = blocks[b, 3], blocks[b, 1]
                assert band >= prev_band
                prev_band = band
                lanes = [lane_rows(word) for word in group_rows[group]]
                seg = lambda r: segments.get((r0 + r, int(band)), [])
                members = []
                for first, second, switch in lanes:
                    if first == NO_ROW:
                        assert (second, switch) == (NO_ROW, 0)
                        continue
                    members.append(first)
                    if second == NO_ROW:
                        assert switch == 0
                    else:
                        assert switch == len(seg(first)) and switch <= 255
                        members.append(second)
                assert len(set(members)) == len(members)
                for r in members:
                    assert 0 <= r < min(rows, n - r0)
                    assert (r0 + r, band) not in seen_bands                 # one group per band
                    seen_bands[(r0 + r, band)] = True
                    assert len(seg(r)) > 0
                t = 0
                while True:
                    start, bband, info, bgroup = blocks[b]
                    assert (bband, bgroup) == (band, group) and start == step
                    count, last, t0 = info & 0xFF, (info >> 8) & 1, info >> 9
                    assert 1 <= count <= steps and t0 == t
                    assert last or count == steps
                    for k in range(count, steps):                 # padding past the count
                        slots = 64 * start + np.arange(64) * steps + k
                        assert np.all(perm[slots] == -1) and np.all(cols[slots] == PAD)
                    for k in range(count):
                        slots = 64 * start + np.arange(64) * steps + k      # lane-major
                        for lane, (first, second, switch) in enumerate(lanes):
                            e = perm[slots[lane]]
                            expected = -1
                            if first != NO_ROW and t + k < len(seg(first)):
                                expected = seg(first)[t + k]
                            elif second != NO_ROW and 0 <= t + k - switch < len(seg(second)):
                                expected = seg(second)[t + k - switch]
                            assert e == expected
                            if e >= 0:
                                assert cols[slots[lane]] == col[e] - band * width
                    step += steps
                    t += count
                    b += 1
                    if last:
                        break
                # the group lasts as long as its longest first segment (lane 0's);
                # a second segment fits in the steps after its lane's first
                assert t == len(seg(lanes[0][0]))
                for first, second, switch in lanes:
                    if first != NO_ROW:
                        assert len(seg(first)) + (len(seg(second)) if second != NO_ROW else 0) <= t
                band_steps[band, w] += t
                group_steps[band] = max(group_steps[band], t)
        # each group went to the wavefront with the fewest steps in its band
        assert np.all(band_steps.max(axis=1) - band_steps.min(axis=1) <= group_steps)
    assert 64 * step + TAIL == plan.n_slots


@pytest.mark.parametrize("n,m,seed,hubs,width,rows,steps", CASES)
def test_band_emulation_matches_csr_product(n, m, seed, hubs, width, rows, steps):
    rowptr, col = random_csr(n, m, seed, hubs)
    rng = np.random.default_rng(seed + 100)
    weight = (rng.standard_normal(col.size) * 0.05).astype(np.float32)
    s = rng.random((n, 16), dtype=np.float32)
    plan, wave_blocks, blocks, group_rows, perm, cols = layout(rowptr, col, width, rows, steps)
    padded = np.concatenate([weight, np.zeros(1, np.float32)])     # index -1: padding weight 0
    slot_w = padded[perm]
    sums = np.zeros((n, 16), np.float32)
    for q in range(plan.n_row_blocks):
        r0 = q * rows
        for band_now, w in ((k, w) for k in range(plan.n_bands) for w in range(WAVES)):
            acc = np.zeros((64, 16), np.float32)
            for b in range(wave_blocks[WAVES * q + w], wave_blocks[WAVES * q + w + 1]):
                start, band, info, group = blocks[b]
                if band != band_now:
                    continue
                lanes = [lane_rows(word) for word in group_rows[group]]
                for k in range(info & 0xFF):
                    slots = 64 * start + np.arange(64) * steps + k
                    c = cols[slots].astype(np.int64)
                    real = c != PAD
                    g = np.zeros((64, 16), np.float32)
                    g[real] = s[band * width + c[real]]
                    acc += slot_w[slots][:, None] * g
                    for lane, (first, second, switch) in enumerate(lanes):
                        if (info >> 9) + k + 1 == switch:       # the lane moves to its second row
                            sums[r0 + first] += acc[lane]
                            acc[lane] = 0
                if (info >> 8) & 1:
                    for lane, (first, second, switch) in enumerate(lanes):
                        row = second if second != NO_ROW else first
                        if row != NO_ROW:
                            sums[r0 + row] += acc[lane]
                    acc[:] = 0
    expected = np.zeros((n, 16), np.float64)
    np.add.at(expected, np.repeat(np.arange(n), np.diff(rowptr)),
              weight.astype(np.float64)[:, None] * s.astype(np.float64)[col])
    assert np.allclose(sums, expected, rtol=1e-5, atol=1e-5)


def test_band_planner_rejects_bad_arguments():
    lib = native.load_library()
    rowptr, col = random_csr(100, 500, 1)
    plan = native._BandPlan()

    def rc(rp=rowptr, c=col, n=100, width=10, rows=16, steps=8):
        code = lib.ns_plan_bands(rp.ctypes.data, c.ctypes.data, n, width, rows, steps,
                                 ctypes.byref(plan), None, None, None, None, None)
        return code, lib.ns_last_error().decode()

    assert rc()[0] == 0
    assert "band_width" in rc(width=0)[1] and "band_width" in rc(width=65536)[1]
    assert "block_rows" in rc(rows=0)[1]
    assert "block_rows" in rc(rows=band_max_block_rows(8) + 1)[1]
    assert "block_steps" in rc(steps=0)[1] and "block_steps" in rc(steps=9)[1]
    bad = rowptr.copy()
    bad[5] = bad[6] + 1
    assert "non-decreasing" in rc(rp=bad)[1]
    bad_col = col.copy()
    bad_col[3] = 100
    assert "out of range" in rc(c=bad_col)[1]
    assert "N must be" in rc(n=0)[1]
    bad_col[3] = -1
    assert "out of range" in rc(c=bad_col)[1]


def test_band_plan_does_not_depend_on_thread_count(monkeypatch):
    """Row blocks are laid out on up to 16 host threads and concatenated in order."""
    rowptr, col = random_csr(40_000, 400_000, 9, ((5, 3000),))
    plans = []
    for threads in ("1", "16"):
        monkeypatch.setenv("NEUROSIM_PLAN_THREADS", threads)
        plans.append(plan_bands_host(torch.from_numpy(rowptr), torch.from_numpy(col), 4096, 300, 4))
    one, many = plans
    for field in ("n_bands", "n_row_blocks", "n_blocks", "n_groups", "n_slots"):
        assert getattr(one[0], field) == getattr(many[0], field)
    for x, y in zip(one[1:], many[1:]):
        assert np.array_equal(x, y)


def test_band_padding_at_scale_out_density():
    """About 3.3 edges per (row, band), as at N=1M, M=100M with bands of 32,768
    sources (the default 53,248 gives 5.3, with less padding), and 1954-row
    blocks of 16 wavefronts, as there: with a block's rows pooled per band and
    a second row per lane where one fits, the groups' steps hold at most 1.05
    lanes per edge (rows dealt to the wavefronts first: 1.13; one row per lane:
    about 1.48).  Blocks padded to whole register blocks of 4 steps add the rest
    of the slots: 1.39 slots per edge in all here, where groups are short."""
    rng = np.random.default_rng(5)
    n, m = 100_000, 10_000_000
    dst = np.sort(rng.integers(0, n, m))
    rowptr = np.zeros(n + 1, np.int64)
    rowptr[1:] = np.cumsum(np.bincount(dst, minlength=n))
    col = rng.integers(0, n, m).astype(np.int32)
    plan, _, blocks, *_ = plan_bands_host(torch.from_numpy(rowptr.astype(np.int32)),
                                          torch.from_numpy(col), 3277, 1954, 4)
    lanes = 64 * int((blocks.reshape(-1, 4)[:-1, 2] & 0xFF).sum()) / m
    slots = (plan.n_slots - TAIL) / m
    print(f"lanes per edge {lanes:.3f}, slots per edge {slots:.3f}")
    assert lanes <= 1.05 and slots <= 1.45


def test_auto_picks_bands_by_tile_bytes():
    """"auto" takes bands for batches that are multiples of 4 once a workgroup's
    column tile of the state (16 columns, or 8 or 4 for odd multiples of 8 or 4)
    holds 4 MB."""
    from neurosim_gpu.native_compartmental import (band_tile_columns, bands_pay_off,
                                                   default_band_steps)

    assert [band_tile_columns(b) for b in (4, 8, 12, 16, 24, 32, 48)] == [4, 8, 4, 16, 8, 16, 16]
    assert bands_pay_off(262_144, 4) and not bands_pay_off(262_143, 4)
    assert bands_pay_off(65_536, 16) and not bands_pay_off(65_535, 16)
    assert bands_pay_off(131_072, 8) and not bands_pay_off(131_071, 8)
    assert bands_pay_off(131_072, 24) and bands_pay_off(1_000_000, 8)
    assert not bands_pay_off(50_000, 8)
    assert not any(bands_pay_off(1_000_000, b) for b in (0, 1, 2, 6, 10))
    assert [default_band_steps(b) for b in (4, 8, 12, 16, 24, 32)] == [8, 8, 8, 4, 8, 4]
