"""The column-panel tick (batch 1 and 2) on the MI355X.

Several panels are forced with small panel widths so the per-panel partial
sums and their combination (in the tick kernel's last tile of each row range,
or in a second kernel) run on small graphs; hub rows take whole
wavefronts (64 lanes per row) and rows of every length class mix in one tile.  Bars: float32 within 1e-5 of the
oracle; fp16/fp8/nvfp4 storage bitwise equal to the panel tick on the
decoded float32 weights; bitwise repeatable.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import column_drive, make_case, max_err, model_to, standard_model
from oracle import precision as op
from oracle import runtime as ort
from oracle import topology as otop
from neurosim_gpu import NativeDendriticMatrixRuntime, SparseTopology, topology_to
from neurosim_gpu.native import PanelLayout

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


def errors(native, oracle) -> float:
    return max(max_err(getattr(native, f), getattr(oracle, f)) for f in FIELDS)


def hub_case(gpu, n=12_000, seed=2):
    """Random rows plus two hub rows (9000 and n/2 edges)."""
    rng = np.random.default_rng(seed)
    hub = min(n, 9000)
    dst = np.concatenate([np.zeros(hub, np.int64), np.full(n // 2, 3), rng.integers(0, n, 8 * n)])
    src = np.concatenate([np.arange(hub), rng.permutation(n)[: n // 2], rng.integers(0, n, 8 * n)])
    weight = (rng.standard_normal(dst.size) * 0.01).astype(np.float32)
    graph = otop.build(n, src, dst, weight)
    topology = SparseTopology.from_edges(n, torch.from_numpy(src), torch.from_numpy(dst),
                                         torch.from_numpy(weight))
    model, params = standard_model(n)
    return graph, topology_to(topology, gpu), model_to(model, gpu), params


@pytest.mark.parametrize("pairs", [False, True])
@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("width,tiles", [(None, None), (1000, 7), (256, 2)])
def test_panels_match_oracle(gpu, batch, width, tiles, pairs):
    print(f"case panels batch={batch} width={width} tiles={tiles} pairs={pairs}", flush=True)
    graph, topology, model, params = hub_case(gpu)
    drive = column_drive(batch)
    native = NativeDendriticMatrixRuntime(topology, model, torch.zeros(batch, graph.n, device=gpu),
                                          kernel="panels", panel_width=width, panel_tiles=tiles,
                                          panel_pairs=pairs)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, graph.n))
    assert native.kernel == "panels"
    worst = 0.0
    for _ in range(30):
        native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        worst = max(worst, errors(native, oracle))
    print(f"panels batch={batch} width={width}: {worst:.3e} over 30 ticks "
          f"({native._panels.n_panels} panels, {native._panels.n_tiles} tiles)")
    assert worst <= 1e-5


@pytest.mark.parametrize("fmt", ["fp32", "nvfp4"])
@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("width,tiles", [(1000, 7), (256, 3), (4096, 40)])
def test_one_launch_equals_combine_launch(gpu, batch, width, tiles, fmt):
    """The tick kernel's last tile of each row range adds the panels' sums and
    updates the range (one launch per tick); a second kernel doing the same
    (NS_PANEL_COMBINE_LAUNCH) must give bitwise the same states every tick,
    and every launch leaves the range counters zero."""
    print(f"case one-launch batch={batch} width={width} tiles={tiles} fmt={fmt}", flush=True)
    graph, topology, model, params = hub_case(gpu)
    kwargs = {"weight_format": "nvfp4"} if fmt == "nvfp4" else {}
    runs = []
    for combine in (False, True):
        native = NativeDendriticMatrixRuntime(topology, model,
                                              torch.zeros(batch, graph.n, device=gpu),
                                              kernel="panels", panel_width=width,
                                              panel_tiles=tiles, **kwargs)
        if combine:
            native._panels = PanelLayout(topology, batch, gpu, tiles_per_panel=tiles,
                                         max_panel_width=width, pairs=native._panels.pairs,
                                         combine_launch=True)
        runs.append(native)
    one, two = runs
    if one._panels.combine_launch:       # ranges too long for one launch by default
        one._panels = PanelLayout(topology, batch, gpu, tiles_per_panel=tiles,
                                  max_panel_width=width, pairs=one._panels.pairs,
                                  combine_launch=False)
    assert one._panels.n_panels > 1 and not one._panels.combine_launch
    assert one._panels.n_tiles == one._panels.n_panels * one._panels.n_ranges
    drive = column_drive(batch).to(gpu)
    for tick in range(40):
        for native in runs:
            native.step(drive if tick < 20 else 0.05, dendritic_drive=0.1)
        for field in FIELDS:
            assert torch.equal(getattr(one, field), getattr(two, field)), (tick, field)
    assert int(one._panels.range_counters.abs().sum()) == 0
    print(f"one launch: {one._panels.n_panels} panels x {one._panels.n_ranges} ranges bitwise equal")


@pytest.mark.parametrize("batch", [1, 2])
def test_panels_and_rows_agree_and_repeat(gpu, batch):
    case = make_case(20_000, 400_000, 5, gpu)
    runs = {}
    for kernel in ("panels", "rows", "panels"):
        native = NativeDendriticMatrixRuntime(case.topology, case.model,
                                              torch.zeros(batch, 20_000, device=gpu), kernel=kernel,
                                              panel_width=4096)
        for _ in range(25):
            native.step(0.2, dendritic_drive=0.1)
        if kernel in runs:
            assert torch.equal(native.state, runs[kernel].state)      # bitwise repeatable
        runs[kernel] = native
    assert errors(runs["panels"], runs["rows"]) <= 2e-6


@pytest.mark.parametrize("fmt", ["fp16", "fp8", "nvfp4"])
@pytest.mark.parametrize("batch", [1, 2])
def test_panel_formats_equal_decoded_fp32(gpu, fmt, batch):
    graph, topology, model, params = hub_case(gpu, n=6000, seed=9)
    kwargs = {"weight_dtype": torch.float16} if fmt == "fp16" else {"weight_format": fmt}
    native = NativeDendriticMatrixRuntime(topology, model, torch.zeros(batch, 6000, device=gpu),
                                          kernel="panels", panel_width=1024, panel_tiles=5,
                                          **kwargs)
    native._weights()
    if fmt == "fp16":
        decoded_host = topology.in_weight.half().float().cpu().numpy()
    else:
        codes, *scales = native._packed_weight
        block = scales[0].cpu().numpy() if fmt == "nvfp4" else None
        decoded_host = op.decode_packed(codes.cpu().numpy(), block, np.float32(scales[-1].item()),
                                        topology.n_edges, fmt)
    decoded = SparseTopology.from_edges(
        6000, topology.src, topology.dst,
        torch.from_numpy(decoded_host).to(gpu)[topology.out_weight_index.long()])
    # the same layout as the packed runtime (NVFP4 defaults to the pair layout)
    reference = NativeDendriticMatrixRuntime(decoded, model, torch.zeros(batch, 6000, device=gpu),
                                             kernel="panels", panel_width=1024, panel_tiles=5,
                                             panel_pairs=native._panels.pairs)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, 6000), in_weight=decoded_host)
    for _ in range(10):
        native.step(0.2, dendritic_drive=0.1)
        reference.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
        for field in FIELDS:
            assert torch.equal(getattr(native, field), getattr(reference, field))
    assert errors(native, oracle) <= 1e-5


@pytest.mark.parametrize("batch", [1, 2])
def test_nvfp4_pair_layout_is_the_default_and_matches_per_slot_scales(gpu, batch):
    """NVFP4 on the pair layout (one scale byte per slot pair) against NVFP4 on the
    plain layout (one per slot): the same decoded weights, so the same states up to
    summation order (the layouts differ), and both within 1e-5 of the oracle."""
    graph, topology, model, params = hub_case(gpu, n=6000, seed=9)
    runs = {}
    for pairs in (None, False):
        runs[pairs] = NativeDendriticMatrixRuntime(
            topology, model, torch.zeros(batch, 6000, device=gpu), kernel="panels",
            panel_width=1024, panel_tiles=5, weight_format="nvfp4", panel_pairs=pairs)
    assert runs[None]._panels.pairs and not runs[False]._panels.pairs
    runs[None]._weights()
    codes, block, scale = runs[None]._packed_weight
    decoded_host = op.decode_packed(codes.cpu().numpy(), block.cpu().numpy(),
                                    np.float32(scale.item()), topology.n_edges, "nvfp4")
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, 6000), in_weight=decoded_host)
    for _ in range(10):
        for native in runs.values():
            native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
    assert errors(runs[None], runs[False]) <= 2e-6
    assert errors(runs[None], oracle) <= 1e-5


def test_panel_fp32_follows_in_place_edits_of_in_weight(gpu):
    """The reference's fp32 tick reads in_weight on every tick, so an in-place edit
    of in_weight (no topology weight version bump) takes effect at once; the
    panel path's slot-order copy is keyed on the tensor's version counter."""
    case = make_case(3000, 60_000, 4, gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 3000, device=gpu),
                                          kernel="panels", panel_width=512, panel_tiles=4)
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(1, 3000))
    for tick in range(8):
        if tick == 4:
            with torch.no_grad():
                case.topology.in_weight.mul_(0.5)
            oracle.matrix = ort.csr_matrix(case.graph, torch.float32,
                                           case.topology.in_weight.cpu().numpy())
        native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
    assert errors(native, oracle) <= 1e-5


def test_panel_fp32_warns_once_about_inference_mode_weights(gpu):
    """An in_weight made under torch.inference_mode has no version counter, so the
    slot-order copy cannot see an in-place edit: the runtime says so, once; after
    mark_weights_mutated_() the edit takes effect.  Versioned weights do not warn."""
    import dataclasses
    import warnings

    case = make_case(3000, 60_000, 4, gpu)
    with torch.inference_mode():
        frozen = case.topology.in_weight.clone()
    topology = dataclasses.replace(case.topology, in_weight=frozen)
    native = NativeDendriticMatrixRuntime(topology, case.model, torch.zeros(1, 3000, device=gpu),
                                          kernel="panels", panel_width=512, panel_tiles=4)
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(1, 3000))
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        for tick in range(8):
            if tick == 4:
                with torch.inference_mode():
                    frozen.mul_(0.5)
                topology.mark_weights_mutated_()
                oracle.matrix = ort.csr_matrix(case.graph, torch.float32, frozen.cpu().numpy())
            native.step(0.2, dendritic_drive=0.1)
            oracle.step(0.2, 0.1)
    notes = [w for w in caught if "inference_mode" in str(w.message)]
    assert len(notes) == 1 and issubclass(notes[0].category, RuntimeWarning)
    assert errors(native, oracle) <= 1e-5
    versioned = NativeDendriticMatrixRuntime(case.topology, case.model,
                                             torch.zeros(1, 3000, device=gpu), kernel="panels",
                                             panel_width=512, panel_tiles=4)
    with warnings.catch_warnings(record=True) as caught:
        warnings.simplefilter("always")
        versioned.step(0.2, dendritic_drive=0.1)
    assert not [w for w in caught if "inference_mode" in str(w.message)]


@pytest.mark.parametrize("batch", [1, 2])
@pytest.mark.parametrize("width,tiles,pairs", [(None, None, False), (1000, 7, False),
                                               (256, 2, True)])
def test_indexed_first_tick_equals_the_slot_copy(gpu, batch, width, tiles, pairs):
    """The first panel tick of a float32 weight version reads in_weight in CSR order
    through the slots' edge numbers (NS_PANEL_INDEXED); the ticks after it read the
    slot-order copy.  Same layout, same sums: bitwise equal every tick, through
    several weight changes, and within 1e-5 of the oracle."""
    print(f"case indexed panels batch={batch} width={width} tiles={tiles} pairs={pairs}",
          flush=True)
    graph, topology, model, params = hub_case(gpu)
    drive = column_drive(batch)
    runs = []
    for indexed in (True, False):
        native = NativeDendriticMatrixRuntime(topology, model,
                                              torch.zeros(batch, graph.n, device=gpu),
                                              kernel="panels", panel_width=width,
                                              panel_tiles=tiles, panel_pairs=pairs)
        native.indexed_first_tick = indexed
        runs.append(native)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, graph.n))
    indexed_ticks = 0
    for tick in range(15):
        if tick in (4, 5, 9):
            topology.apply_source_weights_(topology.weight * 0.9)
            oracle.matrix = ort.csr_matrix(otop.with_weights(graph, topology.weight.cpu().numpy()))
        for native in runs:
            native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        indexed_ticks += runs[0]._panel_struct_key != runs[0]._indexed_key
        for field in FIELDS:
            assert torch.equal(getattr(runs[0], field), getattr(runs[1], field)), (tick, field)
    assert indexed_ticks == 4        # ticks 0, 4, 5 and 9 began a weight version
    assert errors(runs[0], oracle) <= 1e-5


def test_panel_weight_refresh_after_mutation(gpu):
    case = make_case(3000, 60_000, 4, gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 3000, device=gpu),
                                          kernel="panels", panel_width=512, panel_tiles=4)
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(1, 3000))
    for tick in range(12):
        if tick == 6:
            case.topology.apply_source_weights_(case.topology.weight * 0.7)
            oracle.matrix = ort.csr_matrix(otop.with_weights(case.graph,
                                                             case.topology.weight.cpu().numpy()))
        native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
    assert errors(native, oracle) <= 1e-5


@pytest.mark.parametrize("pairs", [False, True])
def test_slot_gather_matches_host_emulation(gpu, pairs):
    """ns_gather_slot_weights against a numpy restatement of the slot order:
    slot k holds edge perm[k] (padding: code 0); NVFP4 nibbles two per byte,
    scales one per slot or, in pairs, the pair's first real edge's code."""
    print(f"case slot gather pairs={pairs}", flush=True)
    graph, topology, model, params = hub_case(gpu, n=6000, seed=9)
    layout = PanelLayout(topology, 1, gpu, tiles_per_panel=5, max_panel_width=1024, pairs=pairs)
    perm = layout.perm.cpu().numpy()
    real = perm >= 0
    edge = np.where(real, perm, 0)
    weight32 = topology.in_weight
    from neurosim_gpu.native import encode_weights
    codes, block, _ = encode_weights(weight32, "nvfp4")
    fp8, _, _ = encode_weights(weight32, "fp8")
    for payload in (weight32, weight32.half(), fp8):
        slots, scales = layout.slot_weights(("t", payload.dtype), payload, None)
        host = payload.cpu().numpy()
        expected = np.where(real, host[edge], np.zeros((), host.dtype))
        assert scales is None and np.array_equal(slots.cpu().numpy(), expected)
    slots, scales = layout.slot_weights(("t", "nvfp4"), codes, block)
    c, b = codes.cpu().numpy(), block.cpu().numpy()
    nib = np.where(real, (c[edge >> 1] >> ((edge & 1) * 4)) & 15, 0).astype(np.uint8)
    packed = nib[0::2] | (nib[1::2] << 4)
    if pairs:
        first = np.where(real[0::2], edge[0::2], edge[1::2])
        code = np.where(real[0::2] | real[1::2], b[first >> 4], 0).astype(np.uint16)
        word = packed.astype(np.uint16) | (code << 8)
        assert scales is None
        assert np.array_equal(slots.cpu().numpy().view(np.uint16), word)
    else:
        assert np.array_equal(slots.cpu().numpy(), packed)
        assert np.array_equal(scales.cpu().numpy(), np.where(real, b[edge >> 4], 0))
