"""The source-band tick (batch a multiple of 4: workgroups of 16 state columns
when the batch is a multiple of 16, else of 8 or 4) on the MI355X.

Small band widths and row blocks force many bands, many row blocks and short
register blocks on small graphs; hub rows give segments of hundreds to
thousands of steps, and rows of every length mix in one group.  Bars: float32
within 1e-5 of the oracle; fp16/fp8/nvfp4 storage bitwise equal to the band
tick on the decoded float32 weights; bitwise repeatable; a graph-captured
rollout bitwise equal to eager ticks.
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
from neurosim_gpu.native import band_max_block_rows as native_band_limit
from neurosim_gpu.rollout import MatrixRollout

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


def band_runtime(topology, model, state, **kwargs):
    native = NativeDendriticMatrixRuntime(topology, model, state, kernel="bands", **kwargs)
    assert native.kernel == "bands"
    return native


@pytest.mark.parametrize("batch", [4, 8, 12, 16, 24, 32])
@pytest.mark.parametrize("width,rows,steps", [(None, None, 8), (1000, 256, 8), (512, 64, 4),
                                              (4096, 2496, 8), (777, 1001, 4), (640, 128, 2),
                                              (333, 32, 4)])   # 375 row blocks, two rounds
def test_bands_match_oracle(gpu, batch, width, rows, steps):
    print(f"case bands batch={batch} width={width} rows={rows} steps={steps}", flush=True)
    graph, topology, model, params = hub_case(gpu)
    drive = column_drive(batch)
    native = band_runtime(topology, model, torch.zeros(batch, graph.n, device=gpu),
                          band_width=width, band_rows=rows, band_steps=steps)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, graph.n))
    worst = 0.0
    for _ in range(30):
        native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        worst = max(worst, errors(native, oracle))
    layout = native._bands
    print(f"bands batch={batch} width={width}: {worst:.3e} over 30 ticks ({layout.n_bands} bands, "
          f"{layout.n_row_blocks} row blocks, {layout.n_blocks} register blocks)")
    assert worst <= 1e-5


@pytest.mark.parametrize("batch", [4, 8, 12, 24])
@pytest.mark.parametrize("width", [None, 2000])
def test_bands_at_the_largest_row_block(gpu, batch, width):
    """8- and 4-column tiles (batch 24 and 8, 12 and 4) at 4095 rows per block, the
    most a lane word's 12-bit row index holds next to the 0xFFF no-row sentinel:
    the hub graph's first two blocks use row indices up to 4094, and its short
    rows take second rows in their lanes."""
    rows = 4095
    assert native_band_limit(batch) >= rows
    print(f"case bands batch={batch} width={width} rows={rows}", flush=True)
    graph, topology, model, params = hub_case(gpu)
    drive = column_drive(batch)
    native = band_runtime(topology, model, torch.zeros(batch, graph.n, device=gpu),
                          band_width=width, band_rows=rows)
    assert native._bands.block_rows == rows and native._bands.n_row_blocks == 3
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, graph.n))
    worst = 0.0
    for _ in range(30):
        native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        worst = max(worst, errors(native, oracle))
    print(f"bands batch={batch} width={width} rows={rows}: {worst:.3e} over 30 ticks")
    assert worst <= 1e-5


@pytest.mark.parametrize("batch", [4, 8, 16])
def test_bands_and_rows_agree_and_repeat(gpu, batch):
    case = make_case(20_000, 400_000, 5, gpu)
    runs = {}
    for kernel in ("bands", "rows", "bands"):
        native = NativeDendriticMatrixRuntime(case.topology, case.model,
                                              torch.zeros(batch, 20_000, device=gpu),
                                              kernel=kernel, band_width=2048, band_rows=300)
        for _ in range(25):
            native.step(column_drive(batch).to(gpu), dendritic_drive=0.1)
        if kernel in runs:
            assert torch.equal(native.state, runs[kernel].state)      # bitwise repeatable
        runs[kernel] = native
    assert errors(runs["bands"], runs["rows"]) <= 2e-6


@pytest.mark.parametrize("batch,steps", [(4, None), (8, None), (16, None), (4, 2), (16, 2)])
@pytest.mark.parametrize("fmt", ["fp16", "fp8", "nvfp4"])
def test_band_formats_equal_decoded_fp32(gpu, fmt, batch, steps):
    """Each format's lane runs (source indices, weight codes, NVFP4 nibbles and block
    scales) at the default register depth and at 2 steps (runs of 1 to 4 bytes)."""
    graph, topology, model, params = hub_case(gpu, n=6000, seed=9)
    kwargs = {"weight_dtype": torch.float16} if fmt == "fp16" else {"weight_format": fmt}
    native = band_runtime(topology, model, torch.zeros(batch, 6000, device=gpu), band_width=1024,
                          band_rows=500, band_steps=steps, **kwargs)
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
    reference = band_runtime(decoded, model, torch.zeros(batch, 6000, device=gpu),
                             band_width=1024, band_rows=500, band_steps=steps)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, 6000), in_weight=decoded_host)
    drive = column_drive(batch)
    for _ in range(10):
        native.step(drive.to(gpu), dendritic_drive=0.1)
        reference.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        for field in FIELDS:
            assert torch.equal(getattr(native, field), getattr(reference, field))
    assert errors(native, oracle) <= 1e-5


def test_band_state_layouts_drives_and_weight_refresh(gpu):
    """A state that is not neuron-major (copied once), [B,N] drive tensors and a weight
    change between ticks."""
    case = make_case(3000, 60_000, 4, gpu)
    gen = torch.Generator().manual_seed(3)
    start = torch.rand(32, 3000, generator=gen) * 0.2             # [B,N] contiguous
    native = band_runtime(case.topology, case.model, start.to(gpu), band_width=700, band_rows=96)
    oracle = ort.MatrixOracle(case.graph, case.params, start.clone())
    drive = torch.rand(32, 3000, generator=gen) * 0.4
    ddrive = torch.rand(32, 3000, generator=gen) * 0.2
    for tick in range(12):
        if tick == 6:
            case.topology.apply_source_weights_(case.topology.weight * 0.7)
            oracle.matrix = ort.csr_matrix(otop.with_weights(case.graph,
                                                             case.topology.weight.cpu().numpy()))
        native.step(drive.to(gpu), dendritic_drive=ddrive.to(gpu))
        oracle.step(drive, ddrive)
    assert errors(native, oracle) <= 1e-5


@pytest.mark.parametrize("batch", [4, 8, 16])
def test_band_rollout_graph_equals_eager_ticks(gpu, batch):
    case = make_case(5000, 100_000, 6, gpu)
    drive = column_drive(batch).to(gpu)
    eager = band_runtime(case.topology, case.model, torch.zeros(batch, 5000, device=gpu),
                         band_width=1500, band_rows=200, weight_format="fp8")
    rolled = band_runtime(case.topology, case.model, torch.zeros(batch, 5000, device=gpu),
                          band_width=1500, band_rows=200, weight_format="fp8")
    rollout = MatrixRollout(rolled, 8, drive=drive, dendritic_drive=0.1)
    for replay in range(3):
        rollout.run()
        for _ in range(8):
            eager.step(drive, dendritic_drive=0.1)
        torch.cuda.synchronize()
        assert torch.equal(rollout.state, eager.state), replay
        assert torch.equal(rollout.dendritic_state, eager.dendritic_state), replay
        assert torch.equal(rollout.adaptation_state, eager.adaptation_state), replay


def test_band_empty_graph_and_isolated_rows(gpu):
    """No edges at all (every slot padding), then a graph whose last band is short and
    whose rows mostly have no edges in most bands."""
    model, params = standard_model(1000)
    empty = SparseTopology.from_edges(1000, torch.zeros(0, dtype=torch.long),
                                      torch.zeros(0, dtype=torch.long), torch.zeros(0))
    native = band_runtime(topology_to(empty, gpu), model_to(model, gpu),
                          torch.zeros(16, 1000, device=gpu), band_width=300, band_rows=128)
    graph = otop.build(1000, np.zeros(0, np.int64), np.zeros(0, np.int64), np.zeros(0, np.float32))
    oracle = ort.MatrixOracle(graph, params, torch.zeros(16, 1000))
    for _ in range(5):
        native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
    assert errors(native, oracle) <= 1e-5

    rng = np.random.default_rng(11)
    src = rng.integers(0, 1000, 700)
    dst = rng.integers(0, 1000, 700)
    weight = (rng.standard_normal(700) * 0.05).astype(np.float32)
    graph = otop.build(1000, src, dst, weight)
    topology = SparseTopology.from_edges(1000, torch.from_numpy(src), torch.from_numpy(dst),
                                         torch.from_numpy(weight))
    native = band_runtime(topology_to(topology, gpu), model_to(model, gpu),
                          torch.zeros(16, 1000, device=gpu), band_width=333, band_rows=70,
                          band_steps=4)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(16, 1000))
    for _ in range(5):
        native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
    assert errors(native, oracle) <= 1e-5


@pytest.mark.parametrize("batch,n", [(8, 140_000), (4, 270_000), (16, 70_000)])
def test_auto_takes_bands_past_the_tile_threshold(gpu, batch, n):
    """kernel="auto" picks bands once a workgroup's column tile of the state (16, 8 or
    4 columns) holds 4 MB, with the default band width, rows and register depth."""
    print(f"case auto bands batch={batch} n={n}", flush=True)
    case = make_case(n, 10 * n, 12, gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(batch, n, device=gpu))
    assert native.kernel == "bands"
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(batch, n))
    drive = column_drive(batch)
    worst = 0.0
    for _ in range(5):
        native.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        worst = max(worst, errors(native, oracle))
    print(f"auto bands batch={batch} n={n}: {worst:.3e} over 5 ticks")
    assert worst <= 1e-5
