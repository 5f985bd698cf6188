"""Native fused matrix tick vs the CPU oracle (MI355X).

Tolerances: float32 states within 1e-5 max-abs of the oracle's float32 run
over the whole rollout; low-precision weight formats within 1e-5 of the
oracle run on the decoded float32 weights; fp16 storage and fp8/nvfp4 storage
bitwise equal to the native float32 tick on the decoded weights (the kernels
sum in the same order for every encoding).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from cases import column_drive, make_case, max_err, model_to, progress, standard_model
from oracle import precision as op
from oracle import runtime as ort
from oracle import topology as otop
from neurosim_gpu import (MatrixRollout, NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime,
                          SparseTopology, encode_sparse_weights, load_native_extension,
                          random_topology, topology_to)

pytestmark = pytest.mark.gpu
FIELDS = ("state", "dendritic_state", "adaptation_state")


def errors(native, oracle) -> float:
    return max(max_err(getattr(native, f), getattr(oracle, f)) for f in FIELDS)


def test_cfg1_plumbing_fp32_100_ticks(gpu):
    """random_topology(1000, 20000, seed=0), B=1, drive .2, dendritic .1, 100 ticks."""
    print("case cfg1 N=1000 M=20000 B=1", flush=True)
    case = make_case(1000, 20_000, 0, gpu)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 1000, device=gpu))
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(1, 1000))
    worst = 0.0
    for _ in range(100):
        native.step(0.2, dendritic_drive=0.1)
        oracle.step(0.2, 0.1)
        worst = max(worst, errors(native, oracle))
    print(f"cfg1 max abs error over 100 ticks: {worst:.3e}")
    assert worst <= 1e-5
    assert native.last_backend == "native"


def test_widths_strided_state_params_and_drives(gpu):
    """Reference test_native_compartmental.py:40-57 (N=97, B=3, 600 edges, seed 83)."""
    from dataclasses import replace

    from oracle import dynamics as od

    for width in (8, 16, 32):
        case = make_case(97, 600, 83, gpu, kind="reference")
        state = torch.full((3, 97), 0.2, device=gpu).T.contiguous().T     # transposed strides
        coupling = torch.ones(194, device=gpu)[::2] * 0.6                 # strided parameter
        model = replace(case.model, coupling=coupling)
        params = od.Params(*case.params.as_list())
        params.coupling = coupling.cpu()
        native = NativeDendriticMatrixRuntime(case.topology, model, state.clone(),
                                              threads_per_row=width)
        oracle = ort.MatrixOracle(case.graph, params, state.cpu())
        drives = [0.2, torch.tensor(0.2), torch.tensor([[0.1], [0.3], [0.5]]),
                  torch.linspace(0.1, 0.3, 194)[::2]]
        for value in drives:
            for _ in range(8):
                native.step(value.to(gpu) if isinstance(value, torch.Tensor) else value,
                            dendritic_drive=-0.1)
                oracle.step(value, -0.1)
            assert errors(native, oracle) <= 2e-6
        assert native.last_backend == "native"


@pytest.mark.parametrize("n,batch,edges", [(1, 2, 0), (9, 0, 20), (65, 3, 4000)])
def test_empty_edges_empty_batch_and_large_degree(gpu, n, batch, edges):
    """Reference test_native_compartmental.py:59-69 (row degree up to ~100 at N=65)."""
    case = make_case(n, edges, 83, gpu, kind="reference")
    state = torch.full((batch, n), 0.2)
    for kind, kwargs in ((NativeDendriticMatrixRuntime, {}),
                         (NativeDendriticPELSRuntime, {"theta": 0.0})):
        native = kind(case.topology, case.model, state.to(gpu), **kwargs)
        oracle = ort.MatrixOracle(case.graph, case.params, state.clone())
        for _ in range(8):
            native.step(0.2)
            oracle.step(0.2)
        assert errors(native, oracle) <= 2e-6


def test_long_rows_take_the_whole_workgroup(gpu):
    """Rows longer than one block (4500 and 2500 edges) among short random rows."""
    from cases import model_to, standard_model
    from neurosim_gpu import topology_to

    n = 5000
    rng = np.random.default_rng(4)
    dst = np.concatenate([np.zeros(4500, np.int64), np.full(2500, 5), rng.integers(0, n, 30000)])
    src = np.concatenate([np.arange(4500), np.arange(100, 2600), rng.integers(0, n, 30000)])
    weight = (rng.standard_normal(dst.size) * 0.02).astype(np.float32)
    graph = otop.build(n, src, dst, weight)
    assert np.diff(graph.in_rowptr).max() == 4500
    topology = SparseTopology.from_edges(n, torch.from_numpy(src), torch.from_numpy(dst),
                                         torch.from_numpy(weight))
    assert np.array_equal(topology.in_col.numpy(), graph.in_col)
    model, params = standard_model(n)
    for batch in (1, 3, 16):
        native = NativeDendriticMatrixRuntime(topology_to(topology, gpu), model_to(model, gpu),
                                              torch.zeros(batch, n, device=gpu))
        oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, n))
        drive = column_drive(batch)
        for _ in range(20):
            native.step(drive.to(gpu), dendritic_drive=0.1)
            oracle.step(drive, 0.1)
        assert errors(native, oracle) <= 1e-5


def test_fp16_storage_is_bitwise_the_rounded_fp32_tick(gpu):
    """Reference test_native_compartmental.py:71-90, including a weight change mid-run."""
    case = make_case(97, 600, 83, gpu, kind="reference")
    graph = case.topology
    rounded = SparseTopology.from_edges(97, graph.src, graph.dst, graph.weight.half().float())
    state = torch.full((3, 97), 0.2, device=gpu)
    native = NativeDendriticMatrixRuntime(graph, case.model, state.clone(), weight_dtype=torch.float16)
    reference = NativeDendriticMatrixRuntime(rounded, case.model, state.clone())
    with torch.inference_mode():
        for tick in range(12):
            if tick == 6:
                graph.apply_source_weights_(graph.weight * 0.7)
                rounded.apply_source_weights_(graph.weight.half().float())
            native.step(0.2, dendritic_drive=0.1)
            reference.step(0.2, dendritic_drive=0.1)
            for field in FIELDS:
                assert torch.equal(getattr(native, field), getattr(reference, field))
    assert native.last_backend == "native-fp16-weight"
    assert native.weight_storage_bytes == 2 * graph.n_edges
    drive = torch.tensor(0.3, device=gpu, requires_grad=True)
    with pytest.raises(RuntimeError, match="inference-only"):
        native.step(drive)


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
@pytest.mark.parametrize("edges", [0, 605])
def test_packed_formats_equal_decoded_fp32(gpu, fmt, edges):
    """Reference test_native_compartmental.py:112-140; bitwise here, plus the oracle."""
    case = make_case(97, edges, 83, gpu, kind="reference")
    graph = case.topology
    if edges and graph.n_edges % 2 == 0:      # odd edge counts exercise the last nibble
        graph = SparseTopology.from_edges(97, graph.src[:-1], graph.dst[:-1], graph.weight[:-1])
    decoded = SparseTopology.from_edges(97, graph.src, graph.dst, graph.weight)
    state = torch.full((3, 97), 0.2, device=gpu)
    native = NativeDendriticMatrixRuntime(graph, case.model, state.clone(), weight_format=fmt)
    reference = NativeDendriticMatrixRuntime(decoded, case.model, state.clone())
    with torch.inference_mode():
        for tick in range(6):
            if tick == 3:
                graph.apply_source_weights_(graph.weight * 0.7)
            if tick in (0, 3):
                # decode exactly the payload the kernel reads (oracle decoder, edge by edge)
                native._weights()
                codes, *scales = native._packed_weight
                block = scales[0].cpu().numpy() if fmt == "nvfp4" else None
                host = op.decode_packed(codes.cpu().numpy(), block, np.float32(scales[-1].item()),
                                        graph.n_edges, fmt)
                csr = torch.from_numpy(host).to(gpu)
                decoded.apply_source_weights_(csr[graph.out_weight_index.long()])
                oracle_graph = otop.build(97, graph.src.cpu().numpy(), graph.dst.cpu().numpy(),
                                          decoded.weight.cpu().numpy())
                if tick == 0:
                    oracle = ort.MatrixOracle(oracle_graph, case.params, state.cpu())
                else:
                    oracle.matrix = ort.csr_matrix(oracle_graph)
            native.step(0.2, dendritic_drive=0.1)
            reference.step(0.2, dendritic_drive=0.1)
            oracle.step(0.2, 0.1)
            for field in FIELDS:
                assert torch.equal(getattr(native, field), getattr(reference, field))
            assert errors(native, oracle) <= 1e-5
    assert native.last_backend == f"native-{fmt}-weight"
    assert native.weight_storage_bytes == sum(
        v.numel() * v.element_size() for v in native._packed_weight if v is not None)


def test_decoders_exhaustive(gpu):
    """Every fp8 code and every (nibble, block-scale code) pair through the kernel.

    Row r holds one edge whose weight is the decode under test; s = 1 so
    J = W @ s returns the decoded weight, compared bitwise to the oracle tables.
    """
    ext = load_native_extension()
    # fp8: 256 rows, row r = code r, global scale 1.
    n = 256
    rowptr = torch.arange(n + 1, dtype=torch.int32, device=gpu)
    col = torch.zeros(n, dtype=torch.int32, device=gpu)
    codes = torch.arange(n, dtype=torch.uint8, device=gpu)
    one = torch.ones(1, n, device=gpu)
    scale = torch.ones(1, device=gpu)
    got = ext.csr_spmm(one, rowptr, col, codes, None, scale).cpu().numpy()[0]
    want = op.e4m3_decode(np.arange(n, dtype=np.uint8))
    assert np.array_equal(got, want, equal_nan=True)
    # nvfp4: 16 nibbles x 256 scale codes; edge e = 16*s + nibble -> block s.
    n = 4096
    edges = np.arange(n)
    nibble = (edges & 15).astype(np.uint8)
    packed = (nibble[0::2] | (nibble[1::2] << 4)).astype(np.uint8)
    block_codes = np.arange(256, dtype=np.uint8)
    scale_value = np.float32(0.37)
    got = ext.csr_spmm(torch.ones(1, n, device=gpu), torch.arange(n + 1, dtype=torch.int32, device=gpu),
                       torch.zeros(n, dtype=torch.int32, device=gpu),
                       torch.from_numpy(packed).to(gpu), torch.from_numpy(block_codes).to(gpu),
                       torch.tensor([scale_value], device=gpu)).cpu().numpy()[0]
    want = op.decode_packed(packed, block_codes, scale_value, n, "nvfp4")
    assert np.array_equal(got, want, equal_nan=True)


def test_matrix_tick_is_bitwise_repeatable(gpu):
    case = make_case(5000, 100_000, 3, gpu)
    runs = []
    for _ in range(2):
        native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(4, 5000, device=gpu))
        for _ in range(20):
            native.step(0.2, dendritic_drive=0.1)
        runs.append(native.state.clone())
    assert torch.equal(runs[0], runs[1])


def test_cfg2_batched_fp32_1000_ticks(gpu):
    """random_topology(50000, 1000000, seed=0), B=8, per-column drive U(0,.4) seed 1."""
    print("case cfg2 N=50000 M=1000000 B=8 ticks=1000", flush=True)
    case = make_case(50_000, 1_000_000, 0, gpu)
    drive = column_drive(8)
    native = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(8, 50_000, device=gpu))
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(8, 50_000))
    drive_gpu = drive.to(gpu)
    # The timed path as well: 100-tick graph replays, checked at every chunk end.
    rolled = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(8, 50_000, device=gpu))
    rollout = MatrixRollout(rolled, 100, drive=drive_gpu, dendritic_drive=0.1)
    worst = worst_rollout = 0.0
    for tick in range(1000):
        native.step(drive_gpu, dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        if tick % 10 == 9:
            worst = max(worst, errors(native, oracle))
        if tick % 100 == 99:
            rollout.run()
            worst_rollout = max(worst_rollout, errors(rollout, oracle))
    worst = max(worst, errors(native, oracle))
    print(f"cfg2 max abs error over 1000 ticks: eager {worst:.3e}, graph chunks {worst_rollout:.3e}")
    assert worst <= 1e-5 and worst_rollout <= 1e-5


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
def test_device_encoder_is_bitwise_the_oracle_at_25m_edges(gpu, large_case, fmt):
    """Codes, block scales and global scale encoded on the GPU == the CPU oracle's.

    A Python-number divisor lets PyTorch's GPU division multiply by a rounded
    reciprocal; at this size that moved the NVFP4 global scale by one ulp and
    flipped codes.  The encoder must reproduce the CPU's true quotients.
    """
    print(f"case encode N=166000 M=25M fmt={fmt}", flush=True)
    weight = large_case.graph.in_weight
    codes, scales, scale = encode_sparse_weights(torch.from_numpy(weight).to(gpu), fmt)
    want_codes, want_scales, want_scale = op.encode_sparse_weights(weight, fmt)
    assert np.float32(scale.item()).tobytes() == np.float32(want_scale).tobytes()
    assert np.array_equal(codes.cpu().numpy(), want_codes)
    if fmt == "nvfp4":
        assert np.array_equal(scales.cpu().numpy(), want_scales)


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
def test_hip_encoder_is_bitwise_the_oracle_at_25m_edges(gpu, large_case, fmt):
    """ns_encode_weights on the headline graph's 25M weights == the CPU oracle's payload."""
    from neurosim_gpu.native import encode_weights

    print(f"case hip encode N=166000 M=25M fmt={fmt}", flush=True)
    weight = large_case.graph.in_weight
    codes, scales, scale = encode_weights(torch.from_numpy(weight).to(gpu), fmt)
    want_codes, want_scales, want_scale = op.encode_sparse_weights(weight, fmt)
    assert np.float32(scale.item()).tobytes() == np.float32(want_scale).tobytes()
    assert np.array_equal(codes.cpu().numpy(), want_codes)
    if fmt == "nvfp4":
        assert np.array_equal(scales.cpu().numpy(), want_scales)


@pytest.mark.parametrize("fmt", ["fp32", "fp16", "fp8", "nvfp4"])
def test_cfg3_large_1000_ticks(gpu, large_case, fmt):
    """N=166000, M~25M, B=1: fp32 vs oracle; fp16/fp8/nvfp4 vs oracle on decoded weights."""
    print(f"case cfg3 N=166000 M=25M B=1 fmt={fmt} ticks=1000", flush=True)
    case = large_case
    kwargs = {"fp32": {}, "fp16": {"weight_dtype": torch.float16},
              "fp8": {"weight_format": "fp8"}, "nvfp4": {"weight_format": "nvfp4"}}[fmt]
    native = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(1, 166_000, device=gpu), **kwargs)
    in_weight = op.quantize_dequantize(case.graph.in_weight, fmt)
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(1, 166_000), in_weight=in_weight)
    # The path bench.py times: 100-tick graph replays, checked at every chunk end.
    rolled = NativeDendriticMatrixRuntime(case.topology, case.model,
                                          torch.zeros(1, 166_000, device=gpu), **kwargs)
    rollout = MatrixRollout(rolled, 100, drive=0.2, dendritic_drive=0.1)
    worst = worst_rollout = 0.0
    with torch.inference_mode():
        for tick in range(1000):
            native.step(0.2, dendritic_drive=0.1)
            oracle.step(0.2, 0.1)
            if tick % 50 == 49:
                worst = max(worst, errors(native, oracle))
            if tick % 100 == 99:
                rollout.run()
                worst_rollout = max(worst_rollout, errors(rollout, oracle))
    print(f"cfg3 {fmt} max abs error over 1000 ticks: eager {worst:.3e}, "
          f"graph chunks {worst_rollout:.3e}")
    assert worst <= 1e-5 and worst_rollout <= 1e-5


@pytest.fixture(scope="module")
def cfg5(gpu):
    """N=1000000, M~100M candidates (seed 0): the oracle's own graph from the
    draws (oracle.topology, numpy coalescing), the product's CPU build and its
    GPU build (ns_build_topology).  Several minutes of host work in all, so each
    phase reports on the real stderr."""
    n = 1_000_000
    progress("cfg5: oracle graph from 100M candidate draws (numpy coalescing)")
    graph = otop.random_graph(n, 100_000_000, seed=0)
    progress("cfg5: the product's CPU build")
    topology_cpu = random_topology(n, 100_000_000, device="cpu", seed=0)
    progress("cfg5: the product's GPU build")
    topology = random_topology(n, 100_000_000, device="cpu", seed=0, build_device=gpu)
    progress(f"cfg5: {graph.n_edges} edges built three ways")
    return graph, topology_cpu, topology


def test_cfg5_three_constructions_of_the_scaleout_graph_are_bitwise_equal(cfg5):
    graph, topology_cpu, topology = cfg5
    for name in ("src", "dst", "weight", "out_rowptr", "in_rowptr", "in_col", "in_weight",
                 "out_weight_index"):
        assert np.array_equal(getattr(topology_cpu, name).numpy(), getattr(graph, name)), name
        assert torch.equal(getattr(topology, name).cpu(), getattr(topology_cpu, name)), name


def test_cfg5_scaleout_fp8_against_an_independent_graph(gpu, cfg5):
    """N=1000000, M~100M, B=16, drive [16,1] U(0,.4) seed 1, fp8 weights, on the
    GPU build of the graph; the oracle runs on its own construction (bitwise
    the same arrays, previous test).  10 eager ticks against the oracle's float32
    run on the decoded weights, every tick, and the timed path: a graph of 100
    captured ticks replayed from the same zero state, against the oracle at tick
    100."""
    print("case cfg5 N=1000000 M=100M B=16 fp8 ticks=10 eager + 100 graph", flush=True)
    graph, _, topology = cfg5
    n, batch = 1_000_000, 16
    model, params = standard_model(n)
    native = NativeDendriticMatrixRuntime(topology, model_to(model, gpu),
                                          torch.zeros(batch, n, device=gpu), weight_format="fp8")
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, n),
                              in_weight=op.quantize_dequantize(graph.in_weight, "fp8"))
    drive = column_drive(batch)
    # The timed path: 100 captured ticks from the same zero state.
    rollout = MatrixRollout(native, 100, drive=drive.to(gpu), dendritic_drive=0.1)
    worst = 0.0
    with torch.inference_mode():
        for _ in range(10):
            native.step(drive.to(gpu), dendritic_drive=0.1)
            oracle.step(drive, 0.1)
            worst = max(worst, errors(native, oracle))
        rollout.run()
        for k in range(90):
            oracle.step(drive, 0.1)
            if k % 30 == 29:
                progress(f"cfg5: oracle tick {k + 11} of 100")
        worst_rollout = errors(rollout, oracle)
    print(f"cfg5 fp8 max abs error: eager ticks 1-10 {worst:.3e}, "
          f"graph of 100 ticks {worst_rollout:.3e}", flush=True)
    assert worst <= 1e-5 and worst_rollout <= 1e-5


@pytest.mark.parametrize("fmt", ["fp32", "nvfp4"])
@pytest.mark.parametrize("batch", [4, 5, 6, 7, 8, 9, 12, 17, 20, 33])
def test_row_blocks_at_every_column_tile(gpu, batch, fmt):
    """The row-block kernel's column tiles (4, 8 or 16 columns, the last one of a
    batch partial) against the oracle, at B=8 with the paired 32-byte row gathers.
    A twin runtime whose states are copied row-major before every tick gathers
    element by element instead (no 16-byte row loads, no pairs); the products and
    their order are the same, so its states must be bitwise those of the first."""
    print(f"case row blocks B={batch} fmt={fmt}", flush=True)
    n, m = 600, 9000
    case = make_case(n, m, 5, gpu)
    options = {} if fmt == "fp32" else {"weight_format": fmt}
    neuron_major, row_major = (
        NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(batch, n, device=gpu),
                                     kernel="rows", **options) for _ in range(2))
    weight = (case.graph.in_weight if fmt == "fp32"
              else op.quantize_dequantize(case.graph.in_weight, fmt))
    oracle = ort.MatrixOracle(case.graph, case.params, torch.zeros(batch, n), in_weight=weight)
    drive = column_drive(batch)
    for t in range(20):
        neuron_major.step(drive.to(gpu), dendritic_drive=0.1)
        for f in FIELDS:
            setattr(row_major, f, getattr(row_major, f).contiguous())
        row_major.step(drive.to(gpu), dendritic_drive=0.1)
        oracle.step(drive, 0.1)
        for f in FIELDS:
            assert torch.equal(getattr(neuron_major, f), getattr(row_major, f)), (batch, fmt, t, f)
    assert neuron_major.state.stride(0) == 1 or batch == 1
    assert errors(neuron_major, oracle) <= 1e-5
