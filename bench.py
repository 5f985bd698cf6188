"""Benchmark of the native dendritic matrix tick on one MI355X.

Workload (the headline configuration): random_topology(N=166000, M=25000000
candidates, seed=0) -> 24,988,875 coalesced edges, B=1, alpha .72, gain .8,
tau_d 4, tau_a 25, coupling .5, strength .2, zero initial state, drive .2,
dendritic drive .1.  One step = one fused tick (CSR gather-product + three-state
update) over the whole graph, run as graph-captured ticks on the current
stream with every input resident in HBM.  The same graph is also timed with
fp16, fp8 e4m3 and nvfp4 weight storage.

Prints one JSON line.  ``value`` is ms per fp32 tick (lower is better);
``roofline`` prices the fp32 tick's algorithmic bytes against MI355X's 8 TB/s;
``cpu_baseline`` times the CPU oracle (the reference's float32 torch CPU path,
restated) on a bounded sample of the same tick on this host.  ``configs``
adds the other workloads, each timed the same way: the batched tick
(N=50000, M~1M, B=8, per-column drive), the PELS event tick (N=50000, M~1M,
B=1, theta 0.02, driven and with inputs withdrawn), the scale-out tick
(N=1000000, M~100M, B=16, fp8 weights, 200 graph-captured ticks, with the
CPU oracle on a 10-tick sample), the fp8/NVFP4 device encoding of the
headline graph's weights, one recorded tick plus its native backward on
the headline graph next to autograd through the torch step, and headline
ticks with a new weight version before each, and the reference's own benchmark
protocol (five shapes, eager ticks, its published RTX 5070 figures beside each
row, kernels per tick counted in a captured graph), and the reference's
reduced-weight-storage protocol (two B=8 shapes, fp32/fp16/fp8/NVFP4, eager ticks and
each mode's trajectory error against fp32, its published figures beside).  ``host`` names the CPU model,
torch and HIP versions; ``cpu_baseline`` also gives the one-thread figure.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50]
"""

from __future__ import annotations

import argparse
import dataclasses
import gc
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "neurosim-gpu_amd"))

from neurosim_gpu import (DendriticDynamics, Dynamics, MatrixRollout,  # noqa: E402
                          NativeDendriticMatrixRuntime, NativeDendriticPELSRuntime,
                          random_topology, topology_to)

N_NEURONS, CANDIDATES, SEED, BATCH = 166_000, 25_000_000, 0, 1
HBM_PEAK_GBPS = 8000.0
METRIC = "ms/tick + achieved HBM GB/s (% peak), N=166k M=25M B=1 fp32/fp8/nvfp4"
WORKLOAD = "dendritic matrix tick, N=166000 M=24988875 B=1, fp32 weights"
CHUNK = 100   # ticks per captured graph


def log(message: str) -> None:
    print(f"[bench] {message}", file=sys.stderr, flush=True)


def weight_bytes(fmt: str, m: int) -> int:
    return {"fp32": 4 * m, "fp16": 2 * m, "fp8": m + 4,
            "nvfp4": (m + 1) // 2 + (m + 15) // 16 + 4}[fmt]


def parameter_bytes(model, n: int) -> int:
    """Bytes of the six parameter vectors: 4N each, 4 for a stride-0 (scalar) one."""
    vectors = (model.soma.alpha, model.soma.gain, model.dendrite_decay, model.adaptation_decay,
               model.coupling, model.adaptation_strength)
    return sum(4 if v.stride(0) == 0 else 4 * n for v in vectors)


def algorithmic_bytes(fmt: str, n: int, m: int, batch: int, params: int | None = None) -> int:
    """rowptr + col + weights + s,d,a reads + s,d,a writes + the parameter vectors
    (``params`` bytes; six full vectors when not given)."""
    params = 24 * n if params is None else params
    return 4 * (n + 1) + 4 * m + weight_bytes(fmt, m) + 24 * batch * n + params


def build_runtime(fmt: str, topology, model, device, kernel: str = "auto"):
    kwargs = {"fp32": {}, "fp16": {"weight_dtype": torch.float16},
              "fp8": {"weight_format": "fp8"}, "nvfp4": {"weight_format": "nvfp4"}}[fmt]
    return NativeDendriticMatrixRuntime(topology, model, torch.zeros(BATCH, N_NEURONS, device=device),
                                        kernel=kernel, **kwargs)


def copy_calibration(mib: int = 256, repeats: int = 10) -> None:
    """Plain device-to-device copies of a known size, for scaling PMC byte counters:
    each launch reads and writes exactly ``mib`` MiB."""
    source = torch.ones(mib * 1024 * 1024 // 4, dtype=torch.float32, device="cuda")
    target = torch.empty_like(source)
    for _ in range(repeats):
        target.copy_(source)
    torch.cuda.synchronize()
    log(f"copy calibration: {repeats} copies of {mib} MiB")


def launches_per_tick(runtime) -> int:
    """Kernel launches of one eager tick, counted as the kernel nodes of a graph
    capturing it (the runtime's states are put back afterwards).  Where the HIP
    runtime cannot be queried, the count the layout implies: two on column
    panels finished by the combine kernel, one otherwise."""
    graph, saved = captured_steps(runtime, [(0.2, 0.1)], STATE_FIELDS, keep_graph=True)
    for f, value in zip(STATE_FIELDS, saved):
        setattr(runtime, f, value)
    counted = graph_nodes(graph)
    del graph
    if counted is not None:
        return counted["kernels"]
    panels = getattr(runtime, "_panels", None)
    return 2 if panels is not None and panels.n_panels > 1 and panels.combine_launch else 1


def time_ticks(runtime, steps: int, warmup: int) -> tuple[float, MatrixRollout]:
    """ms per tick over exactly ``steps`` ticks: captured graphs of CHUNK ticks
    (plus one graph for an even tail and one eager tick for an odd count),
    bracketed by device synchronisations and timed with HIP events."""
    chunk = CHUNK if steps >= CHUNK else max(2, steps - steps % 2)
    rollout = MatrixRollout(runtime, chunk, drive=0.2, dendritic_drive=0.1)
    full = steps // chunk
    tail = steps - full * chunk
    tail_rollout = (MatrixRollout(runtime, tail - tail % 2, drive=0.2, dendritic_drive=0.1)
                    if tail >= 2 else None)
    odd = tail % 2
    # Every graph is replayed once before the timed region (the first replay uploads it).
    rollout.run(max(1, warmup // chunk))
    if tail_rollout is not None:
        tail_rollout.run()
    for _ in range(warmup % chunk):
        runtime.step(0.2, dendritic_drive=0.1)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    rollout.run(full)
    if tail_rollout is not None:
        tail_rollout.run()
    if odd:
        runtime.step(0.2, dendritic_drive=0.1)
    end.record()
    torch.cuda.synchronize()
    if not bool(torch.isfinite(rollout.state).all()):
        raise RuntimeError("non-finite state after the timed ticks")
    return start.elapsed_time(end) / steps, rollout


def mall_flushed_ms(rollout: MatrixRollout, ticks: int = 20, repeats: int = 7) -> dict:
    """ms per tick when reading 1 GiB first evicts the graph from the 256 MB last-level
    cache.  The eviction reads (a column sum into a 4 MB result), so it leaves clean
    lines: no write-back of it competes with the tick for HBM.

    ``ms_per_tick``: two captured graphs, ``ticks`` evictions each, one with a tick
    after every eviction; the difference of their replay times over ``ticks`` is the
    flushed tick as graph replays run it (median of ``repeats`` pairs).
    ``eager_ms_per_tick``: one eager tick after each eviction, timed with HIP events
    around its two launches (host launch costs included)."""
    scratch = torch.ones(256, 1024 * 1024, dtype=torch.float32, device="cuda")
    column_sums = torch.empty(1024 * 1024, dtype=torch.float32, device="cuda")
    launch, planes = rollout._launch, rollout._sets

    def evict():
        torch.sum(scratch, dim=0, out=column_sums)

    eager = []
    for i in range(ticks):
        evict()                                   # ~0.2 ms of reads keeps the queue ahead of the host
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        launch(planes[0], planes[1])
        end.record()
        end.synchronize()
        eager.append(start.elapsed_time(end))

    def capture(with_ticks: bool):
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            evict()
            if with_ticks:
                launch(planes[0], planes[1])
                launch(planes[1], planes[0])
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for k in range(ticks):
                evict()
                if with_ticks:
                    launch(planes[k % 2], planes[(k + 1) % 2])
        return graph

    def replay_ms(graph) -> float:
        graph.replay()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        return start.elapsed_time(end)

    flush_and_tick, flush_only = capture(True), capture(False)
    differences = sorted((replay_ms(flush_and_tick) - replay_ms(flush_only)) / ticks
                         for _ in range(repeats))
    del flush_and_tick, flush_only, scratch
    return {"ms_per_tick": differences[len(differences) // 2],
            "eager_ms_per_tick": sum(eager) / ticks}


def standard_model(n: int, device):
    """alpha .72, gain .8, dt 1, tau_d 4, tau_a 25, coupling .5, strength .2, as
    (host model, device model).  Each is built where it lives, as the reference's
    benchmark builds its model on the GPU (benchmarks/compartmental.py:62-65):
    alpha, gain and the two retention factors are [N] vectors, coupling and
    strength stride-0 views of one scalar."""
    def build(where):
        soma = Dynamics(torch.full((n,), .72, device=where), torch.full((n,), .8, device=where))
        return DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4.,
                                                     tau_adaptation=25., coupling=.5,
                                                     adaptation_strength=.2)
    return build("cpu"), build(device)


def column_drive(batch: int, seed: int = 1) -> torch.Tensor:
    """Per-column somatic drive U(0, 0.4) of shape [B, 1] from a host generator."""
    return torch.rand((batch, 1), generator=torch.Generator().manual_seed(seed)) * 0.4


def oracle_tick_ms(topology_cpu, model_cpu, batch: int, drive, ticks: int, warmup: int = 3,
                   weight=None, threads: int | None = None) -> tuple[float, int]:
    """ms per float32 tick of the CPU oracle (all host threads unless ``threads``)."""
    sys.path.insert(0, str(ROOT))
    from oracle import dynamics as od
    from oracle import runtime as ort
    from oracle import topology as otop

    graph = otop.Graph(
        n=topology_cpu.n_neurons, src=topology_cpu.src.numpy(), dst=topology_cpu.dst.numpy(),
        weight=topology_cpu.weight.numpy(), out_rowptr=topology_cpu.out_rowptr.numpy(),
        in_rowptr=topology_cpu.in_rowptr.numpy(), in_col=topology_cpu.in_col.numpy(),
        in_weight=topology_cpu.in_weight.numpy(),
        out_weight_index=topology_cpu.out_weight_index.numpy())
    params = od.Params(model_cpu.soma.alpha, model_cpu.soma.gain, model_cpu.dendrite_decay,
                       model_cpu.adaptation_decay, model_cpu.coupling, model_cpu.adaptation_strength)
    if threads is None:
        cores = os.cpu_count() or 1
        threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    previous = torch.get_num_threads()
    torch.set_num_threads(threads)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(batch, topology_cpu.n_neurons),
                              in_weight=weight)
    for _ in range(warmup):
        oracle.step(drive, 0.1)
    begin = time.perf_counter()
    for _ in range(ticks):
        oracle.step(drive, 0.1)
    elapsed = time.perf_counter() - begin
    torch.set_num_threads(previous)
    return elapsed * 1000 / ticks, threads


def host_info() -> dict:
    """CPU model (as lscpu names it, from /proc/cpuinfo), thread counts and the
    software the numbers were taken with."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "host_threads": os.cpu_count(),
            "torch": torch.__version__, "hip": torch.version.hip,
            "gpu": torch.cuda.get_device_name(0)}


def cpu_baseline(topology_cpu, model_cpu, ticks: int = 20, single_ticks: int = 5) -> dict:
    """The CPU oracle's float32 tick on this host (bounded samples): on every
    thread the process may use, and on one thread."""
    ms, threads = oracle_tick_ms(topology_cpu, model_cpu, BATCH, 0.2, ticks)
    single_ms, _ = oracle_tick_ms(topology_cpu, model_cpu, BATCH, 0.2, single_ticks, warmup=1,
                                  threads=1)
    return {"value": round(ms, 3), "unit": "ms/tick", "cores": threads, "kind": "port",
            "sample": f"{ticks} fp32 ticks (after 3 warm-up) of the same N=166000 M=24988875 B=1 "
                      f"graph, torch CPU CSR product + elementwise update, {threads} threads",
            "single_thread": {"value": round(single_ms, 3), "unit": "ms/tick", "cores": 1,
                              "sample": f"{single_ticks} fp32 ticks (after 1 warm-up), same "
                                        "graph and code, one thread"}}


def measured_traffic(fmt: str) -> float | None:
    """HBM bytes per launch from the committed rocprofv3 PMC summary, if present."""
    path = ROOT / "profiles" / "tick_pmc_n166k_m25m_b1.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        fields = line.split()
        if len(fields) >= 2 and fields[0] == f"traffic_bytes_{fmt}":
            return float(fields[1])
    return None


def rollout_ms(runtime, ticks: int, repeats: int, drive, dendritic_drive) -> float:
    """ms per tick of `repeats` replays of one graph of `ticks` matrix ticks."""
    rollout = MatrixRollout(runtime, ticks, drive=drive, dendritic_drive=dendritic_drive)
    rollout.run(1)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    rollout.run(repeats)
    end.record()
    torch.cuda.synchronize()
    if not bool(torch.isfinite(rollout.state).all()):
        raise RuntimeError("non-finite state after the timed ticks")
    return start.elapsed_time(end) / (ticks * repeats)


def measure_encode(weight: torch.Tensor, repeats: int = 20) -> dict:
    """fp8 and NVFP4 encoding of the headline graph's float32 CSR weights on
    the device: ns_encode_weights (two launches) against the torch-op
    encoder it replaces, each timed over ``repeats`` calls with HIP events,
    plus a bitwise comparison of the two payloads."""
    from neurosim_gpu.native import encode_weights
    from neurosim_gpu.precision import encode_sparse_weights

    m = weight.numel()
    out = {"workload": f"weight encoding, M={m} float32 CSR weights", "repeats": repeats}
    for fmt in ("fp8", "nvfp4"):
        # weight read twice (amax, then encode), payload written once
        alg = 8 * m + (m if fmt == "fp8" else (m + 1) // 2 + (m + 15) // 16) + 4
        timed = {}
        for name, fn in (("hip", encode_weights), ("torch_ops", encode_sparse_weights)):
            for _ in range(3):
                result = fn(weight, fmt)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(repeats):
                result = fn(weight, fmt)
            end.record()
            torch.cuda.synchronize()
            timed[name] = (start.elapsed_time(end) / repeats, result)
        hip_ms, (codes, scales, scale) = timed["hip"]
        ops_ms, (codes_ref, scales_ref, scale_ref) = timed["torch_ops"]
        same = bool(torch.equal(codes, codes_ref)) and bool(torch.equal(scale.reshape(()), scale_ref.reshape(())))
        if fmt == "nvfp4":
            same = same and bool(torch.equal(scales, scales_ref))
        out[fmt] = {"hip_ms": round(hip_ms, 4), "torch_ops_ms": round(ops_ms, 4),
                    "algorithmic_bytes": alg, "hip_GBps": round(alg / hip_ms / 1e6, 1),
                    "pct_hbm_peak": round(100 * alg / hip_ms / 1e6 / HBM_PEAK_GBPS, 1),
                    "payload_equal_to_torch_ops": same}
    return out


def measure_backward(topology, model, repeats: int = 10) -> dict:
    """One recorded fp32 tick plus its backward on the headline graph (B=1,
    every parameter, the weights and the state requiring gradients, loss =
    sum of the new state): the native backward against autograd through the
    torch step that the reference runs for such ticks, each timed with HIP
    events over ``repeats`` forward+backward passes (the median pass, and the
    slowest).  The weights do not
    change between passes, so from the second pass on the native forward runs
    on panels over a slot-order copy of them and the transposed product streams
    a source-major copy (each built once per weight version).
    ``native_changing_weights_ms`` marks the weights modified before every pass
    (a new version, as after an optimizer step, values unchanged), so neither
    copy is reused; ``native_bptt8_ms_per_tick`` times eight recorded ticks and
    one backward through them, per tick."""
    from neurosim_gpu import DendriticMatrixRuntime

    n = topology.n_neurons
    weight = topology.in_weight.detach().clone().requires_grad_(True)
    trained = dataclasses.replace(topology, in_weight=weight)
    params = [p.detach().clone().requires_grad_(True) for p in (
        model.soma.alpha, model.soma.gain, model.dendrite_decay, model.adaptation_decay,
        model.coupling, model.adaptation_strength)]
    dyn = DendriticDynamics(Dynamics(params[0], params[1]), *params[2:])
    out = {"workload": f"one fp32 tick + backward, N={n} M={topology.n_edges} B=1, gradients of "
                       "the weights, the six parameters and the state", "repeats": repeats}
    runs = (("native", NativeDendriticMatrixRuntime, 1, False),
            ("native_changing_weights", NativeDendriticMatrixRuntime, 1, True),
            ("native_bptt8", NativeDendriticMatrixRuntime, 8, False),
            ("torch_autograd", DendriticMatrixRuntime, 1, False))
    for name, cls, ticks, new_version in runs:
        state = torch.full((1, n), 0.2, device=weight.device)
        runtime = cls(trained, dyn, state)

        def once():
            if new_version:
                torch.autograd.graph.increment_version(weight)
            runtime.state = state.clone().requires_grad_(True)
            runtime.dendritic_state = torch.zeros_like(state)
            runtime.adaptation_state = torch.zeros_like(state)
            for _ in range(ticks):
                runtime.step(0.2, dendritic_drive=0.1)
            runtime.state.sum().backward()

        try:
            # The first two passes of a weight version build its slot-order and
            # transposed copies.
            for _ in range(2):
                once()
        except RuntimeError as error:
            # torch's sparse CSR backward on this ROCm build asks for an absurd
            # allocation at this size (HIP out of memory): the leg is skipped.
            out[f"{name}_ms"] = None
            out[f"{name}_skipped"] = ("torch autograd through the reference step failed: "
                                      + str(error).splitlines()[0][:160])
            del runtime
            torch.cuda.empty_cache()
            continue
        torch.cuda.synchronize()
        # A full collection of Python's cyclic garbage collector walks every
        # tracked object (about 170k here, 40 ms) and stalls the host while it
        # enqueues a pass, which the GPU then spends idle.  The objects alive now
        # are moved out of its reach, as a training loop would do, so the passes
        # time the GPU work.
        gc.collect()
        gc.freeze()
        # The collection leaves the GPU idle for tens of milliseconds, and the
        # first pass after such a pause runs 1.5-2x slower: one more untimed pass.
        once()
        passes = []
        for _ in range(repeats):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            once()
            end.record()
            end.synchronize()
            passes.append(start.elapsed_time(end))
        gc.unfreeze()
        ms = sorted(passes)[len(passes) // 2]        # median pass
        if ticks == 1:
            out[f"{name}_ms"] = round(ms, 4)
        else:
            out[f"{name}_ms_per_tick"] = round(ms / ticks, 4)
        out[f"{name}_slowest_pass_ms"] = round(max(passes), 4)
        out[f"{name}_passes_ms"] = [round(p, 3) for p in passes]
        weight.grad = None
        for p in params:
            p.grad = None
        del runtime
    return out


def measure_weight_change(topology, model, device, ticks: int = 20) -> dict:
    """The headline graph with a new weight version before every tick
    (``mark_weights_mutated_``, as after an optimizer step or a plasticity
    update), so each tick first rebuilds what the runtime derives from the
    weights (the encoded payload, the slot-order copy) and then runs.  ms per
    tick over ``ticks`` eager ticks, with the weights unchanged next to it."""
    out = {"workload": f"dendritic matrix tick, N={topology.n_neurons} M={topology.n_edges} B=1, "
                       "a new weight version before every tick", "ticks": ticks}

    def timed(runtime, mutate: bool) -> float:
        for _ in range(3):
            if mutate:
                topology.mark_weights_mutated_()
            runtime.step(0.2, dendritic_drive=0.1)
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(ticks):
            if mutate:
                topology.mark_weights_mutated_()
            runtime.step(0.2, dendritic_drive=0.1)
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / ticks

    with torch.inference_mode():
        for fmt in ("fp32", "fp8", "nvfp4"):
            for kernel in ("auto", "rows"):
                runtime = build_runtime(fmt, topology, model, device, kernel)
                out[f"{fmt}_{kernel}"] = {"kernel": runtime.kernel,
                                          "new_weights_ms_per_tick": round(timed(runtime, True), 4),
                                          "same_weights_eager_ms_per_tick":
                                              round(timed(runtime, False), 4)}
                del runtime
                torch.cuda.empty_cache()
    return out


def measure_batched(device) -> dict:
    """N=50000, M~1M, B=8, drive [8,1] U(0,.4) (seed 1), dendritic .1, fp32, 1000 ticks."""
    n, candidates, batch = 50_000, 1_000_000, 8
    topology_cpu = random_topology(n, candidates, device="cpu", seed=0)
    m = topology_cpu.n_edges
    _, model = standard_model(n, device)
    runtime = NativeDendriticMatrixRuntime(topology_to(topology_cpu, device), model,
                                           torch.zeros(batch, n, device=device))
    ms = rollout_ms(runtime, 100, 10, column_drive(batch).to(device), 0.1)
    alg = algorithmic_bytes("fp32", n, m, batch, parameter_bytes(model, n)) + 4 * batch
    return {"workload": f"dendritic matrix tick, N={n} M={m} B={batch}, fp32 weights, "
                        "per-column drive", "kernel": runtime.kernel,
            "ms_per_tick": round(ms, 5), "algorithmic_bytes": alg,
            "achieved_GBps": round(alg / ms / 1e6, 1),
            "pct_hbm_peak": round(100 * alg / ms / 1e6 / HBM_PEAK_GBPS, 1)}


def _hip_runtime():
    """The HIP runtime library this process already uses (None if it cannot be found)."""
    import ctypes
    try:
        maps = Path("/proc/self/maps").read_text().splitlines()
    except OSError:
        return None
    for line in maps:
        path = line.split()[-1]
        if "libamdhip64.so" in path:
            try:
                hip = ctypes.CDLL(path, mode=os.RTLD_NOLOAD | os.RTLD_NOW)
            except OSError:
                return None
            hip.hipGraphGetNodes.argtypes = (ctypes.c_void_p, ctypes.c_void_p,
                                             ctypes.POINTER(ctypes.c_size_t))
            hip.hipGraphNodeGetType.argtypes = (ctypes.c_void_p, ctypes.POINTER(ctypes.c_int))
            return hip
    return None


def graph_nodes(graph) -> dict | None:
    """Kernel nodes and other nodes of a graph captured with ``keep_graph=True``."""
    import ctypes
    hip = _hip_runtime()
    if hip is None:
        return None
    handle = ctypes.c_void_p(graph.raw_cuda_graph())
    count = ctypes.c_size_t(0)
    if hip.hipGraphGetNodes(handle, None, ctypes.byref(count)) != 0:
        return None
    nodes = (ctypes.c_void_p * max(count.value, 1))()
    if hip.hipGraphGetNodes(handle, nodes, ctypes.byref(count)) != 0:
        return None
    kernels = 0
    for k in range(count.value):
        kind = ctypes.c_int(-1)
        if hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[k]), ctypes.byref(kind)) != 0:
            return None
        kernels += kind.value == 0          # hipGraphNodeTypeKernel
    return {"kernels": kernels, "other_nodes": count.value - kernels}


def captured_steps(runtime, inputs: list, fields: tuple, *, keep_graph: bool = False):
    """A graph of ``runtime.step(drive, dendritic_drive=...)`` over ``inputs``
    ((drive, dendritic drive) per tick), captured after one warm-up tick on a side
    stream.  The runtime's ``fields`` are restored afterwards, so its own state is
    as before.  Every replay starts from the states it held at capture; a
    persistent current (updated in place) must be reset by the caller."""
    saved = [getattr(runtime, f).clone() for f in fields]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        runtime.step(inputs[0][0], dendritic_drive=inputs[0][1])
    torch.cuda.current_stream().wait_stream(side)
    for f, value in zip(fields, saved):
        setattr(runtime, f, value.clone())
    graph = torch.cuda.CUDAGraph(keep_graph=keep_graph)
    with torch.cuda.graph(graph):
        for drive, dendritic in inputs:
            runtime.step(drive, dendritic_drive=dendritic)
    return graph, saved


def replayed_ms(runtime, graph, saved: list, fields: tuple, ticks: int, replays: int = 8) -> float:
    """Median ms per tick over ``replays`` replays of a ``captured_steps`` graph;
    the runtime's ``fields`` are restored to ``saved`` afterwards."""
    timings = []
    for _ in range(replays):
        if "persistent_current" in fields:
            runtime.persistent_current.copy_(saved[fields.index("persistent_current")])
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        timings.append(start.elapsed_time(end) / ticks)
    for f, value in zip(fields, saved):
        setattr(runtime, f, value)
    return sorted(timings)[len(timings) // 2]


def measure_pels(device, theta: float = 0.02) -> dict:
    """N=50000, M~1M, B=1: ms/tick of the one-launch event tick in graphs of 64
    ticks, for three activity regimes: drive .2/.1 switched on at a zero state,
    both inputs withdrawn after 512 driven ticks, and quiescence after 4096
    withdrawn ticks.  Each regime's activity (emitting sources and pushed
    edges per tick) is counted on an eager run of the same 64 ticks.  The
    driven regime is also timed on the two-launch tick (advance, then scatter)."""
    n, candidates, chunk = 50_000, 1_000_000, 64
    topology_cpu = random_topology(n, candidates, device="cpu", seed=0)
    topology = topology_to(topology_cpu, device)
    _, model = standard_model(n, device)
    runtime = NativeDendriticPELSRuntime(topology, model, torch.zeros(1, n, device=device),
                                         theta=theta)
    two_launch = NativeDendriticPELSRuntime(topology, model, torch.zeros(1, n, device=device),
                                            theta=theta, one_launch=False)
    out_degree = (topology.out_rowptr[1:] - topology.out_rowptr[:-1]).to(torch.int64)
    fields = ("state", "dendritic_state", "adaptation_state", "emitted_state",
              "persistent_current")
    result = {"workload": f"PELS event tick, N={n} M={topology_cpu.n_edges} B=1, theta {theta}",
              "ticks_per_graph": chunk}

    def phase(drive: float, dendritic: float, runtime=runtime) -> dict:
        with torch.inference_mode():
            saved = [getattr(runtime, f).clone() for f in fields]
            sources = edges = 0
            for _ in range(chunk):
                before = runtime.emitted_state
                runtime.step(drive, dendritic_drive=dendritic)
                changed = runtime.emitted_state[0] != before[0]
                sources += int(changed.sum())
                edges += int(out_degree[changed].sum())
            for f, value in zip(fields, saved):
                setattr(runtime, f, value.clone())
            # The graph's first tick reads these input tensors again on every replay;
            # only the persistent current (with the pending buffer of the one-launch
            # tick) is updated in place, so it is reset each time: reading the
            # attribute folds the outstanding buffer, then the copy overwrites.
            graph, saved = captured_steps(runtime, [(drive, dendritic)] * chunk, fields)
            ms = replayed_ms(runtime, graph, saved, fields, chunk)
        per_tick_sources, per_tick_edges = sources / chunk, edges / chunk
        alg = int(44 * n + 28 * n + 8 * per_tick_sources + 20 * per_tick_edges)
        return {"ms_per_tick": round(ms, 5), "emitting_sources_per_tick": round(per_tick_sources, 1),
                "pushed_edges_per_tick": round(per_tick_edges, 1), "algorithmic_bytes": alg,
                "achieved_GBps": round(alg / ms / 1e6, 1)}

    result["driven_onset"] = phase(0.2, 0.1)
    result["driven_onset_two_launch"] = phase(0.2, 0.1, two_launch)
    # The same onset with the emitted deltas propagated by the matrix product
    # (current += W @ delta after an advance-only launch) instead of the scatter.
    by_matrix = NativeDendriticPELSRuntime(topology, model, torch.zeros(1, n, device=device),
                                           theta=theta, propagation="matrix")
    result["driven_onset_matrix"] = phase(0.2, 0.1, by_matrix)
    del by_matrix
    if theta != 0.0:
        # theta 0: every changed (neuron, column) emits, the exact matrix-equivalent tick
        for name, propagation in (("theta0_driven_onset", "event"),
                                  ("theta0_driven_onset_matrix", "matrix")):
            exact = NativeDendriticPELSRuntime(topology, model, torch.zeros(1, n, device=device),
                                               theta=0.0, propagation=propagation)
            result[name] = phase(0.2, 0.1, exact)
            del exact
    # propagation="auto": the eager ticks that count each regime's activity also
    # let the policy sample it; the captured ticks keep the path it chose.
    for name, value in (("driven_onset_auto", theta), ("theta0_driven_onset_auto", 0.0)):
        chooser = NativeDendriticPELSRuntime(topology, model, torch.zeros(1, n, device=device),
                                             theta=value, propagation="auto")
        result[name] = phase(0.2, 0.1, chooser)
        result[name]["path"] = chooser.selected_path
        del chooser
    del two_launch
    with torch.inference_mode():
        for _ in range(512):
            runtime.step(0.2, dendritic_drive=0.1)
    result["withdrawn_onset"] = phase(0.0, 0.0)
    with torch.inference_mode():
        for _ in range(4096):
            runtime.step(0.0, dendritic_drive=0.0)
    result["quiescent"] = phase(0.0, 0.0)
    return result


def measure_scaleout(device, cpu_sample: bool) -> dict:
    """N=1000000, M~100M, B=16, drive [16,1] U(0,.4) (seed 1), fp8 e4m3 weights,
    200 graph-captured ticks; CPU oracle (fp32, decoded weights) on 10 ticks.  The
    same graph is also timed at B=8 and B=4 (100 ticks each, auto kernel and row
    blocks) under `narrow_batches`."""
    n, candidates, batch = 1_000_000, 100_000_000, 16
    log("scale-out: drawing N=1000000 M=100M candidates on the host, coalescing on the GPU")
    torch.cuda.synchronize()
    start = time.perf_counter()
    topology = random_topology(n, candidates, device="cpu", seed=0, build_device=device)
    torch.cuda.synchronize()
    build_s = time.perf_counter() - start
    topology_cpu = topology_to(topology, "cpu") if cpu_sample else None
    m = topology.n_edges
    model_cpu, model = standard_model(n, device)
    start = time.perf_counter()
    runtime = NativeDendriticMatrixRuntime(topology, model, torch.zeros(batch, n, device=device),
                                           weight_format="fp8")
    torch.cuda.synchronize()
    layout_s = time.perf_counter() - start
    drive = column_drive(batch)
    ms = rollout_ms(runtime, 100, 2, drive.to(device), 0.1)
    alg = algorithmic_bytes("fp8", n, m, batch, parameter_bytes(model, n)) + 4 * batch
    result = {"workload": f"dendritic matrix tick, N={n} M={m} B={batch}, fp8 e4m3 weights, "
                          "per-column drive", "kernel": runtime.kernel, "ticks": 200,
              "ms_per_tick": round(ms, 5), "algorithmic_bytes": alg,
              "achieved_GBps": round(alg / ms / 1e6, 1),
              "pct_hbm_peak": round(100 * alg / ms / 1e6 / HBM_PEAK_GBPS, 1),
              "graph_build_s": round(build_s, 2),
              "graph_build": "host draws (torch CPU generator), ns_build_topology on the GPU",
              "layout_build_s": round(layout_s, 2)}
    if runtime.kernel != "rows":
        del runtime
        rows = NativeDendriticMatrixRuntime(topology, model, torch.zeros(batch, n, device=device),
                                            weight_format="fp8", kernel="rows")
        result["rows_kernel_ms_per_tick"] = round(rollout_ms(rows, 100, 2, drive.to(device), 0.1), 5)
        runtime = rows
    # The same graph at batches 8 and 4 (band tiles of 8 and 4 columns), auto kernel
    # and row blocks, 100 graph-replayed ticks each.
    del runtime
    runtime = None
    narrow = {}
    for b in (8, 4):
        entry = {}
        for kernel in ("auto", "rows"):
            rt = NativeDendriticMatrixRuntime(topology, model, torch.zeros(b, n, device=device),
                                              weight_format="fp8", kernel=kernel)
            key = "ms_per_tick" if kernel == "auto" else "rows_kernel_ms_per_tick"
            if kernel == "auto":
                entry["kernel"] = rt.kernel
            entry[key] = round(rollout_ms(rt, 50, 2, column_drive(b).to(device), 0.1), 5)
            del rt
        narrow[str(b)] = entry
    result["narrow_batches"] = narrow
    if cpu_sample:
        log("scale-out: timing the CPU oracle on 10 ticks")
        from neurosim_gpu.precision import quantize_dequantize
        decoded = quantize_dequantize(topology_cpu.in_weight, "fp8").numpy()
        cpu_ms, threads = oracle_tick_ms(topology_cpu, model_cpu, batch, drive, 10, warmup=1,
                                         weight=decoded)
        result["cpu_baseline"] = {"value": round(cpu_ms, 1), "unit": "ms/tick", "cores": threads,
                                  "kind": "port", "sample": "10 fp32 ticks on the decoded fp8 "
                                  "weights, torch CPU CSR product + elementwise update"}
    torch.cuda.empty_cache()
    return result


# The reference's benchmark protocol (benchmarks/compartmental.py:38-150) and the
# figures it published for it (results/compartmental_performance.json: NVIDIA GeForce
# RTX 5070 Laptop GPU, CUDA 13.2): median ms per eager tick over 7 repeats of 100,
# CUDA-event time, per runtime; "edges" is its graph's coalesced edge count.
PROTOCOL_CASES = ((4096, 65_536, 1), (50_000, 1_000_000, 1), (50_000, 1_000_000, 8),
                  (166_000, 10_000_000, 1), (166_000, 25_000_000, 1))
PROTOCOL_PUBLISHED = {
    (4096, 65_536, 1): dict(edges=65_416, native_matrix=0.01169, native_pels=0.02032,
                            reference_matrix=0.28415, reference_pels_matrix=0.3546),
    (50_000, 1_000_000, 1): dict(edges=999_787, native_matrix=0.06237, native_pels=0.04069,
                                 reference_matrix=0.32694, reference_pels_matrix=0.42247),
    (50_000, 1_000_000, 8): dict(edges=999_787, native_matrix=0.3956, native_pels=0.18265,
                                 reference_matrix=0.66927, reference_pels_matrix=0.74575),
    (166_000, 10_000_000, 1): dict(edges=9_998_214, native_matrix=0.4875, native_pels=0.34573,
                                   reference_matrix=0.76716, reference_pels_matrix=0.84686),
    (166_000, 25_000_000, 1): dict(edges=24_988_704, native_matrix=1.09299, native_pels=0.96258,
                                   reference_matrix=1.44299, reference_pels_matrix=1.53931),
}
# Kernels per tick the reference counted for its native runtimes (first case's profile).
PROTOCOL_PUBLISHED_KERNELS = {"native_matrix": 1, "native_pels": 2}
STATE_FIELDS = ("state", "dendritic_state", "adaptation_state")
PELS_FIELDS = STATE_FIELDS + ("emitted_state", "persistent_current")


def measure_protocol(device, iterations: int = 100, repeats: int = 7) -> dict:
    """The reference's benchmark protocol on this GPU, its published figures beside.

    Per case: random_topology(n, candidates, seed=23) drawn on the GPU, alpha .72,
    gain .8, tau_d 4, tau_a 25 (coupling .5, strength .2), initial state .2, drive
    .2 + .1 sin(0.11 t), dendritic drive .1, theta .02.  Four runtimes: the torch
    matrix runtime, the native matrix runtime, the torch PELS runtime with matrix
    propagation and the native PELS runtime (one launch, scatter).  After 30
    warm-up ticks each runs ``repeats`` blocks of ``iterations`` eager ticks,
    interleaved in an order shuffled per repeat (seed 19); each block is timed with
    HIP events and the host clock, and the medians are kept.  As in the reference,
    every runtime sees the same inputs, so the native states are compared with the
    torch ones at the end (its tolerances: rtol 2e-4 and atol 2e-5 for the matrix
    tick, atol 2e-3 for PELS).  Added here: the native PELS runtime with
    propagation="auto" (a fifth runtime in the same rotation), each native
    runtime's kernels per tick, counted in a captured graph of one tick, and its
    ms per tick when the same inputs run as graph replays of ``iterations`` ticks."""
    import random
    from neurosim_gpu import DendriticMatrixRuntime, DendriticPELSRuntime

    def drive_at(tick: int) -> float:
        return 0.2 + 0.1 * math.sin(tick * 0.11)

    order = random.Random(19)
    cases = []
    with torch.inference_mode():
        for n, candidates, batch in PROTOCOL_CASES:
            log(f"protocol: N={n} candidates={candidates} B={batch}")
            graph = random_topology(n, candidates, device=device, seed=23)
            soma = Dynamics(torch.full((n,), .72, device=device), torch.full((n,), .8, device=device))
            model = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4.,
                                                          tau_adaptation=25.)
            initial = torch.full((batch, n), .2, device=device)
            runtimes = {
                "reference_matrix": DendriticMatrixRuntime(graph, model, initial.clone()),
                "native_matrix": NativeDendriticMatrixRuntime(graph, model, initial.clone()),
                "reference_pels_matrix": DendriticPELSRuntime(graph, model, initial.clone(),
                                                              theta=.02, propagation="matrix"),
                "native_pels": NativeDendriticPELSRuntime(graph, model, initial.clone(), theta=.02),
                # Not in the reference's protocol: the same tick with the propagation
                # chosen from sampled activity (event scatter or matrix product).
                "native_pels_auto": NativeDendriticPELSRuntime(graph, model, initial.clone(),
                                                               theta=.02, propagation="auto"),
            }
            for runtime in runtimes.values():
                for t in range(30):
                    runtime.step(drive_at(t), dendritic_drive=.1)
            torch.cuda.synchronize()
            samples = {name: {"gpu_ms": [], "wall_ms": []} for name in runtimes}
            for repeat in range(repeats):
                names = list(runtimes)
                order.shuffle(names)
                for name in names:
                    runtime = runtimes[name]
                    start = torch.cuda.Event(enable_timing=True)
                    end = torch.cuda.Event(enable_timing=True)
                    torch.cuda.synchronize()
                    wall = time.perf_counter()
                    start.record()
                    for t in range(iterations):
                        runtime.step(drive_at(30 + repeat * iterations + t), dendritic_drive=.1)
                    end.record()
                    end.synchronize()
                    samples[name]["wall_ms"].append((time.perf_counter() - wall) * 1000 / iterations)
                    samples[name]["gpu_ms"].append(start.elapsed_time(end) / iterations)
            published = PROTOCOL_PUBLISHED[(n, candidates, batch)]
            row = {"n": n, "candidate_edges": candidates, "edges": graph.n_edges,
                   "published_edges": published["edges"], "batch": batch,
                   "native_matrix_kernel": runtimes["native_matrix"].kernel, "runtimes": {}}
            for name, data in samples.items():
                gpu = sorted(data["gpu_ms"])[len(data["gpu_ms"]) // 2]
                wall = sorted(data["wall_ms"])[len(data["wall_ms"]) // 2]
                row["runtimes"][name] = {"median_gpu_ms": round(gpu, 5),
                                         "median_wall_ms": round(wall, 5),
                                         "published_rtx5070_gpu_ms": published.get(name)}
            # The reference's memory-probe tick (drive .2), every runtime.
            for name, runtime in runtimes.items():
                torch.cuda.synchronize()
                before = torch.cuda.memory_allocated()
                torch.cuda.reset_peak_memory_stats()
                runtime.step(.2, dendritic_drive=.1)
                torch.cuda.synchronize()
                row["runtimes"][name]["tick_peak_extra_bytes"] = (torch.cuda.max_memory_allocated()
                                                                  - before)
            for native, reference, rtol, atol in (
                    ("native_matrix", "reference_matrix", 2e-4, 2e-5),
                    ("native_pels", "reference_pels_matrix", 0.0, 2e-3),
                    ("native_pels_auto", "reference_pels_matrix", 0.0, 2e-3)):
                a, b = runtimes[native], runtimes[reference]
                errors = [(getattr(a, f) - getattr(b, f)).abs() for f in STATE_FIELDS]
                within = all(bool((e <= atol + rtol * getattr(b, f).abs()).all())
                             for e, f in zip(errors, STATE_FIELDS))
                row["runtimes"][native]["state_max_abs_error"] = float(errors[0].max())
                row["runtimes"][native]["within_reference_tolerance"] = within
                if not within:
                    log(f"protocol: {native} left the reference's tolerance at N={n} B={batch}")
            inputs = [(drive_at(30 + repeats * iterations + 1 + t), .1) for t in range(iterations)]
            row["runtimes"]["native_pels_auto"]["path"] = runtimes["native_pels_auto"].selected_path
            for name, fields in (("native_matrix", STATE_FIELDS), ("native_pels", PELS_FIELDS),
                                 ("native_pels_auto", PELS_FIELDS)):
                runtime = runtimes[name]
                one, saved = captured_steps(runtime, inputs[:1], fields, keep_graph=True)
                row["runtimes"][name]["kernels_per_tick"] = graph_nodes(one)
                for f, value in zip(fields, saved):
                    setattr(runtime, f, value)
                del one
                graph_of_ticks, saved = captured_steps(runtime, inputs, fields)
                row["runtimes"][name]["graph_replay_ms"] = round(
                    replayed_ms(runtime, graph_of_ticks, saved, fields, iterations), 5)
                del graph_of_ticks
            for name in ("native_matrix", "native_pels"):
                entry = row["runtimes"][name]
                entry["rtx5070_over_this_gpu"] = round(published[name] / entry["median_gpu_ms"], 2)
            log(f"protocol: {row}")
            cases.append(row)
            del runtimes, runtime, graph, model, initial
            gc.collect()
            torch.cuda.empty_cache()
    return {"protocol": "benchmarks/compartmental.py: seed 23 (GPU generator), initial .2, "
                        "drive .2+.1*sin(0.11 t), dendritic .1, theta .02, 30 warm-up ticks, "
                        f"{repeats} x {iterations} eager ticks interleaved (shuffle seed 19), "
                        "medians; float32",
            "published": "results/compartmental_performance.json, NVIDIA GeForce RTX 5070 "
                         "Laptop GPU",
            "published_kernels_per_tick": PROTOCOL_PUBLISHED_KERNELS, "cases": cases}


PRECISION_MODES = ("fp32", "fp16", "fp8", "nvfp4")
PRECISION_CASES = (("small", 1024, 16_384, 8), ("large", 50_000, 1_000_000, 8))
# results/precision_native.json (NVIDIA GeForce RTX 5070 Laptop GPU): per mode the
# median GPU and wall ms per tick, the weight payload bytes and the state's peak
# |error| against the fp32 runtime over the 72 probe ticks.
PRECISION_PUBLISHED = {
    "small": {"edges": 16_273,
              "fp32": (0.02098, 0.02208, 65_092, 0.0), "fp16": (0.01871, 0.02554, 32_546, 1.648e-5),
              "fp8": (0.02004, 0.02057, 16_277, 2.105e-3), "nvfp4": (0.02124, 0.02487, 9_159, 5.629e-3)},
    "large": {"edges": 999_787,
              "fp32": (0.44973, 0.45098, 3_999_148, 0.0), "fp16": (0.44543, 0.44796, 1_999_574, 1.745e-5),
              "fp8": (0.44356, 0.44461, 999_791, 2.382e-3), "nvfp4": (0.49787, 0.49992, 562_385, 8.233e-3)},
}


def measure_precision_native(device, iterations: int = 60, repeats: int = 5, warmup: int = 12) -> dict:
    """The reference's reduced-weight-storage benchmark on this GPU, its published figures beside.

    benchmarks/precision_native.py: per workload random_topology(n, candidates,
    seed=23, weight_scale=.15) drawn on the GPU, batch 8, initial state .25, the
    model of benchmarks/precision_compartmental.py:33-41 (alpha .72, gain .8,
    retentions exp(-1/4) and exp(-1/20), coupling .45, adaptation strength .15, all
    per-neuron vectors), drive .16 + .04 (t mod 7)/6 and dendritic drive .025.  For
    each of ``repeats`` orders of the four weight modes (shuffled, seed 19) a fresh
    native matrix runtime takes one tick, ``warmup - 1`` more and then ``iterations``
    timed eager ticks (HIP events and the host clock); medians are kept.  Then fresh
    fp32 and mode runtimes step in lockstep for ``warmup + iterations`` ticks and the
    peak and mean |mode - fp32| of every state field are recorded.  The graph differs
    from the reference's (another device generator draws it), so the error figures
    compare as statistics, not tick by tick."""
    import random

    def drive_at(tick: int) -> float:
        return 0.16 + 0.04 * ((tick % 7) / 6.0)

    options = {"fp32": {}, "fp16": {"weight_dtype": torch.float16},
               "fp8": {"weight_format": "fp8"}, "nvfp4": {"weight_format": "nvfp4"}}
    shuffle = random.Random(19)
    orders = []
    for _ in range(repeats):
        order = list(PRECISION_MODES)
        shuffle.shuffle(order)
        orders.append(order)
    workloads = {}
    with torch.no_grad():
        for name, n, candidates, batch in PRECISION_CASES:
            log(f"precision_native: {name} N={n} candidates={candidates} B={batch}")
            graph = random_topology(n, candidates, device=device, seed=23, weight_scale=0.15)
            initial = torch.full((batch, n), 0.25, device=device)

            def full(value):
                return torch.full((n,), value, device=device)

            model = DendriticDynamics(Dynamics(full(.72), full(.8)), full(math.exp(-1 / 4)),
                                      full(math.exp(-1 / 20)), full(.45), full(.15))

            def fresh(mode):
                return NativeDendriticMatrixRuntime(graph, model, initial.clone(), **options[mode])

            samples = {mode: {"gpu": [], "wall": [], "resident": []} for mode in PRECISION_MODES}
            meta = {}
            for order in orders:
                for mode in order:
                    torch.cuda.synchronize()
                    before = torch.cuda.memory_allocated()
                    runner = fresh(mode)
                    runner.step(drive_at(0), dendritic_drive=.025)
                    torch.cuda.synchronize()
                    samples[mode]["resident"].append(torch.cuda.memory_allocated() - before)
                    for t in range(1, warmup):
                        runner.step(drive_at(t), dendritic_drive=.025)
                    start = torch.cuda.Event(enable_timing=True)
                    end = torch.cuda.Event(enable_timing=True)
                    torch.cuda.synchronize()
                    wall = time.perf_counter()
                    start.record()
                    for t in range(iterations):
                        runner.step(drive_at(warmup + t), dendritic_drive=.025)
                    end.record()
                    end.synchronize()
                    samples[mode]["wall"].append((time.perf_counter() - wall) * 1000 / iterations)
                    samples[mode]["gpu"].append(start.elapsed_time(end) / iterations)
                    meta[mode] = {"execution": runner.last_backend, "kernel": runner.kernel,
                                  "weight_storage_bytes": runner.weight_storage_bytes}
                    del runner
            published = PRECISION_PUBLISHED[name]
            rows = {}
            for mode in PRECISION_MODES:
                gpu = statistics.median(samples[mode]["gpu"])
                wall = statistics.median(samples[mode]["wall"])
                reference, candidate = fresh("fp32"), fresh(mode)
                peaks = {f: [] for f in STATE_FIELDS}
                means = {f: [] for f in STATE_FIELDS}
                for t in range(warmup + iterations):
                    for runner in (reference, candidate):
                        runner.step(drive_at(t), dendritic_drive=.025)
                    for f in STATE_FIELDS:
                        error = (getattr(candidate, f) - getattr(reference, f)).abs()
                        peaks[f].append(error.max())
                        means[f].append(error.mean())
                trajectory = {f: {"max_abs_error": float(torch.stack(peaks[f]).max()),
                                  "mean_abs_error": float(torch.stack(means[f]).mean()),
                                  "final_max_abs_error": float(peaks[f][-1])}
                              for f in STATE_FIELDS}
                del reference, candidate
                pub_gpu, pub_wall, pub_bytes, pub_error = published[mode]
                rows[mode] = {"median_gpu_ms_per_tick": round(gpu, 5),
                              "median_wall_ms_per_tick": round(wall, 5), **meta[mode],
                              "resident_extra_bytes_after_first_tick":
                                  statistics.median(samples[mode]["resident"]),
                              "trajectory_error_vs_fp32": trajectory,
                              "published_rtx5070": {"median_gpu_ms_per_tick": pub_gpu,
                                                    "median_wall_ms_per_tick": pub_wall,
                                                    "weight_storage_bytes": pub_bytes,
                                                    "state_max_abs_error": pub_error},
                              "rtx5070_over_this_gpu_wall": round(pub_wall / wall, 2)}
            for mode in PRECISION_MODES:
                rows[mode]["speedup_wall_vs_fp32"] = round(
                    rows["fp32"]["median_wall_ms_per_tick"] / rows[mode]["median_wall_ms_per_tick"], 3)
            workloads[name] = {"n": n, "candidate_edges": candidates, "edges": graph.n_edges,
                               "published_edges": published["edges"], "batch": batch,
                               "modes": rows}
            log(f"precision_native {name}: " + ", ".join(
                f"{mode} {rows[mode]['median_wall_ms_per_tick']} ms" for mode in PRECISION_MODES))
            del graph, model, initial
            gc.collect()
            torch.cuda.empty_cache()
    return {"protocol": "benchmarks/precision_native.py: seed 23 (GPU generator), weight scale "
                        ".15, B=8, initial .25, drive .16+.04*(t mod 7)/6, dendritic .025, "
                        f"{warmup} warm-up ticks, {repeats} x {iterations} eager ticks per mode "
                        "in shuffled orders (seed 19), medians; trajectory error over "
                        f"{warmup + iterations} ticks against the fp32 runtime",
            "published": "results/precision_native.json, NVIDIA GeForce RTX 5070 Laptop GPU",
            "workloads": workloads}


def main() -> None:
    cli = argparse.ArgumentParser(description=__doc__)
    cli.add_argument("--gpus", type=int, default=1)
    cli.add_argument("--steps", type=int, default=1000)
    cli.add_argument("--warmup", type=int, default=100)
    cli.add_argument("--formats", default="fp32,fp16,fp8,nvfp4")
    cli.add_argument("--no-cpu-baseline", action="store_true")
    cli.add_argument("--no-mall-flush", action="store_true")
    cli.add_argument("--kernel", default="auto", choices=("auto", "rows", "panels", "bands"),
                     help="headline tick kernel: LDS column panels (batch 1-2), source bands "
                          "(batch a multiple of 4) or CSR row blocks")
    cli.add_argument("--copy-calibration", action="store_true",
                     help="only run 256 MiB device copies (PMC byte-counter calibration)")
    cli.add_argument("--configs",
                     default="encode,backward,weights,batched,pels,scaleout,protocol,precision",
                     help="other workloads to time after the headline one ('none' for none)")
    args = cli.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the tick would shard by batch columns or by destination rows); run with --gpus 1",
              file=sys.stderr)
        sys.exit(2)
    if args.steps <= 0 or args.warmup < 0:
        cli.error("steps must be positive and warmup non-negative")
    device = torch.device("cuda:0")
    torch.cuda.set_device(device)
    if args.copy_calibration:
        copy_calibration()
        return
    log("building graph on the host")
    topology_cpu = random_topology(N_NEURONS, CANDIDATES, device="cpu", seed=SEED)
    m = topology_cpu.n_edges
    model_cpu, model = standard_model(N_NEURONS, device)
    topology = topology_to(topology_cpu, device)
    results = {}
    flushed = None
    for fmt in args.formats.split(","):
        log(f"timing {fmt}: {args.warmup} warm-up + {args.steps} ticks")
        runtime = build_runtime(fmt, topology, model, device, args.kernel)
        ms, rollout = time_ticks(runtime, args.steps, args.warmup)
        alg = algorithmic_bytes(fmt, N_NEURONS, m, BATCH, parameter_bytes(model, N_NEURONS))
        results[fmt] = {"ms_per_tick": round(ms, 5), "ticks_per_s": round(1000.0 / ms, 1),
                        "algorithmic_bytes": alg, "achieved_GBps": round(alg / ms / 1e6, 1),
                        "pct_hbm_peak": round(100 * alg / ms / 1e6 / HBM_PEAK_GBPS, 1),
                        "kernel": runtime.kernel, "launches_per_tick": launches_per_tick(runtime),
                        "ticks_per_graph": rollout.ticks}
        if fmt == "fp32" and not args.no_mall_flush:
            flushed_both = mall_flushed_ms(rollout)
            flushed = flushed_both["ms_per_tick"]
            results[fmt]["mall_flushed_ms_per_tick"] = round(flushed, 5)
            results[fmt]["mall_flushed_eager_ms_per_tick"] = round(
                flushed_both["eager_ms_per_tick"], 5)
        log(f"{fmt}: {results[fmt]}")
        del runtime, rollout
        torch.cuda.empty_cache()
    primary_fmt = "fp32" if "fp32" in results else next(iter(results))
    primary = results[primary_fmt]
    ms = primary["ms_per_tick"]
    achieved = primary["algorithmic_bytes"] / ms / 1e6
    traffic = measured_traffic(primary_fmt)
    line = {
        "metric": METRIC, "value": ms, "unit": "ms/tick", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": ms, "higher_is_better": False, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": WORKLOAD, "n_neurons": N_NEURONS, "n_edges": m, "batch": BATCH,
                   "candidate_edges": CANDIDATES, "seed": SEED, "weights": primary_fmt,
                   "ticks_per_graph": primary["ticks_per_graph"], "kernel": primary["kernel"],
                   "launches_per_tick": primary["launches_per_tick"]},
        "ticks_per_s": primary["ticks_per_s"],
        "achieved_GBps": round(achieved, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic},
        "formats": results,
        "host": host_info(),
    }
    if flushed is not None:
        # the same algorithmic bytes over a tick whose graph was first evicted from the MALL
        line["roofline"]["frac_mall_flushed"] = round(
            primary["algorithmic_bytes"] / flushed / 1e6 / HBM_PEAK_GBPS, 4)
    if flushed is not None:
        line["mall_flushed"] = {"ms_per_tick": round(flushed, 5),
                                "achieved_GBps": round(primary["algorithmic_bytes"] / flushed / 1e6, 1),
                                "eager_ms_per_tick": primary.get("mall_flushed_eager_ms_per_tick"),
                                "method": "graph replays: (evictions + ticks) minus evictions "
                                          "alone, per tick; eager: one tick after each eviction"}
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        line["cpu_baseline"] = cpu_baseline(topology_cpu, model_cpu)
    extra = {}
    configs = [c for c in args.configs.split(",") if c and c != "none"]
    if "encode" in configs:
        log("timing encode")
        extra["encode"] = measure_encode(topology.in_weight)
        log(f"encode: {extra['encode']}")
    if "backward" in configs:
        log("timing backward")
        extra["backward"] = measure_backward(topology, model)
        log(f"backward: {extra['backward']}")
    if "weights" in configs:
        log("timing ticks with a new weight version each")
        extra["weight_change"] = measure_weight_change(topology, model, device)
        log(f"weight_change: {extra['weight_change']}")
    del topology
    torch.cuda.empty_cache()
    for name in [c for c in configs if c not in ("encode", "backward", "weights")]:
        log(f"timing {name}")
        if name == "batched":
            extra[name] = measure_batched(device)
        elif name == "pels":
            extra[name] = measure_pels(device)
        elif name == "scaleout":
            extra[name] = measure_scaleout(device, not args.no_cpu_baseline)
        elif name == "protocol":
            extra[name] = measure_protocol(device)
        elif name == "precision":
            extra[name] = measure_precision_native(device)
        else:
            cli.error(f"unknown config {name}")
        log(f"{name}: {extra[name]}")
    if extra:
        line["configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
