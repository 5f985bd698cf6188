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
restated) on a bounded sample of the same tick on this host.

    python bench.py [--gpus 1] [--steps 1000] [--warmup 50]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import torch

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "neurosim-gpu_amd"))

from neurosim_gpu import (DendriticDynamics, Dynamics, MatrixRollout,  # noqa: E402
                          NativeDendriticMatrixRuntime, random_topology, topology_to)

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


def algorithmic_bytes(fmt: str, n: int, m: int, batch: int) -> int:
    """rowptr + col + weights + s,d,a reads + s,d,a writes + six parameter vectors."""
    return 4 * (n + 1) + 4 * m + weight_bytes(fmt, m) + 24 * batch * n + 24 * n


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
    rollout.run(warmup // chunk)
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


def mall_flushed_ms(rollout: MatrixRollout, ticks: int = 20) -> float:
    """ms per tick when a 1 GiB write first evicts the graph from the 256 MB last-level cache."""
    scratch = torch.empty(256 * 1024 * 1024, dtype=torch.float32, device="cuda")
    launch, planes = rollout._launch, rollout._sets
    total = 0.0
    for i in range(ticks):
        scratch.fill_(float(i))          # ~0.13 ms of writes keeps the queue ahead of the host
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        launch(planes[0], planes[1])
        end.record()
        end.synchronize()
        total += start.elapsed_time(end)
    del scratch
    return total / ticks


def cpu_baseline(topology_cpu, model_cpu, ticks: int = 20) -> dict:
    """The CPU oracle's float32 tick on this host (bounded sample, all cores)."""
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
    cores = os.cpu_count() or 1
    threads = min(cores, int(os.environ.get("OMP_NUM_THREADS", cores)))
    torch.set_num_threads(threads)
    oracle = ort.MatrixOracle(graph, params, torch.zeros(BATCH, N_NEURONS))
    for _ in range(3):
        oracle.step(0.2, 0.1)
    begin = time.perf_counter()
    for _ in range(ticks):
        oracle.step(0.2, 0.1)
    ms = (time.perf_counter() - begin) * 1000 / ticks
    return {"value": round(ms, 3), "unit": "ms/tick", "cores": threads, "kind": "port",
            "sample": f"{ticks} fp32 ticks (after 3 warm-up) of the same N=166000 M=24988875 B=1 "
                      f"graph, torch CPU CSR product + elementwise update, {threads} threads"}


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


def main() -> None:
    cli = argparse.ArgumentParser(description=__doc__)
    cli.add_argument("--gpus", type=int, default=1)
    cli.add_argument("--steps", type=int, default=1000)
    cli.add_argument("--warmup", type=int, default=100)
    cli.add_argument("--formats", default="fp32,fp16,fp8,nvfp4")
    cli.add_argument("--no-cpu-baseline", action="store_true")
    cli.add_argument("--no-mall-flush", action="store_true")
    cli.add_argument("--kernel", default="auto", choices=("auto", "rows", "panels"),
                     help="tick kernel: LDS column panels (batch 1-2) or CSR row blocks")
    cli.add_argument("--copy-calibration", action="store_true",
                     help="only run 256 MiB device copies (PMC byte-counter calibration)")
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
    soma = Dynamics(torch.full((N_NEURONS,), .72), torch.full((N_NEURONS,), .8))
    model_cpu = DendriticDynamics.from_time_constants(soma, dt=1., tau_dendrite=4.,
                                                      tau_adaptation=25., coupling=.5,
                                                      adaptation_strength=.2)
    topology = topology_to(topology_cpu, device)
    model = DendriticDynamics(Dynamics(soma.alpha.to(device), soma.gain.to(device)),
                              model_cpu.dendrite_decay.to(device),
                              model_cpu.adaptation_decay.to(device),
                              model_cpu.coupling.to(device),
                              model_cpu.adaptation_strength.to(device))
    results = {}
    flushed = None
    for fmt in args.formats.split(","):
        log(f"timing {fmt}: {args.warmup} warm-up + {args.steps} ticks")
        runtime = build_runtime(fmt, topology, model, device, args.kernel)
        ms, rollout = time_ticks(runtime, args.steps, args.warmup)
        alg = algorithmic_bytes(fmt, N_NEURONS, m, BATCH)
        results[fmt] = {"ms_per_tick": round(ms, 5), "ticks_per_s": round(1000.0 / ms, 1),
                        "algorithmic_bytes": alg, "achieved_GBps": round(alg / ms / 1e6, 1),
                        "pct_hbm_peak": round(100 * alg / ms / 1e6 / HBM_PEAK_GBPS, 1)}
        if fmt == "fp32" and not args.no_mall_flush:
            flushed = mall_flushed_ms(rollout)
            results[fmt]["mall_flushed_ms_per_tick"] = round(flushed, 5)
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
                   "ticks_per_graph": CHUNK, "kernel": args.kernel},
        "ticks_per_s": primary["ticks_per_s"],
        "achieved_GBps": round(achieved, 1),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": traffic},
        "formats": results,
    }
    if flushed is not None:
        line["mall_flushed"] = {"ms_per_tick": round(flushed, 5),
                                "achieved_GBps": round(primary["algorithmic_bytes"] / flushed / 1e6, 1)}
    if not args.no_cpu_baseline:
        log("timing the CPU oracle")
        line["cpu_baseline"] = cpu_baseline(topology_cpu, model_cpu)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
