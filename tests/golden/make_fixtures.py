"""Extract the reference-held result data used as golden vectors.

Reads two result files of the reference checkout (data, not code) and writes
compact fixtures next to this script:

* probe_cpu.json  <- results/compartmental_probe_cpu.json: FP64, N=32, M=0,
  B=2, 400 ticks, five variants, per-tick population means of soma /
  dendrite / adaptation, plus the summary metrics.
* brainwaves.npz + brainwaves_meta.json <- results/compartmental_brainwaves.json:
  N=1024 graph from random_topology(1024, 20480, seed=23) (20295 edges), the
  shared state means after 512 warm-up ticks, the post-warm-up group inputs,
  and the 4096-tick population-mean soma traces of both rows (row 0 keeps
  its inputs, row 1 has both drives withdrawn).
* drift.npz + drift_summary.json <- results/precision_drift.json.gz: the
  100,000-tick schedule of 429 sample ticks; for every scenario and seed
  (11, 23, 47; native backend) the graph's edge count, the per-sample RMSE,
  max-abs and bias curves of fp16/fp8/NVFP4 against FP32 for the three
  states, the mean and standard deviation of the FP32 run's states, and the
  max-abs difference between its native and torch FP32 runs; and
  for seed 11 the summary figures the reference computed from the curves.

Usage: python tests/golden/make_fixtures.py [/root/reference]
"""

from __future__ import annotations

import gzip
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def main(reference: Path) -> None:
    probe = json.loads((reference / "results/compartmental_probe_cpu.json").read_text())
    compact = {
        "config": probe["config"],
        "metrics": probe["metrics"],
        "traces": {name: {key: [row[key] for row in rows]
                          for key in ("drive", "dendritic_drive", "soma", "dendrite", "adaptation")}
                   for name, rows in probe["traces"].items()},
    }
    (HERE / "probe_cpu.json").write_text(json.dumps(compact) + "\n")

    waves = json.loads((reference / "results/compartmental_brainwaves.json").read_text())
    sim = waves["simulation"]
    meta = {key: sim[key] for key in ("neurons", "actual_edges", "candidate_edges", "graph_seed",
                                      "input_seed", "warmup_ticks", "ticks_per_condition",
                                      "groups", "parameters", "shared_initial_state_means",
                                      "topology_sha256")}
    meta["mean_last_512_ticks"] = {k: waves["measurements"][k]["mean_last_512_ticks"]
                                   for k in ("driven", "zero_input")}
    (HERE / "brainwaves_meta.json").write_text(json.dumps(meta, indent=1) + "\n")
    inputs = waves["continued_input_group_traces"]
    np.savez_compressed(
        HERE / "brainwaves.npz",
        somatic=np.asarray(inputs["somatic"], dtype=np.float32),
        dendritic=np.asarray(inputs["dendritic"], dtype=np.float32),
        driven_mean=np.asarray(waves["measurements"]["driven"]["population_mean_trace"]),
        zero_mean=np.asarray(waves["measurements"]["zero_input"]["population_mean_trace"]))

    with gzip.open(reference / "results/precision_drift.json.gz", "rt") as handle:
        drift = json.load(handle)
    modes, fields = ("fp16", "fp8", "nvfp4"), ("state", "dendritic_state", "adaptation_state")
    kept = [case for case in drift["cases"] if case["backend"] == "native"]
    arrays = {"ticks": np.asarray([s["tick"] for s in kept[0]["samples"]], dtype=np.int64)}
    summary = {"steps": drift["protocol"]["steps"],
               "sample_interval": drift["protocol"]["sample_interval"], "cases": {}}
    edges = {}
    for case in kept:
        assert [s["tick"] for s in case["samples"]] == arrays["ticks"].tolist()
        key = f"{case['scenario']}_s{case['seed']}"
        edges[case["seed"]] = case["edges"]
        for stat in ("rmse", "max_abs", "bias"):
            arrays[f"{key}_{stat}"] = np.asarray(
                [[[s["precisions"][m][f][stat] for s in case["samples"]] for f in fields]
                 for m in modes], dtype=np.float64)
        for stat in ("mean", "std"):
            arrays[f"{key}_fp32_{stat}"] = np.asarray(
                [[s["reference"][f][stat] for s in case["samples"]] for f in fields],
                dtype=np.float64)
        # The reference's control: its native FP32 run against its torch FP32 run.
        arrays[f"{key}_control_max_abs"] = np.asarray(
            [[s["fp32_other_backend"][f]["max_abs"] for s in case["samples"]] for f in fields],
            dtype=np.float64)
        if case["seed"] == 11:
            summary["cases"][case["scenario"]] = {
                m: {f: {k: v for k, v in case["summary"][m][f].items() if k != "final"}
                    for f in fields} for m in modes}
    arrays["edges"] = np.asarray(sorted(edges.items()), dtype=np.int64)
    np.savez_compressed(HERE / "drift.npz", **arrays)
    (HERE / "drift_summary.json").write_text(json.dumps(summary, indent=1) + "\n")


if __name__ == "__main__":
    main(Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference"))
