"""The reference's brainwaves protocol (experiments/compartmental_brainwaves.py:45-110)
restated for tests: graph, parameters and AR(1) inputs.

Inputs come from numpy's default_rng(seed + 1): one shared AR(1) somatic series
(rho .75), eight group series (rho .55) and eight dendritic group series
(rho .85), each IIR-filtered with gain sqrt(1 - rho^2), then cast to float32
and repeated over 128 neurons per group.
"""

from __future__ import annotations

import json
import math
from pathlib import Path

import numpy as np

GOLDEN = Path(__file__).resolve().parent / "golden"
NEURONS, CANDIDATES, GROUPS, WARMUP = 1024, 20480, 8, 512


def meta() -> dict:
    return json.loads((GOLDEN / "brainwaves_meta.json").read_text())


def golden() -> dict:
    with np.load(GOLDEN / "brainwaves.npz", allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def group_inputs(ticks: int, seed: int = 24) -> tuple[np.ndarray, np.ndarray]:
    """[ticks, groups] float32 somatic and dendritic drives."""
    from scipy.signal import lfilter

    rng = np.random.default_rng(seed)

    def ar1(columns: int, rho: float) -> np.ndarray:
        noise = rng.standard_normal((ticks, columns))
        return lfilter([math.sqrt(1 - rho ** 2)], [1, -rho], noise, axis=0)

    soma = .20 + .035 * ar1(1, .75) + .075 * ar1(GROUPS, .55)
    dendrite = .10 + .08 * ar1(GROUPS, .85)
    return soma.astype(np.float32), dendrite.astype(np.float32)


def neuron_inputs(ticks: int) -> tuple[np.ndarray, np.ndarray]:
    """[ticks, NEURONS] float32 drives (each group value repeated over its neurons)."""
    soma, dendrite = group_inputs(ticks)
    repeat = NEURONS // GROUPS
    return np.repeat(soma, repeat, axis=1), np.repeat(dendrite, repeat, axis=1)
