"""The device weight encoder (ns_encode_weights) against the oracle's codecs.

Payloads (codes, block scales, global scale) must be bitwise equal to
oracle.precision.encode_sparse_weights, which restates the reference's
encoders (precision.py:45-90) and is pinned against torch's float8_e4m3fn
cast and a brute-force e2m1 search.  Covers empty and odd lengths, partial
NVFP4 blocks, +-0 and all-zero blocks, exact e4m3 rounding midpoints (normal
and subnormal), exact e2m1 level midpoints (ties to the even code), weights
so small the scale clamps to the smallest normal, subnormal weights, and a
huge amax.  The 25M-edge headline payload is checked in test_gpu_matrix.py.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import precision as op
from neurosim_gpu.native import encode_weights

pytestmark = pytest.mark.gpu


def check(values: np.ndarray, fmt: str, gpu) -> None:
    values = np.ascontiguousarray(values, dtype=np.float32)
    codes, scales, scale = encode_weights(torch.from_numpy(values).to(gpu), fmt)
    want_codes, want_scales, want_scale = op.encode_sparse_weights(values, fmt)
    assert scale.dim() == 0
    assert np.float32(scale.item()).tobytes() == np.float32(want_scale).tobytes()
    got = codes.cpu().numpy()
    assert got.shape == want_codes.shape
    bad = np.flatnonzero(got != want_codes)
    assert bad.size == 0, f"{bad.size} codes differ, first at {bad[:5]}: {got[bad[:5]]} vs {want_codes[bad[:5]]}"
    if fmt == "nvfp4":
        assert np.array_equal(scales.cpu().numpy(), want_scales)
    else:
        assert scales is None


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
@pytest.mark.parametrize("size", [0, 1, 3, 15, 16, 17, 31, 33, 1000, 12_345, 1_000_003])
def test_random_weights(gpu, fmt, size):
    print(f"case encode random fmt={fmt} size={size}", flush=True)
    rng = np.random.default_rng(size)
    values = (rng.standard_normal(size) * 0.0335).astype(np.float32)
    check(values, fmt, gpu)


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
def test_signed_zeros_and_zero_blocks(gpu, fmt):
    print(f"case encode zeros fmt={fmt}", flush=True)
    values = np.zeros(53, np.float32)
    values[3] = -0.0
    values[20:36] = -0.0                 # a whole block of negative zeros
    values[40] = 0.5
    values[41] = -0.25
    check(values, fmt, gpu)
    check(np.zeros(16, np.float32), fmt, gpu)
    check(-np.zeros(7, np.float32), fmt, gpu)


def test_e4m3_rounding_midpoints(gpu):
    """amax 448 gives scale 1, so the weights themselves are rounded: every
    midpoint between adjacent codes (ties to even), one float32 step either
    side, normal and subnormal, both signs."""
    print("case encode fp8 midpoints", flush=True)
    grid = op.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)   # 0 .. 448
    mids = ((grid[:-1] + grid[1:]) / 2).astype(np.float32)
    up = np.nextafter(mids, np.float32(np.inf))
    down = np.nextafter(mids, np.float32(0))
    values = np.concatenate([[448.0], mids, up, down, grid.astype(np.float32)]).astype(np.float32)
    values = np.concatenate([values, -values[1:]])
    check(values, "fp8", gpu)


def test_e2m1_level_midpoints(gpu):
    """A block of amax 5.25 has global scale 2^-9, block scale 448 and unit
    0.875 exactly, so (level midpoint x 0.875) normalises to the midpoint
    itself: each tie must go to the even code."""
    print("case encode nvfp4 midpoints", flush=True)
    mids = op.E2M1_MIDPOINTS.astype(np.float32) * np.float32(0.875)
    block = np.concatenate([[5.25], mids, -mids[:5], [0.0, -0.0, 0.875]]).astype(np.float32)
    assert block.size == 16
    near = np.concatenate([[5.25], np.nextafter(mids, np.float32(np.inf)),
                           np.nextafter(mids, np.float32(0)), [0.1]]).astype(np.float32)
    values = np.concatenate([block, near, block[:9]])
    check(values, "nvfp4", gpu)
    check(values, "fp8", gpu)


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
@pytest.mark.parametrize("magnitude", [1e-38, 1e-40, 1e-44, 1e30, 3e38])
def test_extreme_magnitudes(gpu, fmt, magnitude):
    """Scales clamped to the smallest normal float32, subnormal weights, and a
    global scale near the top of the float32 range."""
    print(f"case encode extreme fmt={fmt} magnitude={magnitude}", flush=True)
    rng = np.random.default_rng(7)
    values = (rng.uniform(-1.0, 1.0, 1000) * magnitude).astype(np.float32)
    values[::97] = 0.0
    check(values, fmt, gpu)


def test_runtime_uses_the_device_encoder(gpu):
    """The native runtime's packed payload is the device encoder's, equal to the oracle's."""
    from cases import make_case
    from neurosim_gpu import NativeDendriticMatrixRuntime

    print("case encode runtime payload", flush=True)
    case = make_case(2000, 40_000, 3, gpu)
    for fmt in ("fp8", "nvfp4"):
        rt = NativeDendriticMatrixRuntime(case.topology, case.model, torch.zeros(1, 2000, device=gpu),
                                          weight_format=fmt)
        rt.step(0.2, dendritic_drive=0.1)
        payload, *scales = rt._packed_weight
        want = op.encode_sparse_weights(case.graph.in_weight, fmt)
        assert np.array_equal(payload.cpu().numpy(), want[0])
        assert np.float32(scales[-1].item()) == want[2]
