"""ULP sweep of the device tanh the tick uses (MI355X).

The tick computes d' = rho_d*d + (1-rho_d)*tanh(j + v) with floating-point
contraction off.  With no edges (j = 0), rho_d = 0 and d = 0 that is exactly
0*0 + 1*tanh(v) = tanh(v), so a tick over N neurons whose dendritic drive is a
grid of float32 values returns the device tanh of every value through the
C ABI, as the kernels evaluate it.

The grid is every 29th float32 bit pattern of [0, 10] with both signs (about
75 million values), the first 2^16 patterns above 0 (denormals and tiny
values, where tanh(x) rounds to x), and special values.  Each result is
compared with the correctly rounded tanh (float64 tanh rounded to float32) and
with torch's CPU float32 tanh, which the reference's CPU path calls
(compartmental.py:171).  The ULP distance counts representable float32 values
between two results.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from neurosim_gpu import load_native_extension

pytestmark = pytest.mark.gpu

CHUNK = 1 << 24


def float_grid() -> np.ndarray:
    ten = np.array([10.0], np.float32).view(np.uint32)[0]
    bits = np.concatenate([np.arange(0, ten + 1, 29, dtype=np.uint32),
                           np.arange(1, 1 << 16, dtype=np.uint32)])
    positive = bits.view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 9.0, 9.5, 20.0,
                        -20.0, 88.7, -88.7, 1e30, -1e30, np.finfo(np.float32).max,
                        -np.finfo(np.float32).max, 0.5493, -0.5493], np.float32)
    return np.concatenate([positive, -positive, special])


def ordered(x: np.ndarray) -> np.ndarray:
    """float32 bit patterns mapped to integers in value order (+0 and -0 meet)."""
    bits = x.view(np.int32).astype(np.int64)
    return np.where(bits < 0, -(bits & 0x7FFFFFFF), bits)


def ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.abs(ordered(a) - ordered(b))


def device_tanh(x: np.ndarray, gpu) -> np.ndarray:
    ext = load_native_extension()
    out = np.empty_like(x)
    for start in range(0, x.size, CHUNK):
        part = torch.from_numpy(x[start:start + CHUNK]).to(gpu)
        n = part.numel()
        zero = torch.zeros(1, n, device=gpu)
        one = torch.ones((), device=gpu).expand(n)
        params = [one * 0.72, one * 0.8, torch.zeros((), device=gpu).expand(n), one * 0.96,
                  one * 0.5, one * 0.2]
        rowptr = torch.zeros(n + 1, dtype=torch.int32, device=gpu)
        col = torch.zeros(0, dtype=torch.int32, device=gpu)
        weight = torch.zeros(0, dtype=torch.float32, device=gpu)
        _, dendrite, _ = ext.dendritic_step(zero, zero, zero, params, rowptr, col, weight,
                                            None, 0.0, part.view(1, n), 0.0, 8)
        out[start:start + n] = dendrite[0].cpu().numpy()
    return out


def test_device_tanh_ulp_sweep(gpu):
    print("case tanh ULP sweep (about 75M float32 values)", flush=True)
    x = float_grid()
    got = device_tanh(x, gpu)
    exact = np.tanh(x.astype(np.float64)).astype(np.float32)
    cpu = torch.tanh(torch.from_numpy(x)).numpy()
    nan = np.isnan(x)
    assert np.all(np.isnan(got[nan]))
    finite = ~nan
    vs_exact = ulps(got[finite], exact[finite])
    vs_cpu = ulps(got[finite], cpu[finite])
    cpu_vs_exact = ulps(cpu[finite], exact[finite])
    worst = int(np.argmax(vs_exact))
    print(f"device tanh: max {vs_exact.max()} ulp from correctly rounded "
          f"(at x={x[finite][worst]!r}), max {vs_cpu.max()} ulp from torch CPU tanh; "
          f"torch CPU tanh itself max {cpu_vs_exact.max()} ulp; "
          f"exact on {np.mean(vs_exact == 0):.4%} of the grid")
    # Bounded, exact at zero and at the ends (the tick adds j = +0 first, so -0 gives +0).
    assert np.all(got[x == 0] == 0)
    assert np.all(got[np.isposinf(x)] == 1.0) and np.all(got[np.isneginf(x)] == -1.0)
    assert np.all(np.abs(got[finite]) <= 1.0)
    assert vs_exact.max() <= 2
    assert vs_cpu.max() <= 3
