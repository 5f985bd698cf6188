"""ns_encode_weights_no_alloc against ns_encode_weights, through the C ABI (MI355X).

The no-allocation encoder keeps its amax partials in a library-owned device
array instead of a caller workspace.  Its payload (codes, NVFP4 block scales,
global scale) must be bitwise the workspace encoder's, on two calls in a row
of which the second is smaller (the array keeps the first call's partials),
for both formats; both are also checked against the CPU oracle's encoder.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import precision as op
from neurosim_gpu import native

pytestmark = pytest.mark.gpu


def encode(lib, weight: torch.Tensor, fmt: str, no_alloc: bool):
    m = weight.numel()
    nvfp4 = fmt == "nvfp4"
    device = weight.device
    codes = torch.empty(max((m + 1) // 2 if nvfp4 else m, 1), dtype=torch.uint8, device=device)
    scales = torch.empty(max((m + 15) // 16, 1), dtype=torch.uint8, device=device)
    scale = torch.empty(1, dtype=torch.float32, device=device)
    workspace = (None if no_alloc else
                 torch.empty(int(lib.ns_encode_workspace_bytes()) // 4, dtype=torch.int32,
                             device=device))
    args = native._EncodeArgs(weight.data_ptr() if m else None, m,
                              native.WEIGHT_NVFP4 if nvfp4 else native.WEIGHT_E4M3, 0,
                              codes.data_ptr(), scales.data_ptr() if nvfp4 else None,
                              scale.data_ptr(), None if workspace is None else workspace.data_ptr())
    stream = torch.cuda.current_stream(device).cuda_stream
    fn = lib.ns_encode_weights_no_alloc if no_alloc else lib.ns_encode_weights
    rc = fn(ctypes.byref(args), stream)
    assert rc == 0, lib.ns_last_error()
    payload = (m + 1) // 2 if nvfp4 else m
    return (codes[:payload].cpu().numpy(), scales[:(m + 15) // 16].cpu().numpy() if nvfp4 else None,
            np.float32(scale.item()))


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
def test_no_alloc_encoder_equals_the_workspace_encoder(gpu, fmt):
    lib = native.load_library()
    rng = np.random.default_rng(17)
    # First a large call with a large amax (1024 partials), then a smaller one
    # with a small amax: the encoder takes the max over its partials, so a
    # stale partial of the first call read by the second would raise the
    # second call's global scale and change every code.
    for m, sigma in ((3_000_001, 3.0), (1_003, 0.05)):
        print(f"case no-alloc encode fmt={fmt} M={m}", flush=True)
        host = (rng.standard_normal(m) * sigma).astype(np.float32)
        weight = torch.from_numpy(host).to(gpu)
        got = encode(lib, weight, fmt, no_alloc=True)
        want = encode(lib, weight, fmt, no_alloc=False)
        assert np.array_equal(got[0], want[0])
        assert got[2].tobytes() == want[2].tobytes()
        if fmt == "nvfp4":
            assert np.array_equal(got[1], want[1])
        codes, scales, scale = op.encode_sparse_weights(host, fmt)
        assert np.array_equal(got[0], codes)
        assert got[2].tobytes() == np.float32(scale).tobytes()
        if fmt == "nvfp4":
            assert np.array_equal(got[1], scales)


def test_no_alloc_encoder_on_a_side_stream_and_empty(gpu):
    lib = native.load_library()
    weight = torch.linspace(-1, 1, 4096, device=gpu)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = encode(lib, weight, "fp8", no_alloc=True)
    torch.cuda.current_stream().wait_stream(side)
    want = encode(lib, weight, "fp8", no_alloc=False)
    assert np.array_equal(got[0], want[0]) and got[2] == want[2]
    empty = torch.zeros(0, dtype=torch.float32, device=gpu)
    got = encode(lib, empty, "nvfp4", no_alloc=True)
    want = encode(lib, empty, "nvfp4", no_alloc=False)
    assert got[2].tobytes() == want[2].tobytes()
