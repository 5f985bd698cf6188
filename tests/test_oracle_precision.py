"""Pins of the oracle weight codecs, and product codec == oracle codec bitwise.

e4m3 decode/encode are checked against torch's float8_e4m3fn conversion (an
implementation of the OCP spec) on all 256 codes and on every float32 value at
and next to each rounding boundary of the e4m3 grid.  The e2m1 encoder is
checked against a brute-force nearest-level search whose tie rule is "even
code" (reference precision.py:68-73).  Reference test cases reused:
zero stays zero (test_precision.py:26-29), exact tables
(test_precision_constants.py:14-30).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import precision as op
from neurosim_gpu import precision as pp


def test_e4m3_decode_all_codes_against_torch():
    codes = np.arange(256, dtype=np.uint8)
    ours = op.e4m3_decode(codes)
    torch_values = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    same = (ours == torch_values) | (np.isnan(ours) & np.isnan(torch_values))
    assert same.all()
    assert np.isnan(ours[0x7F]) and np.isnan(ours[0xFF])
    assert ours[0x7E] == 448.0 and ours[0x01] == 2.0 ** -9 and ours[0x08] == 2.0 ** -6


def boundary_probes() -> np.ndarray:
    grid = op.e4m3_decode(np.arange(0x7F, dtype=np.uint8)).astype(np.float64)
    mids = (grid[:-1] + grid[1:]) / 2.0
    values = np.concatenate([grid, mids]).astype(np.float32)
    nxt_up = np.nextafter(values, np.float32(np.inf))
    nxt_dn = np.nextafter(values, np.float32(-np.inf))
    probes = np.concatenate([values, nxt_up, nxt_dn])
    probes = probes[(probes >= 0) & (probes <= 448)]
    return np.concatenate([probes, -probes]).astype(np.float32)


def test_e4m3_encode_rounds_like_torch_at_every_boundary():
    probes = boundary_probes()
    ours = op.e4m3_encode(probes)
    theirs = torch.from_numpy(probes).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    assert np.array_equal(ours, theirs)


def brute_e2m1(normalized: np.ndarray) -> np.ndarray:
    """Nearest level by exhaustive distance; exact ties to the even code."""
    levels = op.E2M1_LEVELS.astype(np.float64)
    out = []
    for x in normalized.astype(np.float64).ravel():
        dist = np.abs(levels - x)
        best = np.flatnonzero(dist == dist.min())
        out.append(best[0] if len(best) == 1 else [b for b in best if b % 2 == 0][0])
    return np.array(out, dtype=np.uint8).reshape(normalized.shape)


def crafted_vectors():
    rng = np.random.default_rng(7)
    yield rng.standard_normal(605).astype(np.float32) * 0.03
    yield np.zeros(19, np.float32)
    yield np.array([-0.0, 0.0, 1.0, -1.0], np.float32)
    yield np.concatenate([np.zeros(16, np.float32), rng.standard_normal(17).astype(np.float32)])
    yield (rng.standard_normal(64) * 1e-30).astype(np.float32)
    yield (rng.standard_normal(48) * 1e30).astype(np.float32)
    # exact midpoints of one block: |w|/unit hits every midpoint when amax = 6*unit
    block = np.array([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, -0.25, -0.75, -1.25, -1.75,
                      -2.5, -3.5, -5.0, 0.0], np.float32)
    yield block
    yield block * np.float32(0.125)


def test_e2m1_encoder_matches_brute_force():
    for vector in crafted_vectors():
        codes, block_codes, scale = op.encode_e2m1(vector)
        pad = (-vector.size) % 16
        blocks = np.concatenate([vector, np.zeros(pad, np.float32)]).reshape(-1, 16)
        unit = (np.float32(scale) * op.e4m3_decode(block_codes)).astype(np.float32)
        safe = np.where(unit > 0, unit, np.float32(1.0)).astype(np.float32)
        normalized = (np.abs(blocks) / safe[:, None]).astype(np.float32)
        assert np.array_equal(codes & 7, brute_e2m1(normalized))
        assert np.array_equal(codes >> 3, np.signbit(blocks).astype(np.uint8))


def test_midpoint_block_hits_even_codes():
    block = np.array([6.0, 0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0] + [0.0] * 8, np.float32)
    codes, block_codes, scale = op.encode_e2m1(block)
    assert op.e4m3_decode(block_codes)[0] * scale == pytest.approx(1.0)
    assert list(codes[0, :8] & 7) == [7, 0, 2, 2, 4, 4, 6, 6]


def test_zero_input_stays_zero_and_tables():
    assert np.array_equal(op.quantize_dequantize(np.zeros(38, np.float32), "nvfp4"),
                          np.zeros(38, np.float32))
    assert list(op.E2M1_LEVELS) == [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    assert list(op.E2M1_MIDPOINTS) == [0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0]


@pytest.mark.parametrize("fmt", ["fp8", "nvfp4"])
def test_product_encoder_equals_oracle_bitwise(fmt):
    for vector in crafted_vectors():
        t = torch.from_numpy(vector.copy())
        codes, scales, scale = pp.encode_sparse_weights(t, fmt)
        ocodes, oscales, oscale = op.encode_sparse_weights(vector, fmt)
        assert np.array_equal(codes.numpy(), ocodes)
        assert np.float32(scale.item()) == oscale
        if fmt == "nvfp4":
            assert np.array_equal(scales.numpy(), oscales)
        else:
            assert scales is None
        decoded = pp.quantize_dequantize(t, fmt).numpy()
        assert np.array_equal(decoded, op.quantize_dequantize(vector, fmt))
        # packed payload decodes edge by edge to the same values
        assert np.array_equal(op.decode_packed(ocodes, oscales, oscale, vector.size, fmt), decoded)


def test_empty_weights_encode():
    for fmt in ("fp8", "nvfp4"):
        codes, scales, scale = pp.encode_sparse_weights(torch.zeros(0), fmt)
        assert codes.numel() == 0
        assert scale.item() == np.finfo(np.float32).tiny
        if fmt == "nvfp4":
            assert scales.numel() == 0


def test_quantize_dequantize_ste_and_validation():
    source = torch.linspace(-2.0, 2.0, 77).reshape(7, 11)
    for fmt in ("fp16", "fp8", "nvfp4"):
        value = source.clone().requires_grad_()
        decoded = pp.quantize_dequantize(value, fmt)
        assert decoded.shape == value.shape and torch.isfinite(decoded).all()
        decoded.sum().backward()
        assert torch.equal(value.grad, torch.ones_like(value))
    with pytest.raises(ValueError, match="precision must be"):
        pp.quantize_dequantize(torch.ones(2), "fp6")


def test_product_e2m1_rounding_matches_brute_force():
    """The product codec rounds on the e2m1 grid's three lattices; brute force:
    the nearest magnitude, ties to the even code, everything above 6 to 7."""
    from neurosim_gpu.precision import _NVFP4Codec

    levels = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], np.float32)
    grid = np.arange(0, 8 * 256 + 1, dtype=np.float32) / 256
    mids = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0, 6.0], np.float32)
    near = np.concatenate([np.nextafter(mids, 0), mids, np.nextafter(mids, 9)])
    x = np.concatenate([grid, near, np.array([7.0, 100.0, 3e38], np.float32)])
    distance = np.abs(x[:, None].astype(np.float64) - levels[None, :])
    best = distance.min(1, keepdims=True)
    candidates = distance == best
    # ties: the even code of the two; otherwise the only candidate
    expected = np.where(candidates.sum(1) > 1,
                        np.argmax(candidates & (np.arange(8) % 2 == 0), 1),
                        np.argmax(candidates, 1))
    expected[x > 6] = 7          # float64 distances cannot tell huge values apart
    got = _NVFP4Codec._nearest_code(torch.from_numpy(x)).numpy()
    assert np.array_equal(got, expected)
