"""Oracle fp8 e4m3 / NVFP4 weight codecs in numpy (test infrastructure only).

Restates _encode_e4m3, _encode_e2m1, encode_sparse_weights and
quantize_dequantize (reference precision.py:45-112) with explicit bit-level
e4m3 rounding written from the OCP 8-bit floating point specification (e4m3fn:
bias 7, three mantissa bits, subnormals, no infinities, 0x7F/0xFF NaN, largest
finite 448) instead of a library cast.

Pins: tests/test_oracle_precision.py compares e4m3_decode on all 256 codes and
e4m3_encode on every float32 midpoint/boundary of the e4m3 grid against
torch's float8_e4m3fn conversion, and the e2m1 encoder against a brute-force
nearest-level search with ties to the even code (precision.py:68-73 states
that rule), plus the reference's zero-stays-zero and table cases
(test_precision.py:26-29, test_precision_constants.py:14-30).
"""

from __future__ import annotations

import numpy as np

F32 = np.float32
TINY = np.finfo(np.float32).tiny
E2M1_LEVELS = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0], dtype=np.float32)
E2M1_MIDPOINTS = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)


def e4m3_decode(codes: np.ndarray) -> np.ndarray:
    """Exact float32 value of each e4m3fn code (NaN for 0x7F/0xFF)."""
    codes = np.asarray(codes, dtype=np.uint8).astype(np.int64)
    sign = np.where(codes & 0x80, -1.0, 1.0)
    exponent = (codes >> 3) & 0xF
    mantissa = codes & 0x7
    magnitude = np.where(exponent == 0, mantissa / 8.0 * 2.0 ** -6,
                         (1.0 + mantissa / 8.0) * np.exp2(exponent - 7.0))
    value = sign * magnitude
    value = np.where((codes & 0x7F) == 0x7F, np.nan, value)
    return value.astype(np.float32)


def e4m3_encode(values: np.ndarray) -> np.ndarray:
    """Round float32 values in [-448, 448] to e4m3fn codes, nearest-even."""
    x = np.asarray(values, dtype=np.float32).astype(np.float64)
    if np.any(np.abs(x) > 448.0) or np.any(np.isnan(x)):
        raise ValueError("e4m3_encode expects finite values within [-448, 448]")
    sign = np.signbit(x).astype(np.int64) << 7
    mag = np.abs(x)
    _, exp2 = np.frexp(mag)              # mag = f * 2**exp2, f in [0.5, 1)
    unbiased = exp2 - 1                  # floor(log2(mag)) for mag > 0
    normal = mag >= 2.0 ** -6
    # Normal: significand q in [1, 2) rounded to 3 fraction bits.
    q = np.where(normal, mag / np.exp2(np.where(normal, unbiased, 0)), 0.0)
    m = np.rint((q - 1.0) * 8.0)
    carry = m >= 8.0
    e_field = np.where(carry, unbiased + 8, unbiased + 7)
    m = np.where(carry, 0.0, m)
    normal_code = (e_field.astype(np.int64) << 3) | m.astype(np.int64)
    # Subnormal: multiples of 2**-9 (a result of 8 is the smallest normal, code 0x08).
    sub_code = np.rint(mag / 2.0 ** -9).astype(np.int64)
    code = np.where(normal, normal_code, sub_code)
    code = np.where(mag == 0.0, 0, code)
    return (code | sign).astype(np.uint8)


def encode_e4m3(value: np.ndarray):
    """Per-tensor fp8: (codes uint8, float32 scale) (precision.py:45-49)."""
    value = np.asarray(value, dtype=np.float32)
    amax = np.abs(value).max() if value.size else F32(0.0)
    scale = max(F32(amax / F32(448.0)), TINY)
    scale = F32(scale)
    scaled = np.clip(value / scale, F32(-448.0), F32(448.0)).astype(np.float32)
    return e4m3_encode(scaled), scale


def encode_e2m1(value: np.ndarray):
    """16-element e2m1 blocks with e4m3 block scales (precision.py:52-73).

    Returns (codes uint8 [blocks, 16] incl. sign bit 3, block-scale codes
    uint8 [blocks], float32 global scale).
    """
    value = np.asarray(value, dtype=np.float32).reshape(-1)
    width = value.size
    pad = (-width) % 16
    blocks = np.concatenate([value, np.zeros(pad, np.float32)]).reshape(-1, 16)
    absolute = np.abs(blocks)
    block_amax = absolute.max(axis=1, keepdims=True) if blocks.size else np.zeros((0, 1), F32)
    amax = block_amax.max() if width else F32(0.0)
    global_scale = F32(max(F32(amax / F32(6.0 * 448.0)), TINY))
    ratio = np.minimum(block_amax / F32(F32(6.0) * global_scale), F32(448.0)).astype(np.float32)
    block_codes = e4m3_encode(ratio)
    block_values = e4m3_decode(block_codes)
    denominator = (global_scale * block_values).astype(np.float32)
    safe = np.where(denominator > 0, denominator, F32(1.0)).astype(np.float32)
    normalized = (absolute / safe).astype(np.float32)
    # Nearest level; an exact midpoint goes to the even code.
    index = np.searchsorted(E2M1_MIDPOINTS, normalized, side="left")
    at_mid = (index < 7) & (normalized == E2M1_MIDPOINTS[np.minimum(index, 6)])
    index = np.where(at_mid & (index % 2 == 1), index + 1, index)
    codes = index.astype(np.uint8) | (np.signbit(blocks).astype(np.uint8) << 3)
    return codes, block_codes.reshape(-1), global_scale


def encode_sparse_weights(value: np.ndarray, precision: str):
    """Packed CSR payloads (precision.py:76-90): (codes, block scales or None, scale)."""
    value = np.asarray(value, dtype=np.float32)
    if precision == "fp8":
        codes, scale = encode_e4m3(value)
        return codes, None, scale
    if precision != "nvfp4":
        raise ValueError("compressed CSR encoding requires fp8 or nvfp4")
    codes, scales, scale = encode_e2m1(value)
    flat = codes.reshape(-1)
    packed = (flat[0::2] | (flat[1::2] << 4)).astype(np.uint8)
    return packed[: (value.size + 1) // 2].copy(), scales, scale


def quantize_dequantize(value: np.ndarray, precision: str) -> np.ndarray:
    """Decode-to-FP32 of a 1-D weight vector (precision.py:93-112)."""
    value = np.asarray(value, dtype=np.float32)
    if precision == "fp32" or value.size == 0:
        return value.copy()
    if precision == "fp16":
        return value.astype(np.float16).astype(np.float32)
    if precision == "fp8":
        codes, scale = encode_e4m3(value)
        return (e4m3_decode(codes) * scale).astype(np.float32)
    codes, block_codes, scale = encode_e2m1(value)
    per_block = (e4m3_decode(block_codes) * scale).astype(np.float32)
    magnitude = (E2M1_LEVELS[codes & 7] * per_block[:, None]).astype(np.float32)
    decoded = np.where(codes >= 8, -magnitude, magnitude).reshape(-1)
    return decoded[: value.size].astype(np.float32)


def decode_packed(packed: np.ndarray, block_codes, scale, n_edges: int,
                  precision: str) -> np.ndarray:
    """Decode packed payloads back to float32 weights, edge by edge."""
    if precision == "fp8":
        return (e4m3_decode(packed[:n_edges]) * F32(scale)).astype(np.float32)
    edges = np.arange(n_edges)
    nibble = (packed[edges >> 1] >> (4 * (edges & 1))) & 15
    per_block = (e4m3_decode(block_codes) * F32(scale)).astype(np.float32)
    magnitude = (E2M1_LEVELS[nibble & 7] * per_block[edges >> 4]).astype(np.float32)
    return np.where(nibble >= 8, -magnitude, magnitude).astype(np.float32)
