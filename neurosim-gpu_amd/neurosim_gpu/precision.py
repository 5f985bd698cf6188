"""Reduced-precision weight formats for the three-state sparse core.

API and rounding rules of the reference's precision module
(src/neurosim_gpu/precision.py:12-112):

* fp16  -- IEEE binary16 storage, decoded exactly to float32.
* fp8   -- OCP e4m3fn codes with one per-tensor float32 scale
           scale = max(amax/448, tiny); codes = e4m3(clamp(w/scale, +-448)).
* nvfp4 -- e2m1 codes (levels 0, .5, 1, 1.5, 2, 3, 4, 6; sign in bit 3) in
           16-element blocks along the last dimension, one e4m3 block scale per
           block and one float32 global scale
           global = max(amax/(6*448), tiny); block = e4m3(min(bamax/(6*global), 448));
           code = nearest level of |w|/(global*block), exact midpoints to the even code.
           Two codes per byte, even element in the low nibble.
"""

from __future__ import annotations

from functools import lru_cache
from typing import Literal, cast

import torch

Precision = Literal["fp32", "fp16", "fp8", "nvfp4"]
PRECISIONS = ("fp32", "fp16", "fp8", "nvfp4")
_E2M1_LEVELS = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)
_E2M1_MIDPOINTS = (0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0)
_FP8_MAX = 448.0
_BLOCK = 16


@lru_cache(maxsize=None)
def _e2m1_constants(device: torch.device, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """Device tables (midpoints, levels), created once per device/dtype.

    Created outside inference mode so later autograd use stays legal, and
    reused so graph-captured quantization allocates no per-call constants.
    """
    with torch.inference_mode(False), torch.no_grad():
        return (torch.tensor(_E2M1_MIDPOINTS, device=device, dtype=dtype),
                torch.tensor(_E2M1_LEVELS, device=device, dtype=dtype))


@lru_cache(maxsize=None)
def _divisors(device: torch.device, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    """0-d device tensors 448 and 6*448, created once per device/dtype.

    Dividing a device tensor by a Python number lets PyTorch's GPU kernels
    multiply by the rounded reciprocal instead, which can move the scale by
    one ulp (and flip codes) against the CPU's correctly rounded division;
    a device-tensor divisor keeps the true quotient on every device.
    """
    with torch.inference_mode(False), torch.no_grad():
        return (torch.tensor(_FP8_MAX, device=device, dtype=dtype),
                torch.tensor(6.0 * _FP8_MAX, device=device, dtype=dtype))


def validate_precision(value: str) -> Precision:
    if value not in PRECISIONS:
        raise ValueError("precision must be 'fp32', 'fp16', 'fp8', or 'nvfp4'")
    return cast(Precision, value)


def _ste(value: torch.Tensor, quantized: torch.Tensor) -> torch.Tensor:
    """Straight-through estimator: forward the quantized value, identity gradient."""
    if torch.is_grad_enabled() and value.requires_grad:
        return quantized + (value - value.detach())
    return quantized


def _tiny() -> float:
    return torch.finfo(torch.float32).tiny


def _encode_e4m3(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    amax = value.abs().amax() if value.numel() else value.new_zeros(())
    fp8_max, _ = _divisors(value.device, value.dtype)
    scale = (amax / fp8_max).clamp_min(_tiny())
    codes = (value / scale).clamp(-_FP8_MAX, _FP8_MAX).to(torch.float8_e4m3fn)
    return codes, scale


def _encode_e2m1(value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Encode along the last dimension, zero-padded on the right to whole blocks."""
    width = value.shape[-1]
    pad = (-width) % _BLOCK
    if pad:
        value = torch.nn.functional.pad(value, (0, pad))
    blocks = value.reshape(*value.shape[:-1], (width + pad) // _BLOCK, _BLOCK)
    magnitude = blocks.abs()
    block_amax = magnitude.amax(dim=-1, keepdim=True)
    amax = block_amax.amax() if value.numel() else value.new_zeros(())
    _, six_fp8_max = _divisors(value.device, value.dtype)
    global_scale = (amax / six_fp8_max).clamp_min(_tiny())
    block_scale = (block_amax / (6.0 * global_scale)).clamp_max(_FP8_MAX).to(torch.float8_e4m3fn)
    unit = global_scale * block_scale.float()
    normalized = magnitude / torch.where(unit > 0, unit, 1.0)
    midpoints, _ = _e2m1_constants(value.device, value.dtype)
    index = torch.bucketize(normalized, midpoints)          # ties land on the lower code
    tie_on_odd = (index % 2 == 1) & (normalized == midpoints[index.clamp_max(6)])
    code = (index + tie_on_odd).to(torch.uint8) | (blocks.signbit().to(torch.uint8) << 3)
    return code, block_scale.squeeze(-1), global_scale


def encode_sparse_weights(value: torch.Tensor, precision: str
                          ) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
    """(packed codes uint8, block scales uint8 or None, float32 global scale)."""
    if value.ndim != 1 or value.dtype != torch.float32:
        raise ValueError("encoding requires a vector of FP32 CSR weights")
    if precision == "fp8":
        codes, scale = _encode_e4m3(value.detach())
        return codes.view(torch.uint8), None, scale
    if precision != "nvfp4":
        raise ValueError("compressed CSR encoding requires fp8 or nvfp4")
    codes, scales, scale = _encode_e2m1(value.detach())
    codes = codes.flatten()
    packed = codes[0::2] | (codes[1::2] << 4)
    return packed[: (value.numel() + 1) // 2].contiguous(), scales.view(torch.uint8), scale


def quantize_dequantize(value: torch.Tensor, precision: Precision) -> torch.Tensor:
    """Round-trip through a format (decode-to-FP32), with STE gradients."""
    validate_precision(precision)
    if precision == "fp32" or value.numel() == 0:
        return value
    if value.dtype != torch.float32:
        raise ValueError("reduced-precision quantization requires an FP32 master tensor")
    if precision == "fp16":
        return _ste(value, value.detach().to(torch.float16).to(value.dtype))
    if precision == "fp8":
        codes, scale = _encode_e4m3(value.detach())
        return _ste(value, codes.float() * scale)
    flat = value.detach() if value.ndim else value.detach().reshape(1)
    codes, block_scales, scale = _encode_e2m1(flat)
    _, levels = _e2m1_constants(value.device, value.dtype)
    magnitude = levels[(codes & 7).long()] * (block_scales.float() * scale).unsqueeze(-1)
    decoded = torch.where(codes >= 8, -magnitude, magnitude).flatten(-2)
    decoded = decoded[..., : flat.shape[-1]].reshape(value.shape)
    return _ste(value, decoded)
