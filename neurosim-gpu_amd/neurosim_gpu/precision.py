"""Reduced-precision weight formats: codecs for fp16, fp8 e4m3 and NVFP4.

The public functions keep the reference's interface and bit rules
(src/neurosim_gpu/precision.py:12-112): ``PRECISIONS``, ``validate_precision``,
``encode_sparse_weights`` (packed CSR payloads) and ``quantize_dequantize``
(decode-to-FP32 emulation with straight-through gradients).  The rules:

* fp16: IEEE binary16, decoded exactly.
* fp8: OCP e4m3fn codes of w / scale with one per-tensor float32 scale,
  scale = max(amax / 448, smallest normal float32), w / scale saturated to +-448.
* nvfp4: e2m1 codes (magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6; sign in bit 3) in
  16-element blocks along the last dimension, one e4m3 scale per block and a
  float32 global scale:
  global = max(amax / (6 * 448), smallest normal float32),
  block = e4m3(min(block amax / (6 * global), 448)),
  code = the nearest magnitude to |w| / (global * block), ties to the even code;
  two codes per byte, the even element in the low nibble.

Each format is a codec object.  The e2m1 grid is three uniform segments (step
1/2 below 2, 1 up to 4, 2 up to 6), so a code is found by scaling the
magnitude onto its segment's integer lattice and rounding half to even there:
in every segment, even lattice points are even codes.
"""

from __future__ import annotations

from functools import lru_cache
from typing import Literal, cast

import torch

Precision = Literal["fp32", "fp16", "fp8", "nvfp4"]
PRECISIONS = ("fp32", "fp16", "fp8", "nvfp4")

E4M3_MAX = 448.0
NVFP4_BLOCK = 16
_E2M1_MAGNITUDES = (0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0)


def validate_precision(value: str) -> Precision:
    if value not in PRECISIONS:
        raise ValueError("precision must be 'fp32', 'fp16', 'fp8', or 'nvfp4'")
    return cast(Precision, value)


@lru_cache(maxsize=None)
def _device_constant(value: float, device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    """A 0-d tensor on ``device``, made once (outside inference mode, so later
    autograd use stays legal; no allocation when a capture replays).

    The scales divide by 448 and 6 * 448 held as device tensors: a GPU
    division by a Python number may multiply by its rounded reciprocal, which
    can move a scale by one ulp (and flip codes) against the correctly rounded
    quotient the CPU computes."""
    with torch.inference_mode(False), torch.no_grad():
        return torch.tensor(value, device=device, dtype=dtype)


@lru_cache(maxsize=None)
def _magnitude_table(device: torch.device, dtype: torch.dtype) -> torch.Tensor:
    with torch.inference_mode(False), torch.no_grad():
        return torch.tensor(_E2M1_MAGNITUDES, device=device, dtype=dtype)


_SMALLEST_NORMAL = torch.finfo(torch.float32).tiny


def _with_identity_gradient(master: torch.Tensor, rounded: torch.Tensor) -> torch.Tensor:
    """``rounded`` forward; under autograd the gradient passes to ``master`` unchanged."""
    if not (torch.is_grad_enabled() and master.requires_grad):
        return rounded
    return rounded + (master - master.detach())


class _HalfCodec:
    def roundtrip(self, value: torch.Tensor) -> torch.Tensor:
        return value.to(torch.float16).to(value.dtype)


class _E4M3Codec:
    """One float32 scale for the whole tensor."""

    def encode(self, value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        peak = value.abs().max() if value.numel() else value.new_zeros(())
        scale = torch.clamp(peak / _device_constant(E4M3_MAX, value.device, value.dtype),
                            min=_SMALLEST_NORMAL)
        codes = torch.clamp(value / scale, -E4M3_MAX, E4M3_MAX).to(torch.float8_e4m3fn)
        return codes, scale

    def roundtrip(self, value: torch.Tensor) -> torch.Tensor:
        codes, scale = self.encode(value)
        return codes.to(value.dtype) * scale


class _NVFP4Codec:
    """Blocks of 16 along the last dimension (zero-padded to whole blocks)."""

    @staticmethod
    def _blocks(value: torch.Tensor) -> torch.Tensor:
        width = value.shape[-1]
        padded = -(-width // NVFP4_BLOCK) * NVFP4_BLOCK
        if padded != width:
            value = torch.nn.functional.pad(value, (0, padded - width))
        return value.unflatten(-1, (padded // NVFP4_BLOCK, NVFP4_BLOCK))

    @staticmethod
    def _nearest_code(x: torch.Tensor) -> torch.Tensor:
        """e2m1 magnitude code of x >= 0: nearest grid point, ties to even, >6 -> 7."""
        low = torch.round(x * 2.0)                 # [0, 2): lattice 1/2, codes 0..4
        mid = torch.round(x) + 2.0                 # [2, 4): lattice 1, codes 4..6
        high = torch.round(x * 0.5) + 4.0          # [4, 6]: lattice 2, codes 6..7
        code = torch.where(x < 2.0, low, torch.where(x < 4.0, mid, high))
        return code.clamp_max(7.0).to(torch.uint8)

    def encode(self, value: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(codes uint8 [..., blocks, 16] with the sign in bit 3, e4m3 block
        scales [..., blocks], float32 global scale)."""
        blocks = self._blocks(value)
        magnitude = blocks.abs()
        block_peak = magnitude.max(dim=-1).values
        peak = block_peak.max() if block_peak.numel() else value.new_zeros(())
        global_scale = torch.clamp(
            peak / _device_constant(6.0 * E4M3_MAX, value.device, value.dtype),
            min=_SMALLEST_NORMAL)
        block_scale = torch.clamp(block_peak / (6.0 * global_scale),
                                  max=E4M3_MAX).to(torch.float8_e4m3fn)
        unit = (global_scale * block_scale.to(value.dtype)).unsqueeze(-1)
        # A zero unit only scales an all-zero block: any divisor gives code 0.
        scaled = magnitude / torch.where(unit > 0, unit, torch.ones_like(unit))
        sign = torch.signbit(blocks).to(torch.uint8) << 3
        return self._nearest_code(scaled) | sign, block_scale, global_scale

    def roundtrip(self, value: torch.Tensor) -> torch.Tensor:
        width = value.shape[-1]
        codes, block_scale, global_scale = self.encode(value)
        magnitude = _magnitude_table(value.device, value.dtype)[(codes & 7).long()]
        scaled = magnitude * (block_scale.to(value.dtype) * global_scale).unsqueeze(-1)
        decoded = torch.where(codes >= 8, -scaled, scaled).flatten(-2)
        return decoded[..., :width]


_CODECS = {"fp16": _HalfCodec(), "fp8": _E4M3Codec(), "nvfp4": _NVFP4Codec()}


def encode_sparse_weights(value: torch.Tensor, precision: str
                          ) -> tuple[torch.Tensor, torch.Tensor | None, torch.Tensor]:
    """CSR weight payload: (codes uint8, block scales uint8 or None, float32 global scale).

    fp8 gives one code byte per edge; NVFP4 two codes per byte (even edge in
    the low nibble) and one scale byte per 16 consecutive edges."""
    if value.ndim != 1 or value.dtype != torch.float32:
        raise ValueError("encoding requires a vector of FP32 CSR weights")
    if precision not in ("fp8", "nvfp4"):
        raise ValueError("compressed CSR encoding requires fp8 or nvfp4")
    weights = value.detach()
    if precision == "fp8":
        codes, scale = _CODECS["fp8"].encode(weights)
        return codes.view(torch.uint8), None, scale
    codes, block_scale, scale = _CODECS["nvfp4"].encode(weights)
    nibbles = codes.reshape(-1, 2)
    packed = nibbles[:, 0] | (nibbles[:, 1] << 4)
    return packed[: (value.numel() + 1) // 2].contiguous(), block_scale.view(torch.uint8), scale


def quantize_dequantize(value: torch.Tensor, precision: Precision) -> torch.Tensor:
    """``value`` rounded through ``precision`` and decoded to its own dtype, with
    identity (straight-through) gradients."""
    validate_precision(precision)
    if precision == "fp32" or value.numel() == 0:
        return value
    if value.dtype != torch.float32:
        raise ValueError("reduced-precision quantization requires an FP32 master tensor")
    master = value.detach()
    if precision == "nvfp4" and master.ndim == 0:
        rounded = _CODECS["nvfp4"].roundtrip(master.reshape(1)).reshape(())
    else:
        rounded = _CODECS[precision].roundtrip(master)
    return _with_identity_gradient(value, rounded)
