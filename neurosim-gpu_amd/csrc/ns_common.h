// Shared device-side helpers of the gfx950 dendritic tick library.
//
// Operand views, the exact weight decoders and the per-(neuron, column)
// three-state update.  The update follows the operation order of the
// reference's PyTorch path (compartmental.py:168-183, dynamics.py:305-314)
// with floating-point contraction disabled, so given the same synaptic input
// it rounds exactly like the reference's float32 CPU/GPU tensor ops.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "neurosim_hip.h"
#include "ns_limits.h"

namespace ns {

// A [B, N] operand that is either a strided tensor or one scalar.  `data` is
// never null: a scalar plane points at some valid float with zero strides, so
// a read is one unconditional load and a bitwise blend with `scalar` under
// `mask` (all ones for a tensor, zero for a scalar).  A branch on the pointer,
// or on a flag the compiler can see is boolean, would make a kernel wait for
// each plane's kernel arguments before it requests the next plane's.
struct Plane {
  const float* data;
  int64_t sb, sn;
  float scalar;
  uint32_t mask;
  __device__ __forceinline__ float get(int64_t b, int64_t n) const {
    const uint32_t x = __builtin_bit_cast(uint32_t, data[b * sb + n * sn]);
    return __builtin_bit_cast(float, (x & mask) | (__builtin_bit_cast(uint32_t, scalar) & ~mask));
  }
};

struct OutPlane {
  float* data;
  int64_t sb, sn;
  __device__ __forceinline__ void put(int64_t b, int64_t n, float x) const {
    data[b * sb + n * sn] = x;
  }
};

struct Vec {
  const float* data;
  int64_t stride;
  __device__ __forceinline__ float get(int64_t n) const { return data[n * stride]; }
};

struct Params {
  Vec v[6];  // alpha, gain, rho_d, rho_a, coupling, adaptation_strength
};

struct NextState {
  float soma, dendrite, adaptation;
};

// torch.clamp(x, 0, 1) semantics, including NaN propagation.
__device__ __forceinline__ float clamp01(float x) {
  return x < 0.0f ? 0.0f : (x > 1.0f ? 1.0f : x);
}

// A neuron's six parameters, loaded together so their loads can be issued
// before anything that waits on memory.
struct NeuronParams {
  float alpha, gain, rho_d, rho_a, coupling, strength;
};

__device__ __forceinline__ NeuronParams load_params(const Params& p, int64_t n) {
  return NeuronParams{p.v[0].get(n), p.v[1].get(n), p.v[2].get(n),
                      p.v[3].get(n), p.v[4].get(n), p.v[5].get(n)};
}

// One three-state update.  Each statement is one tensor op of the reference:
//   d' = rho_d*d + (1-rho_d)*tanh(j + v)
//   u  = ((1-c)*j + c*d') - k*a
//   s' = clamp(alpha*s + (1-alpha)*(gain*tanh(u + drive)), 0, 1)
//   a' = rho_a*a + (1-rho_a)*s'
__device__ __forceinline__ NextState advance_loaded(const NeuronParams& p, float j, float s,
                                                    float d, float a, float drive, float ddrive) {
#pragma clang fp contract(off)
  NextState out;
  const float dend_in = tanhf(j + ddrive);
  out.dendrite = p.rho_d * d + (1.0f - p.rho_d) * dend_in;
  const float mixed = (1.0f - p.coupling) * j + p.coupling * out.dendrite;
  const float current = mixed - p.strength * a;
  const float equilibrium = p.gain * tanhf(current + drive);
  out.soma = clamp01(p.alpha * s + (1.0f - p.alpha) * equilibrium);
  out.adaptation = p.rho_a * a + (1.0f - p.rho_a) * out.soma;
  return out;
}

__device__ __forceinline__ NextState advance_one(const Params& p, int64_t n, float j, float s,
                                                 float d, float a, float drive, float ddrive) {
  return advance_loaded(load_params(p, n), j, s, d, a, drive, ddrive);
}

// OCP fp8 e4m3fn -> float32, exact (bias 7, subnormals, 0x7F/0xFF NaN): the
// gfx950 conversion instruction, which decodes the OCP format; every one of
// the 256 codes is checked against the oracle's decoder by the GPU tests.
__device__ __forceinline__ float e4m3_to_float(uint32_t code) {
  return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(code), 0);
}

// The signed e2m1 values (0, 0.5, 1, 1.5, 2, 3, 4, 6; bit 3 the sign) of the
// two nibbles of `byte` (low nibble first), via the gfx950 conversion with a
// unit scale, which is exact.
typedef float ns_v2f __attribute__((ext_vector_type(2)));
__device__ __forceinline__ ns_v2f e2m1_pair(uint32_t byte) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(byte, 1.0f, 0);
}

// Decoded weight of an NVFP4 nibble given its block scale already decoded and
// multiplied by the global scale: the signed level times that product, one
// float32 rounding, as in the reference's levels[code & 7] * (block.float() *
// global) with the sign applied after (precision.py:109-110; negation commutes
// with the rounding).
__device__ __forceinline__ float nvfp4_weight(uint32_t nibble, float block_times_global) {
  return e2m1_pair(nibble & 15u).x * block_times_global;
}

}  // namespace ns
