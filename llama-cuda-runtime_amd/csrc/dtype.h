// The 16-bit element type, chosen at build time, and its exact conversions.
//
// Like the reference's src/dtype.cuh:24-54, the whole pipeline stores one
// 16-bit type: bf16 by default, fp16 when built with LCR_ELEM_FP16
// (-DLCR_DTYPE=fp16 in the reference). Arithmetic is always fp32. The type is
// a plain 16-bit word here, with conversions written out so host code, device
// code and the CPU oracle agree bit for bit:
//   bf16 -> f32   exact (the bits are the top half of the float)
//   f32  -> bf16  round to nearest even; NaN stays a quiet NaN of the same sign
//   fp16 <-> f32  IEEE conversions with round to nearest even
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.h"

namespace lcr {

struct alignas(2) elem_t {
  uint16_t bits;
};
static_assert(sizeof(elem_t) == 2, "elem_t must be 16 bits");

#if defined(LCR_ELEM_FP16)
constexpr DType kElemDType = DType::kF16;
constexpr const char* kElemName = "fp16";
#else
constexpr DType kElemDType = DType::kBF16;
constexpr const char* kElemName = "bf16";
#endif

__host__ __device__ __forceinline__ float u32_as_f32(uint32_t u) {
  return __builtin_bit_cast(float, u);
}
__host__ __device__ __forceinline__ uint32_t f32_as_u32(float f) {
  return __builtin_bit_cast(uint32_t, f);
}

__host__ __device__ __forceinline__ float bf16_bits_to_float(uint32_t b) {
  return u32_as_f32(b << 16);
}

__host__ __device__ __forceinline__ uint16_t float_to_bf16_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  // The hardware conversion (v_cvt_pk_bf16_f32) gives the integer form's
  // result below for every f32 input, NaN payloads included (an exhaustive
  // comparison of all 2^32 inputs on gfx950).
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
#endif
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// The f32 -> f16 rounding is written with integer operations for the host,
// as the bf16 one is; device code issues the hardware conversion as its own
// instruction (below), which rounds every f32 input the same way. Left to
// the compiler, a plain conversion would be merged with the multiply before
// it into one mixed-precision fma with a +0 addend, which rounds the exact
// product once and turns a -0 product into +0.
// Widening f16 -> f32 is exact, so device code uses the hardware conversion
// (which the compiler may merge into a mixed-precision fma, also exact): the
// same value as the integer form below for every input but a signalling NaN,
// which the hardware returns quieted. Every fp16 weight of a decode step is
// widened once, so this is the fp16 GEMVs' inner loop.
__host__ __device__ __forceinline__ float half_bits_to_float(uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b & 0xffffu)));
#endif
  const uint32_t sign = (b & 0x8000u) << 16;
  const uint32_t exp = (b >> 10) & 0x1fu;
  const uint32_t man = b & 0x3ffu;
  const uint32_t normal = sign | ((exp + 112u) << 23) | (man << 13);
  const uint32_t special = sign | 0x7f800000u | (man << 13);  // inf / nan
  // zero and subnormals: man * 2^-24, exact in float
  const uint32_t small = sign | f32_as_u32(static_cast<float>(man) * 5.9604644775390625e-08f);
  return u32_as_f32(exp == 0x1fu ? special : (exp == 0u ? small : normal));
}

__host__ __device__ __forceinline__ uint16_t float_to_half_bits(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
  // v_cvt_f16_f32 gives the integer form's result below for every f32 input
  // (an exhaustive comparison of all 2^32 inputs on gfx950, NaN payloads
  // included). Inline assembly keeps the compiler from folding a preceding
  // multiply into a mixed-precision fma, which would round the exact product
  // once and turn -0 into +0.
  uint32_t hw;
  asm("v_cvt_f16_f32 %0, %1" : "=v"(hw) : "v"(f));
  return static_cast<uint16_t>(hw & 0xffffu);
#endif
  const uint32_t u = f32_as_u32(f);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  // normal: rebias the exponent, round the 13 dropped mantissa bits to even
  const uint32_t h = (a >> 13) - (112u << 10);
  const uint32_t rem = a & 0x1fffu;
  const uint32_t normal = h + ((rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ? 1u : 0u);
  // below the smallest normal (2^-14): round a * 2^24 (exact scaling) to even;
  // the clamp only keeps the conversion defined for the inputs that take
  // another branch
  const uint32_t small =
      static_cast<uint32_t>(__builtin_rintf(__builtin_fminf(u32_as_f32(a) * 16777216.0f, 2048.0f)));
  const uint32_t mag = a > 0x7f800000u   ? 0x7e00u | ((a >> 13) & 0x3ffu)  // quiet nan
                       : a >= 0x477ff000u ? 0x7c00u                         // rounds to inf
                       : a < 0x38800000u  ? small
                                          : normal;
  return static_cast<uint16_t>(sign | mag);
}

#if defined(LCR_ELEM_FP16)
__host__ __device__ __forceinline__ float elem_bits_to_float(uint32_t b) {
  return half_bits_to_float(b & 0xffffu);
}
__host__ __device__ __forceinline__ uint16_t float_to_elem_bits(float f) {
  return float_to_half_bits(f);
}
#else
__host__ __device__ __forceinline__ float elem_bits_to_float(uint32_t b) {
  return bf16_bits_to_float(b & 0xffffu);
}
__host__ __device__ __forceinline__ uint16_t float_to_elem_bits(float f) {
  return float_to_bf16_bits(f);
}
#endif

__host__ __device__ __forceinline__ float elem_to_float(elem_t x) {
  return elem_bits_to_float(x.bits);
}
__host__ __device__ __forceinline__ elem_t float_to_elem(float v) {
  return elem_t{float_to_elem_bits(v)};
}

}  // namespace lcr
