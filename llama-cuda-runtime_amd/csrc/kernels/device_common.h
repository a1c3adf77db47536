// Device-side building blocks shared by every kernel: 16-byte vector access,
// element unpacking, wavefront reductions, and the two transcendental
// functions the token loop needs (exp and sincos).
//
// exp and sincos are written out as fixed sequences of IEEE operations rather
// than taken from a math library, so the CPU oracle can evaluate the very same
// sequence and agree with the GPU bit for bit. Every multiply-add that is meant
// to be fused is an explicit fma; the sources are compiled with
// -ffp-contract=off so nothing else is fused behind the code's back.
//
//   lcr_expf: Cody-Waite reduction x = k*ln2 + r with ln2 split in two parts
//     (the high part has 15 significant bits, so k*ln2_hi is exact), then the
//     degree-7 Taylor polynomial of exp(r) in Horner form, then ldexp by k.
//     |r| <= ~0.35 keeps the truncation error near 5e-9 relative. Inputs below
//     -87 return 0 (the result would be under FLT_MIN), above 88.72283 return
//     +inf. NaN propagates.
//   lcr_sincosf: the float angle is widened to double, reduced by k*pi/2 with
//     fdlibm's two-part pi/2 (the 33-bit leading part makes k*pio2_1 exact for
//     |k| < 2^20), sin and cos of the remainder come from their Maclaurin
//     series to degree 17/18, the quadrant picks signs, and the results are
//     rounded to float once.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cstdint>

#include "../dtype.h"

namespace lcr {

struct alignas(16) vec16 {
  uint32_t w[4];
};

// Identity of the online-softmax accumulator (the reference's
// src/kernels/reduce.cuh:15): finite, so two empty partials combine to zero
// weight instead of NaN.
constexpr float kSoftmaxIdentity = -FLT_MAX;

__device__ __forceinline__ vec16 load16(const void* p) {
  return *reinterpret_cast<const vec16*>(p);
}
__device__ __forceinline__ void store16(void* p, const vec16& v) {
  *reinterpret_cast<vec16*>(p) = v;
}
// A 16-byte load marked non-temporal, for data streamed once (the decode
// GEMVs' weights): it does not displace cached lines. The value is that of
// load16.
__device__ __forceinline__ vec16 load16_stream(const void* p) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return vec16{{v.x, v.y, v.z, v.w}};
}

// Makes a loaded value live here. A load whose only use is in a branch at the
// end of a kernel is otherwise moved into that branch, after the loads it
// was meant to overlap, and costs a whole memory round trip of its own there.
// Called after the loads issued behind it, it waits only for them to arrive.
__device__ __forceinline__ void hold_value(float v) { asm volatile("" : : "v"(v)); }

// Direct global-to-LDS load (global_load_lds_dwordx4): lane L's 16 bytes from
// `src` land at LDS byte address `lds_address` + 16 L (lds_address is the
// wave's base, uniform across the wave). The load counts in the wave's
// vector-memory counter like any other and leaves no registers busy; the
// compiler does not see it as an LDS write, so a reader waits for it by hand
// (vmcnt) and every read of the target is ordered after it by the memory
// clobber.
__device__ __forceinline__ void load_to_lds16(const void* src, uint32_t lds_address) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds_address) : "memory");
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_address_of(const void* p) {
  typedef const __attribute__((address_space(3))) char* lds_char_ptr;
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_char_ptr)p));
}

// The two elements packed in one 32-bit word (element 2i in the low half).
__device__ __forceinline__ float elem_lo(uint32_t p) {
#if defined(LCR_ELEM_FP16)
  return half_bits_to_float(p & 0xffffu);
#else
  return u32_as_f32(p << 16);
#endif
}
__device__ __forceinline__ float elem_hi(uint32_t p) {
#if defined(LCR_ELEM_FP16)
  return half_bits_to_float(p >> 16);
#else
  return u32_as_f32(p & 0xffff0000u);
#endif
}
__device__ __forceinline__ uint32_t pack_elems(float lo, float hi) {
#if defined(LCR_ELEM_FP16)
  return static_cast<uint32_t>(float_to_elem_bits(lo)) |
         (static_cast<uint32_t>(float_to_elem_bits(hi)) << 16);
#else
  // one v_cvt_pk_bf16_f32 for the pair: per element the rounding of
  // float_to_elem_bits
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
#endif
}

// Half-split RoPE of one pair by the angle's (cos, sin): (lo c - hi s,
// hi c + lo s), separate products and a subtract / add.
__device__ __forceinline__ float2 rope_rotate(float lo, float hi, float2 cs) {
  return make_float2(lo * cs.x - hi * cs.y, hi * cs.x + lo * cs.y);
}

// Eight elements of a 16-byte chunk, widened to float, in memory order.
__device__ __forceinline__ void unpack8(const vec16& v, float* out) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    out[2 * i] = elem_lo(v.w[i]);
    out[2 * i + 1] = elem_hi(v.w[i]);
  }
}

__host__ __device__ __forceinline__ float lcr_expf(float in) {
  // The polynomial runs on the input clamped into its range and the special
  // cases are selected afterwards, so a wavefront never diverges here; inside
  // the range the clamp is the identity and the value is the same.
  const float x = __builtin_fminf(__builtin_fmaxf(in, -87.0f), 88.72283f);
  const float k = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(k, -0.693145751953125f, x);
  r = __builtin_fmaf(k, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698413e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float y = __builtin_ldexpf(p, static_cast<int>(k));
  const float special = in < -87.0f ? 0.0f : __builtin_huge_valf();
  const bool in_range = in >= -87.0f && in <= 88.72283f;
  return in != in ? in : (in_range ? y : special);
}

// silu(v) = v / (1 + exp(-v)) with the shared exp, the activation of SwiGLU.
__host__ __device__ __forceinline__ float lcr_silu(float v) { return v / (1.0f + lcr_expf(-v)); }

__host__ __device__ __forceinline__ void lcr_sincosf(float angle, float* s_out, float* c_out) {
  const double x = static_cast<double>(angle);
  const double k = __builtin_rint(x * 6.36619772367581382433e-01);
  double r = __builtin_fma(-k, 1.57079632673412561417e+00, x);
  r = __builtin_fma(-k, 6.07710050650619224932e-11, r);
  const double r2 = r * r;
  double sp = 2.81145725434552076320e-15;
  sp = __builtin_fma(sp, r2, -7.64716373181981647590e-13);
  sp = __builtin_fma(sp, r2, 1.60590438368216145994e-10);
  sp = __builtin_fma(sp, r2, -2.50521083854417187751e-08);
  sp = __builtin_fma(sp, r2, 2.75573192239858906526e-06);
  sp = __builtin_fma(sp, r2, -1.98412698412698412698e-04);
  sp = __builtin_fma(sp, r2, 8.33333333333333333333e-03);
  sp = __builtin_fma(sp, r2, -1.66666666666666666667e-01);
  const double sin_r = __builtin_fma(r * r2, sp, r);
  double cp = -1.56192069685862264622e-16;
  cp = __builtin_fma(cp, r2, 4.77947733238738529744e-14);
  cp = __builtin_fma(cp, r2, -1.14707455977297247139e-11);
  cp = __builtin_fma(cp, r2, 2.08767569878680989792e-09);
  cp = __builtin_fma(cp, r2, -2.75573192239858906526e-07);
  cp = __builtin_fma(cp, r2, 2.48015873015873015873e-05);
  cp = __builtin_fma(cp, r2, -1.38888888888888888889e-03);
  cp = __builtin_fma(cp, r2, 4.16666666666666666667e-02);
  cp = __builtin_fma(cp, r2, -0.5);
  const double cos_r = __builtin_fma(r2, cp, 1.0);
  const int quadrant = static_cast<int>(static_cast<long long>(k) & 3);
  double s, c;
  switch (quadrant) {
    case 0: s = sin_r; c = cos_r; break;
    case 1: s = cos_r; c = -sin_r; break;
    case 2: s = -sin_r; c = -cos_r; break;
    default: s = -cos_r; c = sin_r; break;
  }
  *s_out = static_cast<float>(s);
  *c_out = static_cast<float>(c);
}

// The 32 bits of lane (lane ^ kMask), for a compile-time mask. Lane exchanges
// only move bits, so which hardware path carries them cannot change a result.
// All run in the VALU, without the LDS round trip of ds_bpermute or
// ds_swizzle (lane layouts checked on gfx950 with an in-bounds probe):
//  - 1 and 2: DPP quad permutes;
//  - 4: DPP row_half_mirror (lane i of each 8 reads lane 7 - i), then the
//    quad permute [3, 2, 1, 0] (lane j reads lane 3 - j of its quad): lane i
//    ends with lane i ^ 4;
//  - 8: DPP row_ror:8 within each row of 16;
//  - 16: v_permlane16_swap of the value with itself returns rows (0, 0, 2, 2)
//    and rows (1, 1, 3, 3); a lane of row 1 or 3 takes the first, of row 0
//    or 2 the second;
//  - 32: v_permlane32_swap the same with halves: the upper half takes the
//    lower half's values and the lower half the upper's.
// The lane's index within its wave, from the hardware (any block shape).
__device__ __forceinline__ unsigned hw_lane() {
  return __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
}

template <int kMask>
__device__ __forceinline__ int xor_lane_bits(int x) {
  static_assert(kMask == 1 || kMask == 2 || kMask == 4 || kMask == 8 || kMask == 16 || kMask == 32,
                "a lane distance of one wave64 butterfly step");
  if constexpr (kMask == 1) {
    return __builtin_amdgcn_update_dpp(0, x, 0xB1, 0xF, 0xF, true);   // quad_perm [1,0,3,2]
  } else if constexpr (kMask == 2) {
    return __builtin_amdgcn_update_dpp(0, x, 0x4E, 0xF, 0xF, true);   // quad_perm [2,3,0,1]
  } else if constexpr (kMask == 4) {
    const int mirrored = __builtin_amdgcn_update_dpp(0, x, 0x141, 0xF, 0xF, true);  // row_half_mirror
    return __builtin_amdgcn_update_dpp(0, mirrored, 0x1B, 0xF, 0xF, true);          // quad_perm [3,2,1,0]
  } else if constexpr (kMask == 8) {
    return __builtin_amdgcn_update_dpp(0, x, 0x128, 0xF, 0xF, true);  // row_ror:8
  } else if constexpr (kMask == 16) {
    const auto rows = __builtin_amdgcn_permlane16_swap(static_cast<unsigned>(x), static_cast<unsigned>(x), false,
                                                       false);
    return static_cast<int>((hw_lane() & 16u) ? rows[0] : rows[1]);
  } else {
    const auto halves = __builtin_amdgcn_permlane32_swap(static_cast<unsigned>(x), static_cast<unsigned>(x), false,
                                                         false);
    return static_cast<int>((hw_lane() & 32u) ? halves[0] : halves[1]);
  }
}

template <int kMask>
__device__ __forceinline__ float xor_lane(float v) {
  return __builtin_bit_cast(float, xor_lane_bits<kMask>(__builtin_bit_cast(int, v)));
}

// Butterfly over the 64 lanes of a wavefront, offsets 32, 16, 8, 4, 2, 1.
// Lane i adds lane i^o at each step; addition commutes, so every lane ends
// with the same bits.
__device__ __forceinline__ float wave_sum(float v) {
  v += xor_lane<32>(v);
  v += xor_lane<16>(v);
  v += xor_lane<8>(v);
  v += xor_lane<4>(v);
  v += xor_lane<2>(v);
  v += xor_lane<1>(v);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, xor_lane<32>(v));
  v = fmaxf(v, xor_lane<16>(v));
  v = fmaxf(v, xor_lane<8>(v));
  v = fmaxf(v, xor_lane<4>(v));
  v = fmaxf(v, xor_lane<2>(v));
  v = fmaxf(v, xor_lane<1>(v));
  return v;
}
// The same butterfly restricted to aligned groups of 32 lanes (offsets 16..1).
__device__ __forceinline__ float half_wave_sum(float v) {
  v += xor_lane<16>(v);
  v += xor_lane<8>(v);
  v += xor_lane<4>(v);
  v += xor_lane<2>(v);
  v += xor_lane<1>(v);
  return v;
}

__device__ __forceinline__ int lane_id() { return static_cast<int>(threadIdx.x & 63u); }

}  // namespace lcr
