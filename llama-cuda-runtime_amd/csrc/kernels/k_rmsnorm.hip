// RMSNorm and the fused residual-add + RMSNorm (the reference's
// src/kernels/rmsnorm.cu:21-119), one 256-thread block per token row.
//
//   rmsnorm:              out = rne((f(x) * scale) * f(w)),
//                         scale = 1 / sqrt(sum(f(x)^2) / dim + eps)
//   add_residual_rmsnorm: v = f(x) + f(delta);  x = rne(v);
//                         scale from sum(v^2) over the UNROUNDED v;
//                         out = rne((f(x) * scale) * f(w))
//
// The row is staged in LDS as fp32 so it is read from memory once; the sum of
// squares uses the fixed order of block_sum_squares.
#include <cstdint>

#include "../capi_util.h"
#include "row_norm.h"

namespace lcr {
namespace {

constexpr int kLdsRowLimit = 12288;  // floats of staged row (48 KiB of LDS)

template <bool kResidual, bool kStaged>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(elem_t* __restrict__ out,
                                                               elem_t* __restrict__ x,
                                                               const elem_t* __restrict__ delta,
                                                               const elem_t* __restrict__ weight,
                                                               int dim, float eps) {
  extern __shared__ float row[];
  __shared__ float scratch[9];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
  elem_t* xr = x + base;
  const elem_t* dr = kResidual ? delta + base : nullptr;
  elem_t* orow = out + base;

  auto value = [&](int i) -> float {
    if (kResidual) return elem_to_float(xr[i]) + elem_to_float(dr[i]);
    return elem_to_float(xr[i]);
  };

  float total;
  if (kStaged) {
    for (int i = threadIdx.x; i < dim; i += kNormThreads) {
      const float v = value(i);
      row[i] = v;
      if (kResidual) xr[i] = float_to_elem(v);
    }
    __syncthreads();
    total = block_sum_squares([&](int i) { return row[i]; }, dim, scratch);
  } else {
    // Too wide for LDS: the row is read again for the output, and the residual
    // write waits until every thread has done so.
    total = block_sum_squares(value, dim, scratch);
  }
  const float scale = norm_scale(total, dim, eps);
  for (int i = threadIdx.x; i < dim; i += kNormThreads) {
    float xv;
    if (kStaged) {
      xv = elem_to_float(float_to_elem(row[i]));
    } else {
      const float v = value(i);
      xv = elem_to_float(float_to_elem(v));
    }
    orow[i] = float_to_elem((xv * scale) * elem_to_float(weight[i]));
  }
  if (!kStaged && kResidual) {
    __syncthreads();
    for (int i = threadIdx.x; i < dim; i += kNormThreads) xr[i] = float_to_elem(value(i));
  }
}

// The same arithmetic with 16-byte accesses and the row in registers
// (norm_row_vec), for rows of dim = 8 * chunks elements with at most kChunks
// chunks per thread: bit for bit the kernel above.
template <bool kResidual, int kChunks>
__global__ __launch_bounds__(kNormThreads) void rmsnorm_vec_kernel(elem_t* __restrict__ out,
                                                                   elem_t* __restrict__ x,
                                                                   const elem_t* __restrict__ delta,
                                                                   const elem_t* __restrict__ weight,
                                                                   int dim, float eps) {
  __shared__ float scratch[9];
  const int64_t base = static_cast<int64_t>(blockIdx.x) * dim;
  norm_row_vec<kResidual, kChunks>(
      out + base, x + base, weight, dim, eps,
      [&](int c, float* df) { unpack8(load16(delta + base + 8 * c), df); }, scratch);
}

}  // namespace
}  // namespace lcr

using namespace lcr;

namespace {

int launch_norm(bool residual, void* out, void* x, const void* delta, const void* weight,
                int tokens, int dim, float eps, void* stream) {
  CAPI_CHECK(tokens >= 0 && dim >= 0, "rmsnorm needs non-negative sizes");
  if (tokens == 0 || dim == 0) return LCR_OK;
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* xp = static_cast<elem_t*>(x);
  auto* d = static_cast<const elem_t*>(delta);
  auto* w = static_cast<const elem_t*>(weight);
  const bool vec = dim % 8 == 0 && dim <= 4 * 8 * kNormThreads &&
                   ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(x) |
                     reinterpret_cast<uintptr_t>(delta) | reinterpret_cast<uintptr_t>(weight)) & 15u) == 0;
  if (vec) {
    const int per = (dim / 8 + kNormThreads - 1) / kNormThreads;  // chunks per thread, 1..4
#define LCR_NORM_VEC(R, C) rmsnorm_vec_kernel<R, C><<<tokens, kNormThreads, 0, s>>>(o, xp, d, w, dim, eps)
    if (residual) {
      if (per == 1) LCR_NORM_VEC(true, 1); else if (per == 2) LCR_NORM_VEC(true, 2); else LCR_NORM_VEC(true, 4);
    } else {
      if (per == 1) LCR_NORM_VEC(false, 1); else if (per == 2) LCR_NORM_VEC(false, 2); else LCR_NORM_VEC(false, 4);
    }
#undef LCR_NORM_VEC
    CAPI_LAUNCHED();
    return LCR_OK;
  }
  const bool staged = dim <= kLdsRowLimit;
  const size_t lds = staged ? static_cast<size_t>(dim) * sizeof(float) : sizeof(float);
  if (residual) {
    if (staged) {
      rmsnorm_kernel<true, true><<<tokens, kNormThreads, lds, s>>>(o, xp, d, w, dim, eps);
    } else {
      rmsnorm_kernel<true, false><<<tokens, kNormThreads, lds, s>>>(o, xp, d, w, dim, eps);
    }
  } else {
    if (staged) {
      rmsnorm_kernel<false, true><<<tokens, kNormThreads, lds, s>>>(o, xp, d, w, dim, eps);
    } else {
      rmsnorm_kernel<false, false><<<tokens, kNormThreads, lds, s>>>(o, xp, d, w, dim, eps);
    }
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

}  // namespace

extern "C" int lcr_rmsnorm(void* out, const void* x, const void* weight, int tokens, int dim,
                           float eps, void* stream) {
  return launch_norm(false, out, const_cast<void*>(x), nullptr, weight, tokens, dim, eps, stream);
}

extern "C" int lcr_add_residual_rmsnorm(void* out, void* x, const void* delta, const void* weight,
                                        int tokens, int dim, float eps, void* stream) {
  return launch_norm(true, out, x, delta, weight, tokens, dim, eps, stream);
}
