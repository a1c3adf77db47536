// Streaming elementwise kernels: embedding gather, residual add, SwiGLU (flat
// and row-strided) and the head-major merge. Behaviour follows the reference's
// src/kernels/elementwise.cu:25-143; the arithmetic is restated here:
//   add_residual   x = rne(f(x) + f(delta))
//   swiglu         out = rne(silu(f(g)) * f(u)), silu(v) = v / (1 + exp(-v))
// with exp the shared lcr_expf. Every kernel moves 16-byte chunks (eight
// elements) when the pointers and strides allow, and finishes any remainder one
// element at a time; the launcher picks the vector path only when every pointer
// involved is 16-byte aligned.
#include <algorithm>
#include <cstdint>

#include "../capi_util.h"
#include "device_common.h"

namespace lcr {
namespace {

constexpr int kBlock = 256;

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int grid_for(int64_t work_items) {
  const int64_t blocks = (work_items + kBlock - 1) / kBlock;
  return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(blocks, 8192)));
}

__device__ __forceinline__ float silu(float v) { return lcr_silu(v); }

template <bool kVec>
__global__ __launch_bounds__(kBlock) void embedding_kernel(elem_t* __restrict__ out,
                                                           const elem_t* __restrict__ table,
                                                           const int32_t* __restrict__ ids,
                                                           int dim) {
  const int64_t src = static_cast<int64_t>(ids[blockIdx.x]) * dim;
  const int64_t dst = static_cast<int64_t>(blockIdx.x) * dim;
  int done = 0;
  if (kVec) {
    const int chunks = dim / 8;
    for (int i = threadIdx.x; i < chunks; i += kBlock) {
      store16(out + dst + 8 * i, load16(table + src + 8 * i));
    }
    done = chunks * 8;
  }
  for (int i = done + threadIdx.x; i < dim; i += kBlock) out[dst + i] = table[src + i];
}

template <bool kVec>
__global__ __launch_bounds__(kBlock) void add_residual_kernel(elem_t* __restrict__ x,
                                                              const elem_t* __restrict__ delta,
                                                              int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  int64_t done = 0;
  if (kVec) {
    const int64_t chunks = count / 8;
    for (int64_t i = tid; i < chunks; i += stride) {
      vec16 a = load16(x + 8 * i);
      const vec16 b = load16(delta + 8 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        a.w[j] = pack_elems(elem_lo(a.w[j]) + elem_lo(b.w[j]), elem_hi(a.w[j]) + elem_hi(b.w[j]));
      }
      store16(x + 8 * i, a);
    }
    done = chunks * 8;
  }
  for (int64_t i = done + tid; i < count; i += stride) {
    x[i] = float_to_elem(elem_to_float(x[i]) + elem_to_float(delta[i]));
  }
}

template <bool kVec>
__global__ __launch_bounds__(kBlock) void swiglu_kernel(elem_t* __restrict__ out,
                                                        const elem_t* __restrict__ gate,
                                                        const elem_t* __restrict__ up,
                                                        int64_t count) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kBlock;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  int64_t done = 0;
  if (kVec) {
    const int64_t chunks = count / 8;
    for (int64_t i = tid; i < chunks; i += stride) {
      const vec16 g = load16(gate + 8 * i);
      const vec16 u = load16(up + 8 * i);
      vec16 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r.w[j] = pack_elems(silu(elem_lo(g.w[j])) * elem_lo(u.w[j]),
                            silu(elem_hi(g.w[j])) * elem_hi(u.w[j]));
      }
      store16(out + 8 * i, r);
    }
    done = chunks * 8;
  }
  for (int64_t i = done + tid; i < count; i += stride) {
    out[i] = float_to_elem(silu(elem_to_float(gate[i])) * elem_to_float(up[i]));
  }
}

template <bool kVec>
__global__ __launch_bounds__(kBlock) void swiglu_strided_kernel(elem_t* __restrict__ out,
                                                                const elem_t* __restrict__ gate,
                                                                const elem_t* __restrict__ up,
                                                                int width, int src_row_stride) {
  const int64_t src = static_cast<int64_t>(blockIdx.x) * src_row_stride;
  const int64_t dst = static_cast<int64_t>(blockIdx.x) * width;
  int done = 0;
  if (kVec) {
    const int chunks = width / 8;
    for (int i = threadIdx.x; i < chunks; i += kBlock) {
      const vec16 g = load16(gate + src + 8 * i);
      const vec16 u = load16(up + src + 8 * i);
      vec16 r;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        r.w[j] = pack_elems(silu(elem_lo(g.w[j])) * elem_lo(u.w[j]),
                            silu(elem_hi(g.w[j])) * elem_hi(u.w[j]));
      }
      store16(out + dst + 8 * i, r);
    }
    done = chunks * 8;
  }
  for (int i = done + threadIdx.x; i < width; i += kBlock) {
    out[dst + i] = float_to_elem(silu(elem_to_float(gate[src + i])) * elem_to_float(up[src + i]));
  }
}

// heads[h][t][d] -> out[t][h * head_dim + d]
__global__ void merge_heads_kernel(elem_t* __restrict__ out, const elem_t* __restrict__ heads,
                                   int tokens, int num_heads, int head_dim) {
  const int t = blockIdx.x;
  const int h = blockIdx.y;
  const int64_t src = (static_cast<int64_t>(h) * tokens + t) * head_dim;
  const int64_t dst = static_cast<int64_t>(t) * num_heads * head_dim + static_cast<int64_t>(h) * head_dim;
  for (int i = threadIdx.x; i < head_dim; i += blockDim.x) out[dst + i] = heads[src + i];
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_embedding_lookup(void* out, const void* table, const int32_t* ids,
                                    int tokens, int dim, void* stream) {
  CAPI_CHECK(tokens >= 0 && dim >= 0, "embedding lookup needs non-negative sizes");
  if (tokens == 0 || dim == 0) return LCR_OK;
  const bool vec = aligned16(out) && aligned16(table) && dim % 8 == 0;
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* t = static_cast<const elem_t*>(table);
  if (vec) {
    embedding_kernel<true><<<tokens, kBlock, 0, s>>>(o, t, ids, dim);
  } else {
    embedding_kernel<false><<<tokens, kBlock, 0, s>>>(o, t, ids, dim);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_add_residual(void* x, const void* delta, int64_t count, void* stream) {
  CAPI_CHECK(count >= 0, "residual add needs a non-negative count");
  if (count == 0) return LCR_OK;
  auto s = static_cast<hipStream_t>(stream);
  auto* xp = static_cast<elem_t*>(x);
  auto* dp = static_cast<const elem_t*>(delta);
  if (aligned16(x) && aligned16(delta)) {
    add_residual_kernel<true><<<grid_for(count / 8 + 1), kBlock, 0, s>>>(xp, dp, count);
  } else {
    add_residual_kernel<false><<<grid_for(count), kBlock, 0, s>>>(xp, dp, count);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_swiglu(void* out, const void* gate, const void* up, int64_t count,
                          void* stream) {
  CAPI_CHECK(count >= 0, "swiglu needs a non-negative count");
  if (count == 0) return LCR_OK;
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* g = static_cast<const elem_t*>(gate);
  auto* u = static_cast<const elem_t*>(up);
  if (aligned16(out) && aligned16(gate) && aligned16(up)) {
    swiglu_kernel<true><<<grid_for(count / 8 + 1), kBlock, 0, s>>>(o, g, u, count);
  } else {
    swiglu_kernel<false><<<grid_for(count), kBlock, 0, s>>>(o, g, u, count);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_swiglu_strided(void* out, const void* gate, const void* up, int tokens,
                                  int width, int src_row_stride, void* stream) {
  CAPI_CHECK(tokens >= 0 && width >= 0, "swiglu needs non-negative sizes");
  if (tokens == 0 || width == 0) return LCR_OK;
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* g = static_cast<const elem_t*>(gate);
  auto* u = static_cast<const elem_t*>(up);
  const bool vec = aligned16(out) && aligned16(gate) && aligned16(up) && width % 8 == 0 &&
                   src_row_stride % 8 == 0;
  if (vec) {
    swiglu_strided_kernel<true><<<tokens, kBlock, 0, s>>>(o, g, u, width, src_row_stride);
  } else {
    swiglu_strided_kernel<false><<<tokens, kBlock, 0, s>>>(o, g, u, width, src_row_stride);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_merge_heads(void* out, const void* heads, int tokens, int num_heads,
                               int head_dim, void* stream) {
  CAPI_CHECK(tokens >= 0 && num_heads >= 0 && head_dim >= 0, "merge_heads needs non-negative sizes");
  if (tokens == 0 || num_heads == 0 || head_dim == 0) return LCR_OK;
  const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(num_heads));
  const int block = std::min(kBlock, ((head_dim + 63) / 64) * 64);
  merge_heads_kernel<<<grid, block, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<elem_t*>(out), static_cast<const elem_t*>(heads), tokens, num_heads, head_dim);
  CAPI_LAUNCHED();
  return LCR_OK;
}
