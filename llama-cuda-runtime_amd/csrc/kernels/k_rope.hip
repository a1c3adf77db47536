// Rotary position embedding (the reference's src/kernels/rope.cu:33-87).
//
// Llama pairs element i of a head with element i + head_dim/2 (half-split, not
// interleaved). For angle a = float(position) * inv_freq[i] (one fp32 multiply):
//   out[i]        = lo * cos(a) - hi * sin(a)
//   out[i + half] = hi * cos(a) + lo * sin(a)
// computed as separate multiplies and a subtract/add (no fusion), with
// sin/cos from lcr_sincosf, evaluated once per (token, i) and shared by every
// head of the token. The query kernel writes the head-major
// [num_heads][tokens][head_dim] layout; the key kernel writes K (rotated) and V
// (copied) straight into the cache at KvCacheView::offset.
#include <algorithm>

#include "../capi_util.h"
#include "../kv_cache.h"
#include "device_common.h"
#include "fill.h"

namespace lcr {
namespace {

constexpr int kRopeThreads = 256;
constexpr int kMaxRopeHalf = 256;  // head_dim up to 512

// One block per token: the head_dim/2 angles of the token's position are
// evaluated once into LDS (cos, sin), then every head's pairs are rotated.
__device__ __forceinline__ void token_angles(float2* cs, const float* inv_freq, int position, int half) {
  for (int i = threadIdx.x; i < half; i += kRopeThreads) {
    float s, c;
    lcr_sincosf(static_cast<float>(position) * inv_freq[i], &s, &c);
    cs[i] = make_float2(c, s);
  }
  __syncthreads();
}

__device__ __forceinline__ void rotate(float lo, float hi, float2 cs, float* out_lo, float* out_hi) {
  const float2 r = rope_rotate(lo, hi, cs);
  *out_lo = r.x;
  *out_hi = r.y;
}

__global__ __launch_bounds__(kRopeThreads) void rope_q_kernel(elem_t* __restrict__ q_heads,
                                                             const elem_t* __restrict__ q_proj,
                                                             const float* __restrict__ inv_freq,
                                                             int tokens, int start_position, int num_heads,
                                                             int head_dim, int src_row_stride) {
  __shared__ float2 cs[kMaxRopeHalf];
  const int t = blockIdx.x;
  const int half = head_dim / 2;
  token_angles(cs, inv_freq, start_position + t, half);
  const int64_t src = static_cast<int64_t>(t) * src_row_stride;
  for (int idx = threadIdx.x; idx < num_heads * half; idx += kRopeThreads) {
    const int h = idx / half;
    const int i = idx - h * half;
    const int64_t s = src + static_cast<int64_t>(h) * head_dim + i;
    const int64_t dst = (static_cast<int64_t>(h) * tokens + t) * head_dim + i;
    float a, b;
    rotate(elem_to_float(q_proj[s]), elem_to_float(q_proj[s + half]), cs[i], &a, &b);
    q_heads[dst] = float_to_elem(a);
    q_heads[dst + half] = float_to_elem(b);
  }
}

template <bool kPaged>
__global__ __launch_bounds__(kRopeThreads) void rope_write_kv_kernel(KvCacheView view,
                                                                    const elem_t* __restrict__ k_proj,
                                                                    const elem_t* __restrict__ v_proj,
                                                                    const float* __restrict__ inv_freq,
                                                                    int start_position, int src_row_stride) {
  __shared__ float2 cs[kMaxRopeHalf];
  const int t = blockIdx.x;
  const int head_dim = view.head_dim;
  const int half = head_dim / 2;
  const int position = start_position + t;
  token_angles(cs, inv_freq, position, half);
  const int64_t src = static_cast<int64_t>(t) * src_row_stride;
  for (int idx = threadIdx.x; idx < view.num_kv_heads * half; idx += kRopeThreads) {
    const int h = idx / half;
    const int i = idx - h * half;
    const int64_t s = src + static_cast<int64_t>(h) * head_dim + i;
    const size_t dst = view.offset<kPaged>(h, position) + i;
    float a, b;
    rotate(elem_to_float(k_proj[s]), elem_to_float(k_proj[s + half]), cs[i], &a, &b);
    view.keys[dst] = float_to_elem(a);
    view.keys[dst + half] = float_to_elem(b);
  }
  for (int idx = threadIdx.x; idx < view.num_kv_heads * head_dim; idx += kRopeThreads) {
    const int h = idx / head_dim;
    const int i = idx - h * head_dim;
    view.values[view.offset<kPaged>(h, position) + i] = v_proj[src + static_cast<int64_t>(h) * head_dim + i];
  }
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_rope_q(void* q_heads, const void* q_proj, const float* inv_freq, int tokens,
                          int start_position, int num_heads, int head_dim, int src_row_stride,
                          void* stream) {
  CAPI_CHECK(tokens >= 0 && num_heads >= 0, "rope_q needs non-negative sizes");
  if (tokens == 0 || num_heads == 0) return LCR_OK;
  CAPI_CHECK(head_dim > 0 && head_dim % 2 == 0,
             "head_dim must be positive and even for RoPE, got " << head_dim);
  CAPI_CHECK(head_dim / 2 <= kMaxRopeHalf, "rope_q supports head_dim up to " << 2 * kMaxRopeHalf);
  rope_q_kernel<<<static_cast<unsigned>(tokens), kRopeThreads, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<elem_t*>(q_heads), static_cast<const elem_t*>(q_proj), inv_freq, tokens,
      start_position, num_heads, head_dim, src_row_stride);
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_rope_write_kv(const lcr_kv_view* view, const void* k_proj, const void* v_proj,
                                 const float* inv_freq, int tokens, int start_position, int paged,
                                 int src_row_stride, void* stream) {
  CAPI_CHECK(view != nullptr, "rope_write_kv needs a cache view");
  CAPI_CHECK(tokens >= 0, "rope_write_kv needs a non-negative token count");
  if (tokens == 0) return LCR_OK;
  const KvCacheView v = KvCacheView::from_c(*view);
  CAPI_CHECK(v.head_dim > 0 && v.head_dim % 2 == 0,
             "head_dim must be positive and even for RoPE, got " << v.head_dim);
  CAPI_CHECK(!paged || v.page_table != nullptr, "a paged cache view needs a page table");
  CAPI_CHECK(v.head_dim / 2 <= kMaxRopeHalf, "rope_write_kv supports head_dim up to " << 2 * kMaxRopeHalf);
  if (v.num_kv_heads == 0) return LCR_OK;
  const unsigned grid = static_cast<unsigned>(tokens);
  const int block = kRopeThreads;
  auto s = static_cast<hipStream_t>(stream);
  auto* k = static_cast<const elem_t*>(k_proj);
  auto* vv = static_cast<const elem_t*>(v_proj);
  if (paged) {
    rope_write_kv_kernel<true><<<grid, block, 0, s>>>(v, k, vv, inv_freq, start_position, src_row_stride);
  } else {
    rope_write_kv_kernel<false><<<grid, block, 0, s>>>(v, k, vv, inv_freq, start_position, src_row_stride);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_rope_table(float* table, const float* inv_freq, int positions, int head_dim, void* stream) {
  CAPI_CHECK(positions >= 0, "rope_table needs a non-negative position count");
  CAPI_CHECK(head_dim > 0 && head_dim % 2 == 0,
             "head_dim must be positive and even for RoPE, got " << head_dim);
  if (positions == 0) return LCR_OK;
  CAPI_CHECK(table != nullptr && inv_freq != nullptr, "rope_table needs a table and inverse frequencies");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(table) & 7u) == 0, "rope_table needs an 8-byte aligned table");
  return capi::guarded([&] {
    build_rope_table(reinterpret_cast<float2*>(table), inv_freq, positions, head_dim / 2,
                     static_cast<hipStream_t>(stream));
    return LCR_OK;
  });
}
