// lcr_gemv: y = W x for one token (the reference's gemm_nt at rows = 1,
// src/model.cu:38-45), bf16/fp16 weights, fp32 accumulation, 16-bit or fp32
// output. One wavefront per R rows; the reduction order is gemv_core.h's.
#include <algorithm>

#include "../capi_util.h"
#include "gemv_core.h"

namespace lcr {
namespace {

constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / 64;

template <bool kFp32Out>
__device__ __forceinline__ void store_y(void* y, int row, float v) {
  if (kFp32Out) {
    static_cast<float*>(y)[row] = v;
  } else {
    static_cast<elem_t*>(y)[row] = float_to_elem(v);
  }
}

template <int R, int NCH, bool kFp32Out>
__global__ __launch_bounds__(kGemvThreads) void gemv_kernel(void* __restrict__ y,
                                                            const elem_t* __restrict__ W,
                                                            const elem_t* __restrict__ x, int N) {
  constexpr int K = NCH * 512;
  const int lane = lane_id();
  const int row0 = (blockIdx.x * kGemvWaves + (threadIdx.x >> 6)) * R;
  if (row0 >= N) return;
  const elem_t* rows[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rows[r] = W + static_cast<size_t>(min(row0 + r, N - 1)) * K;
  GemvTile<R, NCH> tile;
  tile.load(rows, lane);
  vec16 xv[NCH];
#pragma unroll
  for (int c = 0; c < NCH; ++c) xv[c] = load16(x + c * 512 + lane * kGemvChunk);
  float out[R];
  tile.dot(out, xv);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (lane == r && row0 + r < N) store_y<kFp32Out>(y, row0 + r, out[r]);
  }
}

template <bool kFp32Out>
__global__ __launch_bounds__(kGemvThreads) void gemv_generic_kernel(void* __restrict__ y,
                                                                    const elem_t* __restrict__ W,
                                                                    const elem_t* __restrict__ x,
                                                                    int N, int K) {
  const int lane = lane_id();
  const int row = blockIdx.x * kGemvWaves + (threadIdx.x >> 6);
  if (row >= N) return;
  const float v = gemv_row_generic(W + static_cast<size_t>(row) * K, x, K, lane);
  if (lane == 0) store_y<kFp32Out>(y, row, v);
}

template <int R, int NCH, bool kFp32Out>
void launch_fixed(void* y, const elem_t* W, const elem_t* x, int N, hipStream_t s) {
  const int waves = (N + R - 1) / R;
  const int blocks = (waves + kGemvWaves - 1) / kGemvWaves;
  gemv_kernel<R, NCH, kFp32Out><<<blocks, kGemvThreads, 0, s>>>(y, W, x, N);
}

template <bool kFp32Out>
void launch_gemv(void* y, const elem_t* W, const elem_t* x, int N, int K, hipStream_t s) {
  if (K == 2048) {
    if (N <= 4096) {
      launch_fixed<2, 4, kFp32Out>(y, W, x, N, s);
    } else {
      launch_fixed<1, 4, kFp32Out>(y, W, x, N, s);
    }
  } else if (K == 8192) {
    launch_fixed<2, 16, kFp32Out>(y, W, x, N, s);
  } else if (K == 4096) {
    launch_fixed<1, 8, kFp32Out>(y, W, x, N, s);
  } else {
    const int blocks = (N + kGemvWaves - 1) / kGemvWaves;
    gemv_generic_kernel<kFp32Out><<<blocks, kGemvThreads, 0, s>>>(y, W, x, N, K);
  }
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_gemv(void* y, int y_fp32, const void* W, const void* x, int N, int K,
                        void* stream) {
  CAPI_CHECK(N >= 0 && K >= 0, "gemv needs non-negative sizes");
  if (N == 0) return LCR_OK;
  CAPI_CHECK(K > 0 && K % 8 == 0, "gemv needs K to be a positive multiple of 8, got " << K);
  CAPI_CHECK((reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(x) & 15u) == 0,
             "gemv needs 16-byte aligned weights and input");
  auto* w = static_cast<const elem_t*>(W);
  auto* xv = static_cast<const elem_t*>(x);
  auto s = static_cast<hipStream_t>(stream);
  if (y_fp32) {
    launch_gemv<true>(y, w, xv, N, K, s);
  } else {
    launch_gemv<false>(y, w, xv, N, K, s);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}
