// Prefill: the projections as a dense GEMM on MFMA matrix cores, and causal
// GQA attention over the cache.
//
// lcr_gemm computes Y[T][N] = X[T][K] . W[N][K]^T (the reference's gemm_nt at
// rows = T, src/model.cu:38-45, which goes to cublasGemmEx). Both operands are
// K-contiguous, which is the natural operand layout of
// v_mfma_f32_16x16x32_bf16: per lane, 8 consecutive K elements of one row of
// A and one column of B. A 256-thread block owns a 128x128 tile of Y; each
// wave owns 64x64 = 4x4 MFMA tiles; K advances 64 at a time through LDS
// (rows padded by 8 elements to spread the 16-byte reads over the banks).
// fp32 accumulation; the fp32 accumulators are rounded once on store.
//
// lcr_prefill_attention replaces the reference's gather + two strided-batched
// GEMMs + causal softmax (src/model.cu:509-560). Query row r of the chunk sits
// at position start + r and sees keys 0..start+r. Two passes per (row, head):
// the first finds the row maximum M and sum L of exp(s - M), the second forms
// p = rne(exp(s - M) * (1/L)) — the probability rounded to the element type
// exactly where the reference rounds its probs buffer — and accumulates
// p * v in fp32. Scores are fp32 (q . k) * scale.
#include <algorithm>

#include "../capi_util.h"
#include "../kv_cache.h"
#include "device_common.h"

namespace lcr {
namespace {

// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------

constexpr int kTileM = 128;  // rows of X (tokens)
constexpr int kTileN = 128;  // rows of W (output features)
constexpr int kTileK = 64;
constexpr int kPitch = kTileK + 8;  // LDS row pitch in elements
constexpr int kGemmThreads = 256;

#if defined(LCR_ELEM_FP16)
typedef _Float16 mfma_in8 __attribute__((ext_vector_type(8)));
#else
typedef __bf16 mfma_in8 __attribute__((ext_vector_type(8)));
#endif
typedef float mfma_acc4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ mfma_acc4 mfma16x16x32(const mfma_in8& a, const mfma_in8& b,
                                                  const mfma_acc4& c) {
#if defined(LCR_ELEM_FP16)
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
#else
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
#endif
}

template <bool kFp32Out>
__global__ __launch_bounds__(kGemmThreads) void gemm_nt_kernel(void* __restrict__ Y,
                                                               const elem_t* __restrict__ X,
                                                               const elem_t* __restrict__ W,
                                                               int T, int N, int K) {
  __shared__ __attribute__((aligned(16))) elem_t a_tile[kTileM * kPitch];
  __shared__ __attribute__((aligned(16))) elem_t b_tile[kTileN * kPitch];

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int m0 = blockIdx.y * kTileM;
  const int n0 = blockIdx.x * kTileN;
  const int wm = (wave >> 1) * 64;  // wave's row offset inside the tile
  const int wn = (wave & 1) * 64;

  mfma_acc4 acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) acc[i][jj] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }

  for (int k0 = 0; k0 < K; k0 += kTileK) {
    // Stage: 128 rows x 64 elements = 1024 chunks of 8 per operand, 4 per thread.
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int chunk = it * kGemmThreads + tid;
      const int r = chunk >> 3;
      const int c = (chunk & 7) * 8;
      vec16 va{{0u, 0u, 0u, 0u}}, vb{{0u, 0u, 0u, 0u}};
      if (m0 + r < T && k0 + c < K) va = load16(X + static_cast<size_t>(m0 + r) * K + k0 + c);
      if (n0 + r < N && k0 + c < K) vb = load16(W + static_cast<size_t>(n0 + r) * K + k0 + c);
      store16(&a_tile[r * kPitch + c], va);
      store16(&b_tile[r * kPitch + c], vb);
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kTileK; kk += 32) {
      mfma_in8 af[4], bf[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int row = wm + i * 16 + (lane & 15);
        af[i] = *reinterpret_cast<const mfma_in8*>(&a_tile[row * kPitch + kk + (lane >> 4) * 8]);
      }
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int row = wn + jj * 16 + (lane & 15);
        bf[jj] = *reinterpret_cast<const mfma_in8*>(&b_tile[row * kPitch + kk + (lane >> 4) * 8]);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) acc[i][jj] = mfma16x16x32(af[i], bf[jj], acc[i][jj]);
      }
    }
    __syncthreads();
  }

  // Accumulator layout of the 16x16 tile: lane holds rows 4*(lane/16)+v,
  // column lane%16.
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int col = n0 + wn + jj * 16 + (lane & 15);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + wm + i * 16 + (lane >> 4) * 4 + v;
        if (row < T && col < N) {
          if (kFp32Out) {
            static_cast<float*>(Y)[static_cast<size_t>(row) * N + col] = acc[i][jj][v];
          } else {
            static_cast<elem_t*>(Y)[static_cast<size_t>(row) * N + col] = float_to_elem(acc[i][jj][v]);
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Prefill attention
// ---------------------------------------------------------------------------

constexpr int kPrefillThreads = 256;  // one wave per query head of the group (up to 4)

// One block per (query row, kv head); wave g handles query head kv*G + g for
// g < G (G <= 4 per block; larger groups use several blocks along z).
template <bool kPaged>
__global__ __launch_bounds__(kPrefillThreads) void prefill_attention_kernel(
    elem_t* __restrict__ out, const elem_t* __restrict__ q_heads, KvCacheView view, int num_heads,
    int group, int tokens, int start_position, float scale) {
  __shared__ float probs[4][64];
  const int row = blockIdx.x;
  const int kv = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int g = blockIdx.z * 4 + wave;
  if (g >= group) return;  // whole wave exits; no block-wide barrier below
  const int head = kv * group + g;
  const int head_dim = view.head_dim;
  const int limit = start_position + row + 1;

  // q in registers (head_dim <= 128: two floats per lane).
  const elem_t* qrow = q_heads + (static_cast<size_t>(head) * tokens + row) * head_dim;
  float q0 = lane < head_dim ? elem_to_float(qrow[lane]) : 0.0f;
  float q1 = lane + 64 < head_dim ? elem_to_float(qrow[lane + 64]) : 0.0f;

  auto score = [&](int key) -> float {
    const elem_t* k = view.keys + view.offset<kPaged>(kv, key);
    float d = 0.0f;
    d = __builtin_fmaf(q0, lane < head_dim ? elem_to_float(k[lane]) : 0.0f, d);
    d = __builtin_fmaf(q1, lane + 64 < head_dim ? elem_to_float(k[lane + 64]) : 0.0f, d);
    return wave_sum(d) * scale;
  };

  // Pass 1: row max and exponential sum (one key per step, all lanes share it).
  float m = kSoftmaxIdentity;
  for (int key = 0; key < limit; ++key) m = fmaxf(m, score(key));
  float l = 0.0f;
  for (int key = 0; key < limit; ++key) l += lcr_expf(score(key) - m);
  const float inv = 1.0f / l;

  // Pass 2: rounded probabilities times values; lane owns dims lane, lane+64.
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int base = 0; base < limit; base += 64) {
    const int n = min(64, limit - base);
    // Each lane computes one probability of this 64-key slab.
    float mine = 0.0f;
    for (int i = 0; i < n; ++i) {
      const float p = elem_to_float(float_to_elem(lcr_expf(score(base + i) - m) * inv));
      if (lane == i) mine = p;
    }
    probs[wave][lane] = mine;
    __builtin_amdgcn_wave_barrier();
    for (int i = 0; i < n; ++i) {
      const float p = probs[wave][i];
      const elem_t* v = view.values + view.offset<kPaged>(kv, base + i);
      if (lane < head_dim) acc0 = __builtin_fmaf(p, elem_to_float(v[lane]), acc0);
      if (lane + 64 < head_dim) acc1 = __builtin_fmaf(p, elem_to_float(v[lane + 64]), acc1);
    }
    __builtin_amdgcn_wave_barrier();
  }
  elem_t* o = out + static_cast<size_t>(row) * num_heads * head_dim + static_cast<size_t>(head) * head_dim;
  if (lane < head_dim) o[lane] = float_to_elem(acc0);
  if (lane + 64 < head_dim) o[lane + 64] = float_to_elem(acc1);
}

}  // namespace
}  // namespace lcr

using namespace lcr;

extern "C" int lcr_gemm(void* Y, int y_fp32, const void* X, const void* W, int T, int N, int K,
                        void* stream) {
  CAPI_CHECK(T >= 0 && N >= 0 && K >= 0, "gemm needs non-negative sizes");
  if (T == 0 || N == 0) return LCR_OK;
  CAPI_CHECK(K > 0 && K % 8 == 0, "gemm needs K to be a positive multiple of 8, got " << K);
  CAPI_CHECK((reinterpret_cast<uintptr_t>(X) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(W) & 15u) == 0,
             "gemm needs 16-byte aligned operands");
  const dim3 grid(static_cast<unsigned>((N + kTileN - 1) / kTileN),
                  static_cast<unsigned>((T + kTileM - 1) / kTileM));
  auto s = static_cast<hipStream_t>(stream);
  auto* x = static_cast<const elem_t*>(X);
  auto* w = static_cast<const elem_t*>(W);
  if (y_fp32) {
    gemm_nt_kernel<true><<<grid, kGemmThreads, 0, s>>>(Y, x, w, T, N, K);
  } else {
    gemm_nt_kernel<false><<<grid, kGemmThreads, 0, s>>>(Y, x, w, T, N, K);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_prefill_attention(void* out, const void* q_heads, const lcr_kv_view* view,
                                     int num_heads, int heads_per_kv, int tokens,
                                     int start_position, float scale, int paged, void* stream) {
  CAPI_CHECK(view != nullptr, "prefill attention needs a cache view");
  CAPI_CHECK(tokens >= 0 && start_position >= 0, "prefill attention needs non-negative sizes");
  if (tokens == 0 || num_heads == 0) return LCR_OK;
  CAPI_CHECK(view->head_dim > 0 && view->head_dim <= 128,
             "prefill attention supports head_dim up to 128, got " << view->head_dim);
  CAPI_CHECK(heads_per_kv > 0 && num_heads == view->num_kv_heads * heads_per_kv,
             "num_heads (" << num_heads << ") must equal num_kv_heads (" << view->num_kv_heads
                           << ") times heads_per_kv (" << heads_per_kv << ")");
  CAPI_CHECK(!paged || view->page_table != nullptr, "a paged cache view needs a page table");
  const KvCacheView v = KvCacheView::from_c(*view);
  const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(v.num_kv_heads),
                  static_cast<unsigned>((heads_per_kv + 3) / 4));
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* q = static_cast<const elem_t*>(q_heads);
  if (paged) {
    prefill_attention_kernel<true><<<grid, kPrefillThreads, 0, s>>>(o, q, v, num_heads, heads_per_kv,
                                                                     tokens, start_position, scale);
  } else {
    prefill_attention_kernel<false><<<grid, kPrefillThreads, 0, s>>>(o, q, v, num_heads, heads_per_kv,
                                                                      tokens, start_position, scale);
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}
