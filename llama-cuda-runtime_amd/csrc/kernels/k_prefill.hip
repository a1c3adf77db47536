// Prefill: the projections as dense GEMMs on the MFMA matrix cores, and
// causal GQA attention over the cache as a flash-style MFMA kernel.
//
// lcr_gemm computes Y[T][N] = X[T][K] . W[N][K]^T (the reference's gemm_nt at
// rows = T, src/model.cu:38-45, which goes to cublasGemmEx). Both operands are
// K-contiguous, the natural operand layout of v_mfma_f32_16x16x32_{bf16,f16}:
// per lane, 8 consecutive K elements of one row. W rows are the MFMA's M side
// and tokens its N side, so an accumulator holds 4 consecutive output features
// of one token and the epilogue stores them as one 8-byte (16-byte for fp32)
// word. A 256-thread block owns a BW x BT tile (W rows x tokens), each of its
// four waves a (BW/2) x (BT/2) quarter; K advances 64 per stage through two
// LDS buffers, the next stage's global loads in flight while the current one
// feeds the matrix cores, one barrier per stage. Tiles are handed out so that
// the blocks of one XCD (block id mod 8) walk a contiguous run of tiles with
// tokens fastest: they share W panels in that XCD's L2. fp32 accumulation,
// rounded once on store.
//
// lcr_prefill_attention replaces the reference's gather + two strided-batched
// GEMMs + causal softmax (src/model.cu:509-560; src/kernels/attention.cu:42-100).
// Query row r of the chunk sits at position start + r and sees keys
// 0..start+r; scores are (q . k) * scale in fp32. A block takes 16*RF
// positions of the query heads that share one kv head (four per block, one
// wave each) and walks 64-key tiles of that kv head staged in LDS (double
// buffered). Each wave computes S^T = K . Q^T, so an accumulator lane holds
// one query row and 4 keys: a row statistic needs two lane exchanges, and the
// probabilities are already in the operand layout of O^T = V^T . P^T (V is
// staged transposed). The softmax follows the reference's rounding points: a
// first pass over the keys finds each row's max M and sum L of exp(s - M),
// the second forms p = exp(s - M) * (1/L), rounds it to the element type (the
// reference's probability buffer) and accumulates p * v in fp32, rounded once
// on store.
#include <algorithm>

#include "../capi_util.h"
#include "../kv_cache.h"
#include "device_common.h"

namespace lcr {
namespace {

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

__device__ __forceinline__ mfma_in8 as_operand(const vec16& v) {
  return __builtin_bit_cast(mfma_in8, v);
}
__device__ __forceinline__ mfma_in8 lds_operand(const elem_t* p) {
  return *reinterpret_cast<const mfma_in8*>(p);
}

int device_compute_units() {
  static int cached[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    cached[dev] = cus;
  }
  return cached[dev];
}

// ---------------------------------------------------------------------------
// MFMA GEMM
// ---------------------------------------------------------------------------

constexpr int kStageK = 64;
constexpr int kGemmPitch = kStageK + 8;  // LDS row pitch in elements: fragment reads hit 64 banks once

// Block tile BW x BT (W rows x tokens) over kWavesW x kWavesT waves; each
// wave owns a (BW / kWavesW) x (BT / kWavesT) piece.
template <int BW, int BT, int kWavesW, int kWavesT, bool kFp32Out>
__global__ __launch_bounds__(64 * kWavesW * kWavesT) void gemm_nt_kernel(
    void* __restrict__ Y, const elem_t* __restrict__ X, const elem_t* __restrict__ W, int T, int N,
    int K, int tiles_t, int total_tiles) {
  constexpr int kThreads = 64 * kWavesW * kWavesT;
  constexpr int kWaveW = BW / kWavesW, kWaveT = BT / kWavesT;
  constexpr int FW = kWaveW / 16, FT = kWaveT / 16;
  constexpr int kRowsPerPass = kThreads / 8;  // rows one pass of 16-byte chunks covers
  constexpr int kPerW = BW / kRowsPerPass, kPerT = BT / kRowsPerPass;
  static_assert(BW % kRowsPerPass == 0 && BT % kRowsPerPass == 0, "stage must split evenly");
  __shared__ __attribute__((aligned(16))) elem_t stage[2][(BW + BT) * kGemmPitch];

  // XCD-aware tile order: XCD x (block id mod 8) takes tiles [x*per, (x+1)*per).
  const int per_xcd = (total_tiles + 7) / 8;
  const int tile = static_cast<int>(blockIdx.x % 8u) * per_xcd + static_cast<int>(blockIdx.x / 8u);
  if (tile >= total_tiles) return;
  const int w0 = (tile / tiles_t) * BW;
  const int t0 = (tile % tiles_t) * BT;

  const int tid = threadIdx.x;
  const int lane = lane_id();
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int ww = (wave / kWavesT) * kWaveW;
  const int wt = (wave % kWavesT) * kWaveT;

  // Chunk c of a thread covers row kRowsPerPass*c + tid/8 of its operand,
  // elements 8*(tid%8) .. +7 of the stage. Rows past the end read a valid
  // row and are zeroed, so the loads carry no branches.
  const int trow = tid >> 3;
  const int kc = (tid & 7) * 8;
  const elem_t* wsrc[kPerW];
  const elem_t* xsrc[kPerT];
  uint32_t live = 0;
#pragma unroll
  for (int c = 0; c < kPerW; ++c) {
    const int row = w0 + kRowsPerPass * c + trow;
    live |= (row < N ? 1u : 0u) << c;
    wsrc[c] = W + static_cast<size_t>(min(row, N - 1)) * K + kc;
  }
#pragma unroll
  for (int c = 0; c < kPerT; ++c) {
    const int row = t0 + kRowsPerPass * c + trow;
    live |= (row < T ? 1u : 0u) << (kPerW + c);
    xsrc[c] = X + static_cast<size_t>(min(row, T - 1)) * K + kc;
  }
  // The loads of a stage are issued a stage ahead; the zeroing select waits
  // until the data is written to LDS, so nothing waits on the loads before
  // the matrix work of the current stage.
  vec16 held[kPerW + kPerT];
  uint32_t held_ok = 0;
  auto fetch = [&](int k0) {
    const int k = min(k0, K - 8 - kc);  // a tail stage reads in bounds; deposit zeroes it
    held_ok = k0 + kc < K ? live : 0u;
#pragma unroll
    for (int c = 0; c < kPerW + kPerT; ++c) held[c] = load16((c < kPerW ? wsrc[c] : xsrc[c - kPerW]) + k);
  };
  auto deposit = [&](int buf) {
#pragma unroll
    for (int c = 0; c < kPerW + kPerT; ++c) {
      const bool ok = (held_ok >> c) & 1u;
      vec16 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v.w[e] = ok ? held[c].w[e] : 0u;
      store16(&stage[buf][(kRowsPerPass * c + trow) * kGemmPitch + kc], v);
    }
  };

  mfma_acc4 acc[FW][FT];
#pragma unroll
  for (int i = 0; i < FW; ++i) {
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }

  const int stages = (K + kStageK - 1) / kStageK;
  fetch(0);
  deposit(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int buf = s & 1;
    if (s + 1 < stages) fetch((s + 1) * kStageK);
    const elem_t* wl = &stage[buf][(ww + col) * kGemmPitch + 8 * grp];
    const elem_t* tl = &stage[buf][(BW + wt + col) * kGemmPitch + 8 * grp];
#pragma unroll
    for (int kk = 0; kk < kStageK; kk += 32) {
      mfma_in8 bt[FT], aw[FW];
#pragma unroll
      for (int j = 0; j < FT; ++j) bt[j] = lds_operand(tl + j * 16 * kGemmPitch + kk);
#pragma unroll
      for (int i = 0; i < FW; ++i) aw[i] = lds_operand(wl + i * 16 * kGemmPitch + kk);
#pragma unroll
      for (int i = 0; i < FW; ++i) {
#pragma unroll
        for (int j = 0; j < FT; ++j) acc[i][j] = mfma16x16x32(aw[i], bt[j], acc[i][j]);
      }
      // Fragment reads ahead of the products (all of the token side and four
      // W rows, then one more W read per group of products), so that LDS
      // latency overlaps matrix work.
      __builtin_amdgcn_sched_group_barrier(0x100, FT + 4, 0);
#pragma unroll
      for (int i = 0; i < FW; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, FT, 0);
        if (i < FW - 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      }
    }
    if (s + 1 < stages) deposit(buf ^ 1);
    __syncthreads();
  }

  // acc[i][j][v] = Y[token t0 + wt + 16j + col][feature w0 + ww + 16i + 4grp + v]
  const bool whole_words = (N & 3) == 0;
#pragma unroll
  for (int j = 0; j < FT; ++j) {
    const int t = t0 + wt + j * 16 + col;
    if (t >= T) continue;
#pragma unroll
    for (int i = 0; i < FW; ++i) {
      const int w = w0 + ww + i * 16 + 4 * grp;
      const size_t at = static_cast<size_t>(t) * N + w;
      if (whole_words && w + 4 <= N) {
        if (kFp32Out) {
          *reinterpret_cast<float4*>(static_cast<float*>(Y) + at) =
              float4{acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        } else {
          uint2 packed;
          packed.x = pack_elems(acc[i][j][0], acc[i][j][1]);
          packed.y = pack_elems(acc[i][j][2], acc[i][j][3]);
          *reinterpret_cast<uint2*>(static_cast<elem_t*>(Y) + at) = packed;
        }
      } else {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          if (w + v >= N) break;
          if (kFp32Out) {
            static_cast<float*>(Y)[at + v] = acc[i][j][v];
          } else {
            static_cast<elem_t*>(Y)[at + v] = float_to_elem(acc[i][j][v]);
          }
        }
      }
    }
  }
}

enum class GemmShape { k256x256, k256x128, k128x128 };

// The tile shape with the least estimated time: whole rounds of tiles over
// the compute units, each tile costing its area over the shape's relative
// efficiency (larger tiles reuse each LDS fragment more often and move fewer
// bytes per flop).
GemmShape choose_gemm_shape(int T, int N, int cus) {
  struct Option {
    GemmShape shape;
    int bw, bt;
    double efficiency;
  };
  static const Option options[] = {{GemmShape::k256x256, 256, 256, 1.0},
                                   {GemmShape::k256x128, 256, 128, 0.85},
                                   {GemmShape::k128x128, 128, 128, 0.6}};
  GemmShape best = GemmShape::k128x128;
  double best_cost = 0.0;
  bool first = true;
  for (const Option& o : options) {
    const long long tiles = static_cast<long long>((N + o.bw - 1) / o.bw) * ((T + o.bt - 1) / o.bt);
    const long long rounds = (tiles + cus - 1) / cus;
    const double cost = static_cast<double>(rounds) * o.bw * o.bt / o.efficiency;
    if (first || cost < best_cost) {
      best = o.shape;
      best_cost = cost;
      first = false;
    }
  }
  return best;
}

template <int BW, int BT, int kWavesW, int kWavesT>
void launch_gemm_tiles(void* Y, bool fp32_out, const elem_t* X, const elem_t* W, int T, int N, int K,
                       hipStream_t s) {
  const int tiles_t = (T + BT - 1) / BT;
  const int total = ((N + BW - 1) / BW) * tiles_t;
  const unsigned blocks = static_cast<unsigned>(((total + 7) / 8) * 8);
  constexpr unsigned kThreads = 64u * kWavesW * kWavesT;
  if (fp32_out) {
    gemm_nt_kernel<BW, BT, kWavesW, kWavesT, true><<<blocks, kThreads, 0, s>>>(Y, X, W, T, N, K, tiles_t, total);
  } else {
    gemm_nt_kernel<BW, BT, kWavesW, kWavesT, false><<<blocks, kThreads, 0, s>>>(Y, X, W, T, N, K, tiles_t, total);
  }
}

// ---------------------------------------------------------------------------
// Prefill attention (MFMA, flash-style)
// ---------------------------------------------------------------------------

constexpr int kFlashThreads = 256;  // four waves: the query heads of one kv head
constexpr int kFlashKeys = 64;      // keys per staged tile

// Slot of key k (0..63) of a tile in the transposed value rows: the order in
// which a wave's S^T accumulators hand keys to the P operand. MFMA k-slot
// 8g + j of a 32-key step holds key 4g + j (j < 4) or 16 + 4g + (j - 4).
__device__ __forceinline__ int value_slot(int k) {
  return (k & 32) | (((k & 15) >> 2) << 3) | ((k & 16) >> 2) | (k & 3);
}
// 16-byte group swizzle of transposed value row d: staging writes are at most
// two-way bank conflicted and the operand reads are conflict free.
__device__ __forceinline__ int value_swizzle(int d) { return ((d >> 3) ^ (d >> 1)) & 7; }

template <int kHeadDim>
struct FlashShared {
  static constexpr int kKeyPitch = kHeadDim + 8;
  elem_t keys[2][kFlashKeys * kKeyPitch];
  elem_t values_t[2][kHeadDim * kFlashKeys];
};

template <bool kPaged, int kHeadDim, int kRF>
__global__ __launch_bounds__(kFlashThreads) void flash_prefill_kernel(
    elem_t* __restrict__ out, const elem_t* __restrict__ q_heads, KvCacheView view, int num_heads,
    int group, int tokens, int start_position, float scale) {
  constexpr float kLog2e = 1.44269504088896341f;
  constexpr int kRows = 16 * kRF;                         // query positions per block
  constexpr int kSteps = kHeadDim / 32;                   // MFMA k-steps over head_dim
  constexpr int kDFrags = kHeadDim / 16;                  // output fragments over head_dim
  constexpr int kChunks = kFlashKeys * kHeadDim / 8;      // 16-byte chunks per K (or V) tile
  constexpr int kPer = kChunks / kFlashThreads;
  constexpr int kKeyPitch = FlashShared<kHeadDim>::kKeyPitch;
  static_assert(kChunks % kFlashThreads == 0, "tile must split evenly over the block");
  __shared__ __attribute__((aligned(16))) FlashShared<kHeadDim> sh;

  const int r0 = static_cast<int>(gridDim.x - 1u - blockIdx.x) * kRows;  // longest rows first
  const int kv = blockIdx.y;
  const int wave = threadIdx.x >> 6;
  const int lane = lane_id();
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int g = blockIdx.z * 4 + wave;
  const bool active = g < group;
  const int head = kv * group + (active ? g : 0);

  const int last_key = start_position + tokens - 1;
  const int block_keys = start_position + min(r0 + kRows, tokens);
  const int tiles = (block_keys + kFlashKeys - 1) / kFlashKeys;

  // Q fragments, the N side of S^T: row r0 + 16rf + col, dims 32ks + 8grp .. +7.
  mfma_in8 qf[kRF][kSteps];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    const int row = r0 + rf * 16 + col;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      vec16 v{{0u, 0u, 0u, 0u}};
      if (active && row < tokens) {
        v = load16(q_heads + (static_cast<size_t>(head) * tokens + row) * kHeadDim + ks * 32 + 8 * grp);
      }
      qf[rf][ks] = as_operand(v);
    }
  }

  vec16 kreg[kPer], vreg[kPer];
  auto fetch = [&](int tile, bool with_values) {
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int chunk = c * kFlashThreads + threadIdx.x;
      const int key = chunk / (kHeadDim / 8);
      const int d0 = (chunk % (kHeadDim / 8)) * 8;
      const size_t at = view.offset<kPaged>(kv, min(tile * kFlashKeys + key, last_key)) + d0;
      kreg[c] = load16(view.keys + at);
      if (with_values) vreg[c] = load16(view.values + at);
    }
  };
  auto deposit = [&](int buf, bool with_values) {
#pragma unroll
    for (int c = 0; c < kPer; ++c) {
      const int chunk = c * kFlashThreads + threadIdx.x;
      const int key = chunk / (kHeadDim / 8);
      const int d0 = (chunk % (kHeadDim / 8)) * 8;
      store16(&sh.keys[buf][key * kKeyPitch + d0], kreg[c]);
      if (!with_values) continue;
      const int slot = value_slot(key);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int d = d0 + j;
        const uint16_t bits = static_cast<uint16_t>(vreg[c].w[j >> 1] >> (16 * (j & 1)));
        sh.values_t[buf][d * kFlashKeys + ((((slot >> 3) ^ value_swizzle(d)) << 3) | (slot & 7))] =
            elem_t{bits};
      }
    }
  };
  // Scaled scores of one staged tile, transposed: s[rf][kf][v] is the score of
  // row 16rf + col against key 16kf + 4grp + v; keys past a row's position are
  // -inf.
  auto scores = [&](int buf, int tile, mfma_acc4 (&s)[kRF][4]) {
#pragma unroll
    for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) s[rf][kf] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
        const mfma_in8 a = lds_operand(&sh.keys[buf][(kf * 16 + col) * kKeyPitch + ks * 32 + 8 * grp]);
#pragma unroll
        for (int rf = 0; rf < kRF; ++rf) s[rf][kf] = mfma16x16x32(a, qf[rf][ks], s[rf][kf]);
      }
    }
    const int key0 = tile * kFlashKeys;
    const bool masked = key0 + kFlashKeys - 1 > start_position + r0;
#pragma unroll
    for (int rf = 0; rf < kRF; ++rf) {
      const int limit = start_position + r0 + rf * 16 + col;  // last key this row sees
#pragma unroll
      for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float x = s[rf][kf][v] * scale;
          s[rf][kf][v] = (masked && key0 + kf * 16 + 4 * grp + v > limit) ? -__builtin_huge_valf() : x;
        }
      }
    }
  };

  // Pass 1: row max M and sum L = sum exp(s - M), keys only. The sum is kept
  // per lane against a running max and rescaled when the max grows.
  float m[kRF], l[kRF];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    m[rf] = -__builtin_huge_valf();
    l[rf] = 0.0f;
  }
  fetch(0, false);
  deposit(0, false);
  __syncthreads();
  for (int tile = 0; tile < tiles; ++tile) {
    const int buf = tile & 1;
    if (tile + 1 < tiles) fetch(tile + 1, false);
    if (active) {
      mfma_acc4 s[kRF][4];
      scores(buf, tile, s);
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) {
        float mt = s[rf][0][0];
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
          for (int v = 0; v < 4; ++v) mt = fmaxf(mt, s[rf][kf][v]);
        }
        mt = fmaxf(mt, xor_lane<16>(mt));
        mt = fmaxf(mt, xor_lane<32>(mt));
        const float m_new = fmaxf(m[rf], mt);
        float sum = 0.0f;
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
          for (int v = 0; v < 4; ++v) sum += __builtin_amdgcn_exp2f((s[rf][kf][v] - m_new) * kLog2e);
        }
        l[rf] = __builtin_fmaf(l[rf], __builtin_amdgcn_exp2f((m[rf] - m_new) * kLog2e), sum);
        m[rf] = m_new;
      }
    }
    if (tile + 1 < tiles) deposit(buf ^ 1, false);
    __syncthreads();
  }
  float inv[kRF];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    float total = l[rf];
    total += xor_lane<16>(total);
    total += xor_lane<32>(total);
    inv[rf] = 1.0f / total;
  }

  // Pass 2: p = exp(s - M) * (1/L) rounded to the element type, where the
  // reference rounds its probability buffer, then O^T += V^T . P^T in fp32.
  mfma_acc4 o[kRF][kDFrags];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
#pragma unroll
    for (int df = 0; df < kDFrags; ++df) o[rf][df] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }
  fetch(0, true);
  deposit(0, true);
  __syncthreads();
  for (int tile = 0; tile < tiles; ++tile) {
    const int buf = tile & 1;
    if (tile + 1 < tiles) fetch(tile + 1, true);
    if (active) {
      mfma_acc4 s[kRF][4];
      scores(buf, tile, s);
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) {
        uint32_t pk[4][2];
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
          float pr[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) pr[v] = __builtin_amdgcn_exp2f((s[rf][kf][v] - m[rf]) * kLog2e) * inv[rf];
          pk[kf][0] = pack_elems(pr[0], pr[1]);
          pk[kf][1] = pack_elems(pr[2], pr[3]);
        }
#pragma unroll
        for (int step = 0; step < 2; ++step) {
          const vec16 pw{{pk[2 * step][0], pk[2 * step][1], pk[2 * step + 1][0], pk[2 * step + 1][1]}};
          const mfma_in8 b = as_operand(pw);
#pragma unroll
          for (int df = 0; df < kDFrags; ++df) {
            const int d = df * 16 + col;
            const mfma_in8 a = lds_operand(
                &sh.values_t[buf][d * kFlashKeys + (((step * 4 + grp) ^ value_swizzle(d)) << 3)]);
            o[rf][df] = mfma16x16x32(a, b, o[rf][df]);
          }
        }
      }
    }
    if (tile + 1 < tiles) deposit(buf ^ 1, true);
    __syncthreads();
  }

  if (!active) return;
  // o[rf][df][v] = O[row 16rf + col][dim 16df + 4grp + v]
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    const int row = r0 + rf * 16 + col;
    if (row >= tokens) continue;
    elem_t* dst = out + static_cast<size_t>(row) * num_heads * kHeadDim +
                  static_cast<size_t>(head) * kHeadDim + 4 * grp;
#pragma unroll
    for (int df = 0; df < kDFrags; ++df) {
      uint2 packed;
      packed.x = pack_elems(o[rf][df][0], o[rf][df][1]);
      packed.y = pack_elems(o[rf][df][2], o[rf][df][3]);
      *reinterpret_cast<uint2*>(dst + df * 16) = packed;
    }
  }
}

// Head dims other than 64 and 128 (up to 128): one block per (query row, kv
// head), one wave per query head, the reference's two-pass rounding.
constexpr int kGenericThreads = 256;

template <bool kPaged>
__global__ __launch_bounds__(kGenericThreads) void prefill_attention_generic_kernel(
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

  const elem_t* qrow = q_heads + (static_cast<size_t>(head) * tokens + row) * head_dim;
  const float q0 = lane < head_dim ? elem_to_float(qrow[lane]) : 0.0f;
  const float q1 = lane + 64 < head_dim ? elem_to_float(qrow[lane + 64]) : 0.0f;

  auto score = [&](int key) -> float {
    const elem_t* k = view.keys + view.offset<kPaged>(kv, key);
    float d = 0.0f;
    d = __builtin_fmaf(q0, lane < head_dim ? elem_to_float(k[lane]) : 0.0f, d);
    d = __builtin_fmaf(q1, lane + 64 < head_dim ? elem_to_float(k[lane + 64]) : 0.0f, d);
    return wave_sum(d) * scale;
  };

  float m = kSoftmaxIdentity;
  for (int key = 0; key < limit; ++key) m = fmaxf(m, score(key));
  float l = 0.0f;
  for (int key = 0; key < limit; ++key) l += lcr_expf(score(key) - m);
  const float inv = 1.0f / l;

  float acc0 = 0.0f, acc1 = 0.0f;
  for (int base = 0; base < limit; base += 64) {
    const int n = min(64, limit - base);
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

template <bool kPaged, int kHeadDim>
void launch_flash(elem_t* o, const elem_t* q, const KvCacheView& v, int num_heads, int group,
                  int tokens, int start_position, float scale, hipStream_t s) {
  const unsigned zs = static_cast<unsigned>((group + 3) / 4);
  // Two row fragments per wave when that still gives two blocks per compute unit.
  const long long wide_blocks = static_cast<long long>((tokens + 31) / 32) * v.num_kv_heads * zs;
  if (wide_blocks >= 2LL * device_compute_units()) {
    const dim3 grid(static_cast<unsigned>((tokens + 31) / 32), static_cast<unsigned>(v.num_kv_heads), zs);
    flash_prefill_kernel<kPaged, kHeadDim, 2><<<grid, kFlashThreads, 0, s>>>(
        o, q, v, num_heads, group, tokens, start_position, scale);
  } else {
    const dim3 grid(static_cast<unsigned>((tokens + 15) / 16), static_cast<unsigned>(v.num_kv_heads), zs);
    flash_prefill_kernel<kPaged, kHeadDim, 1><<<grid, kFlashThreads, 0, s>>>(
        o, q, v, num_heads, group, tokens, start_position, scale);
  }
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
                 (reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(Y) & 15u) == 0,
             "gemm needs 16-byte aligned operands");
  auto s = static_cast<hipStream_t>(stream);
  auto* x = static_cast<const elem_t*>(X);
  auto* w = static_cast<const elem_t*>(W);
  switch (choose_gemm_shape(T, N, device_compute_units())) {
    case GemmShape::k256x256:
      launch_gemm_tiles<256, 256, 2, 4>(Y, y_fp32 != 0, x, w, T, N, K, s);
      break;
    case GemmShape::k256x128:
      launch_gemm_tiles<256, 128, 4, 2>(Y, y_fp32 != 0, x, w, T, N, K, s);
      break;
    case GemmShape::k128x128:
      launch_gemm_tiles<128, 128, 2, 2>(Y, y_fp32 != 0, x, w, T, N, K, s);
      break;
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
  auto s = static_cast<hipStream_t>(stream);
  auto* o = static_cast<elem_t*>(out);
  auto* q = static_cast<const elem_t*>(q_heads);
  const bool aligned = (reinterpret_cast<uintptr_t>(out) & 7u) == 0 &&
                       (reinterpret_cast<uintptr_t>(q_heads) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v.keys) & 15u) == 0 &&
                       (reinterpret_cast<uintptr_t>(v.values) & 15u) == 0 &&
                       v.head_stride % 8 == 0 && v.page_stride % 8 == 0;
  if (aligned && (v.head_dim == 64 || v.head_dim == 128)) {
    if (v.head_dim == 64) {
      if (paged) {
        launch_flash<true, 64>(o, q, v, num_heads, heads_per_kv, tokens, start_position, scale, s);
      } else {
        launch_flash<false, 64>(o, q, v, num_heads, heads_per_kv, tokens, start_position, scale, s);
      }
    } else {
      if (paged) {
        launch_flash<true, 128>(o, q, v, num_heads, heads_per_kv, tokens, start_position, scale, s);
      } else {
        launch_flash<false, 128>(o, q, v, num_heads, heads_per_kv, tokens, start_position, scale, s);
      }
    }
  } else {
    const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>(v.num_kv_heads),
                    static_cast<unsigned>((heads_per_kv + 3) / 4));
    if (paged) {
      prefill_attention_generic_kernel<true><<<grid, kGenericThreads, 0, s>>>(
          o, q, v, num_heads, heads_per_kv, tokens, start_position, scale);
    } else {
      prefill_attention_generic_kernel<false><<<grid, kGenericThreads, 0, s>>>(
          o, q, v, num_heads, heads_per_kv, tokens, start_position, scale);
    }
  }
  CAPI_LAUNCHED();
  return LCR_OK;
}
