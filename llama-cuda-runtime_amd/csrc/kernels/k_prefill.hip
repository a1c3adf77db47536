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
#include "row_norm.h"

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

// Two floats rounded to the element type (nearest even) by the packed
// hardware conversion, low half first.
__device__ __forceinline__ uint32_t pack_rounded(float lo, float hi) {
  typedef float f32x2 __attribute__((ext_vector_type(2)));
#if defined(LCR_ELEM_FP16)
  typedef _Float16 e16x2 __attribute__((ext_vector_type(2)));
#else
  typedef __bf16 e16x2 __attribute__((ext_vector_type(2)));
#endif
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, e16x2));
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
// A stage row is 64 elements (128 bytes) with its 16-byte chunk c stored at
// position c ^ (row & 7): the fragment reads of 16 consecutive rows are then
// free of bank conflicts (measured on MI355X; a padded 72-element pitch costs
// about half again as much per read).
constexpr int kGemmPitch = kStageK;

// The work of one launch: tiles of W rows x tokens, each optionally split
// over K into `splits` slices of k_chunk elements. A split launch writes
// fp32 partial products, slice s to partial + s * T * N, and a second kernel
// sums the slices in slice order.
//
// Gated launches (ffn > 0) compute SwiGLU of the fused gate/up projection,
// whose weight holds the ffn gate rows then the ffn up rows: logical row p
// reads weight row weight_row(p), so that each 32 logical rows hold 16 gate
// rows then the 16 up rows of the same features. A wave's fragments 2m and
// 2m + 1 then pair gate and up values of the same outputs, and the epilogue
// writes act = rne(silu(rne(gate)) * rne(up)), the same roundings as a GEMM
// to 16-bit followed by the SwiGLU kernel.
//
// Projection launches with RoPE (rope.table != nullptr) write nothing to Y:
// the q/k/v projection's output rows are num_heads query heads, then the
// cache's key heads and value heads, head_dim rows each. Each output is
// rounded to the element type, as a 16-bit GEMM output would be; queries are
// then rotated into q_heads [num_heads][T][head_dim], keys rotated and values
// copied into the cache at position start_position + t, with the arithmetic
// of the separate RoPE kernels reading a 16-bit output. The unsplit epilogue
// pairs element i of a head with i + head_dim / 2 inside one lane (fragments
// m and m + head_dim / 32 of a 64- or 128-row head block), so a wave's rows
// must hold whole heads; split launches rotate in the reduction.
struct GemmRope {
  const float2* table;  // (cos, sin) of position p, pair i at p * head_dim / 2 + i
  elem_t* q_heads;
  KvCacheView view;
  int start_position;
  int q_dim;  // num_heads * head_dim: the rows before it are queries
  int paged;
};

struct GemmGrid {
  int tiles_t;
  int tiles_w;
  int splits;
  int k_chunk;
  float* partial;  // nullptr: no split, write Y
  int ffn;         // > 0: gated (Y is act[T][ffn], N == 2 * ffn)
  GemmRope rope;
};

__device__ __forceinline__ int weight_row(int p, int ffn) {
  return ffn == 0 ? p : (((p >> 5) << 4) | (p & 15)) + ((p & 16) ? ffn : 0);
}

__device__ __forceinline__ float swiglu_rounded(float gate, float up) {
  const float g = elem_bits_to_float(float_to_elem_bits(gate));
  const float u = elem_bits_to_float(float_to_elem_bits(up));
  return elem_bits_to_float(float_to_elem_bits(lcr_silu(g) * u));
}

__device__ __forceinline__ float round_to_elem(float x) { return elem_bits_to_float(float_to_elem_bits(x)); }

// Four pairs (i .. i + 3 with i + half .. i + half + 3) of output row t of the
// head whose first projection row is row0, already rounded to the element
// type: rotated into q_heads or the keys, or copied into the values.
template <bool kPaged>
__device__ __forceinline__ void emit_rope_quad(const GemmRope& r, int T, int t, int row0, int i, int head_dim,
                                               const float (&lo)[4], const float (&hi)[4]) {
  const int half = head_dim >> 1;
  const int position = r.start_position + t;
  const int kv_dim = r.view.num_kv_heads * head_dim;
  float a[4], b[4];
  elem_t* dst;
  if (row0 < r.q_dim + kv_dim) {
    const float4* cs = reinterpret_cast<const float4*>(r.table + static_cast<size_t>(position) * half + i);
    const float4 c01 = cs[0], c23 = cs[1];
    const float2 c[4] = {{c01.x, c01.y}, {c01.z, c01.w}, {c23.x, c23.y}, {c23.z, c23.w}};
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float2 rot = rope_rotate(lo[v], hi[v], c[v]);
      a[v] = rot.x;
      b[v] = rot.y;
    }
    dst = row0 < r.q_dim
              ? r.q_heads + (static_cast<size_t>(row0 / head_dim) * T + t) * head_dim + i
              : r.view.keys + r.view.offset<kPaged>((row0 - r.q_dim) / head_dim, position) + i;
  } else {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      a[v] = lo[v];
      b[v] = hi[v];
    }
    dst = r.view.values + r.view.offset<kPaged>((row0 - r.q_dim - kv_dim) / head_dim, position) + i;
  }
  *reinterpret_cast<uint2*>(dst) = uint2{pack_elems(a[0], a[1]), pack_elems(a[2], a[3])};
  *reinterpret_cast<uint2*>(dst + half) = uint2{pack_elems(b[0], b[1]), pack_elems(b[2], b[3])};
}

// The unsplit RoPE epilogue for heads of 32 kHalfFrags rows: fragment m of a
// head block holds pairs 16 m + 4 grp + v, its partner fragment m + kHalfFrags
// the matching high halves.
template <int FW, int FT, int kHalfFrags, bool kPaged>
__device__ __forceinline__ void store_rope_tile(const mfma_acc4 (&acc)[FW][FT], const GemmRope& r, int T, int N,
                                                int t_base, int w_base, int col, int grp) {
  constexpr int kHeadDim = 32 * kHalfFrags;
  static_assert(FW % (2 * kHalfFrags) == 0, "a wave's rows hold whole heads");
#pragma unroll
  for (int j = 0; j < FT; ++j) {
    const int t = t_base + j * 16 + col;
    if (t >= T) continue;
#pragma unroll
    for (int hb = 0; hb < FW / (2 * kHalfFrags); ++hb) {
      const int row0 = w_base + hb * kHeadDim;
      if (row0 >= N) continue;
#pragma unroll
      for (int m = 0; m < kHalfFrags; ++m) {
        const int f = 2 * kHalfFrags * hb + m;
        float lo[4], hi[4];
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          lo[v] = round_to_elem(acc[f][j][v]);
          hi[v] = round_to_elem(acc[f + kHalfFrags][j][v]);
        }
        emit_rope_quad<kPaged>(r, T, t, row0, 16 * m + 4 * grp, kHeadDim, lo, hi);
      }
    }
  }
}

template <int FW, int FT>
__device__ __forceinline__ void store_rope_heads(const mfma_acc4 (&acc)[FW][FT], const GemmRope& r, int T, int N,
                                                 int t_base, int w_base, int col, int grp) {
  // Waves whose rows are not whole heads (the 192-row tile) always take the
  // staged epilogue; the planner gives them no other case.
  if (r.view.head_dim == 64) {
    if constexpr (FW % 4 == 0) {
      if (r.paged) {
        store_rope_tile<FW, FT, 2, true>(acc, r, T, N, t_base, w_base, col, grp);
      } else {
        store_rope_tile<FW, FT, 2, false>(acc, r, T, N, t_base, w_base, col, grp);
      }
    }
  } else if constexpr (FW % 8 == 0) {
    if (r.paged) {
      store_rope_tile<FW, FT, 4, true>(acc, r, T, N, t_base, w_base, col, grp);
    } else {
      store_rope_tile<FW, FT, 4, false>(acc, r, T, N, t_base, w_base, col, grp);
    }
  }
}

struct GemmWork {
  int w0, t0, k_first, k_len, split;
};

// XCD-aware order: XCD x (block id mod 8) takes work units [x*per, (x+1)*per),
// tokens fastest, so the blocks of one XCD share W slices in its L2.
__device__ __forceinline__ bool gemm_work(const GemmGrid& g, int BW, int BT, int K, GemmWork& w) {
  const int units = g.tiles_t * g.tiles_w * g.splits;
  const int per_xcd = (units + 7) / 8;
  const int u = static_cast<int>(blockIdx.x % 8u) * per_xcd + static_cast<int>(blockIdx.x / 8u);
  if (u >= units) return false;
  const int tt = u % g.tiles_t;
  const int rest = u / g.tiles_t;
  w.split = rest % g.splits;
  w.w0 = (rest / g.splits) * BW;
  w.t0 = tt * BT;
  w.k_first = w.split * g.k_chunk;
  w.k_len = min(K, w.k_first + g.k_chunk) - w.k_first;
  return true;
}

// acc[i][j][v] is output (token t0 + tw + 16j + col, feature w0 + ww + 16i + 4grp + v).
template <int FW, int FT, bool kFp32Out>
__device__ __forceinline__ void store_gemm_tile(const mfma_acc4 (&acc)[FW][FT], void* Y, float* partial,
                                                int T, int N, int t_base, int w_base, int col, int grp,
                                                const GemmGrid& grid) {
  const int ffn = grid.ffn;
  if constexpr (!kFp32Out) {
    if (grid.rope.table != nullptr && partial == nullptr) {
      store_rope_heads<FW, FT>(acc, grid.rope, T, N, t_base, w_base, col, grp);
      return;
    }
  }
  if (ffn > 0 && partial == nullptr) {
    // fragments 2m (gate) and 2m + 1 (up): features (w_base + 32m) / 2 + 4grp + v
#pragma unroll
    for (int j = 0; j < FT; ++j) {
      const int t = t_base + j * 16 + col;
      if (t >= T) continue;
#pragma unroll
      for (int m = 0; m < FW / 2; ++m) {
        const int f = (w_base + 32 * m) / 2 + 4 * grp;
        if (f >= ffn) continue;
        uint2 packed;
        packed.x = pack_elems(swiglu_rounded(acc[2 * m][j][0], acc[2 * m + 1][j][0]),
                              swiglu_rounded(acc[2 * m][j][1], acc[2 * m + 1][j][1]));
        packed.y = pack_elems(swiglu_rounded(acc[2 * m][j][2], acc[2 * m + 1][j][2]),
                              swiglu_rounded(acc[2 * m][j][3], acc[2 * m + 1][j][3]));
        *reinterpret_cast<uint2*>(static_cast<elem_t*>(Y) + static_cast<size_t>(t) * ffn + f) = packed;
      }
    }
    return;
  }
  const bool whole_words = (N & 3) == 0;
#pragma unroll
  for (int j = 0; j < FT; ++j) {
    const int t = t_base + j * 16 + col;
    if (t >= T) continue;
#pragma unroll
    for (int i = 0; i < FW; ++i) {
      const int w = w_base + i * 16 + 4 * grp;
      const size_t at = static_cast<size_t>(t) * N + w;
      const bool fp32 = kFp32Out || partial != nullptr;
      float* out32 = partial != nullptr ? partial : static_cast<float*>(Y);
      if (whole_words && w + 4 <= N) {
        if (fp32) {
          *reinterpret_cast<float4*>(out32 + at) = float4{acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
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
          if (fp32) {
            out32[at + v] = acc[i][j][v];
          } else {
            static_cast<elem_t*>(Y)[at + v] = float_to_elem(acc[i][j][v]);
          }
        }
      }
    }
  }
}

// The ring kernel's output through LDS. A fragment's 16 lanes of one group
// hold 16 consecutive tokens, so a direct store writes 8 or 16 bytes into each
// of 16 output rows N elements apart; with N = 16384 that ran at about
// 2 TB/s. Here each wave writes its finished 4-value groups, converted to the
// output type, into a staged [token][column] tile in the ring (free after the
// last stage): 16-byte chunk c of staged row r sits at slot c ^ (r & mask), so
// a fragment's 16 rows land on distinct slots. The block then copies whole
// 16-byte chunks row by row, each wave store covering 1 KB of consecutive
// columns. Tiles larger than the ring go in passes of kRowsPerPass tokens.
// Needs row widths in bytes that are multiples of 16 (the caller checks);
// chunks past the last column or token are skipped whole.
template <int kRowBytes, int kRowsPerPass>
struct StagedTile {
  static constexpr int kChunks = kRowBytes / 16;
  // XOR inside aligned groups of 16, 8 or 4 chunks (the largest that divides
  // the row), so the swizzle stays a permutation of the row's chunks.
  static constexpr int kMask = (kChunks % 16 == 0 ? 16 : kChunks % 8 == 0 ? 8 : 4) - 1;
  char* lds;
  __device__ __forceinline__ char* slot(int row, int byte) const {
    return lds + row * kRowBytes + ((((byte >> 4) ^ (row & kMask)) << 4) | (byte & 15));
  }
  // Copies staged rows [0, rows) to dst row by row (ld_bytes apart), columns
  // [0, col_bytes) of each.
  template <int kThreads>
  __device__ __forceinline__ void copy_out(char* dst, size_t ld_bytes, int rows, int col_bytes) const {
    static_assert((kRowsPerPass * kChunks) % kThreads == 0, "whole copy rounds");
#pragma unroll 4
    for (int it = 0; it < kRowsPerPass * kChunks / kThreads; ++it) {
      const int idx = it * kThreads + static_cast<int>(threadIdx.x);
      const int r = idx / kChunks, c = idx % kChunks;
      if (r < rows && c * 16 < col_bytes) {
        const uint4 v = *reinterpret_cast<const uint4*>(lds + r * kRowBytes + ((c ^ (r & kMask)) << 4));
        *reinterpret_cast<uint4*>(dst + r * ld_bytes + c * 16) = v;
      }
    }
  }
};

// Whether the ring kernel's epilogue goes through StagedTile: when every
// destination is 16-byte aligned and its rows are whole 16-byte chunks.
__device__ __forceinline__ bool staged_store_ok(const GemmGrid& grid, const void* Y, const float* partial,
                                                bool fp32_out, int N) {
  if (partial == nullptr && !fp32_out && grid.rope.table != nullptr) {
    // The RoPE epilogue writes 16-byte chunks of query rows and cache rows.
    const KvCacheView& v = grid.rope.view;
    return ((reinterpret_cast<uintptr_t>(grid.rope.q_heads) | reinterpret_cast<uintptr_t>(v.keys) |
             reinterpret_cast<uintptr_t>(v.values)) & 15) == 0 &&
           (v.page_stride & 7) == 0 && (v.head_stride & 7) == 0;
  }
  const void* out = partial != nullptr ? static_cast<const void*>(partial) : Y;
  if ((reinterpret_cast<uintptr_t>(out) & 15) != 0) return false;
  if (grid.ffn > 0 && partial == nullptr) return (grid.ffn & 7) == 0;
  return (partial != nullptr || fp32_out) ? (N & 3) == 0 : (N & 7) == 0;
}

// The RoPE epilogue from a staged tile of 16-bit projection outputs (already
// rounded, as the unfused path rounds the q/k/v buffer): thread item (token
// row, group of eight pairs i .. i + 7) loads that position's eight (cos, sin)
// once and serves every head of the tile with them, rotating a query or key
// head's pairs (i, i + half) into q_heads or the keys, or copying a value
// head's; each write is a 16-byte chunk. The same arithmetic as
// emit_rope_quad, so the same bits.
template <int kHd, bool kPaged, int BW, int BT, int kThreads, class Tile>
__device__ __forceinline__ void rope_copy_out(const Tile& tile, const GemmRope& r, int T, int N, int t0, int w0) {
  constexpr int kHalf = kHd / 2;
  constexpr int kGroups = kHalf / 8;
  constexpr int kHeads = BW / kHd;
  constexpr int kItems = BT * kGroups;
  static_assert(BW % kHd == 0 && kItems % kThreads == 0, "whole heads per tile, whole item rounds");
  const int kv_dim = r.view.num_kv_heads * kHd;
#pragma unroll
  for (int it = 0; it < kItems / kThreads; ++it) {
    const int item = it * kThreads + static_cast<int>(threadIdx.x);
    const int row = item / kGroups;
    const int i = 8 * (item % kGroups);
    const int t = t0 + row;
    if (t >= T) continue;
    const int position = r.start_position + t;
    const float4* cs4 = reinterpret_cast<const float4*>(r.table + static_cast<size_t>(position) * kHalf + i);
    float2 c[8];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 w = cs4[q];
      c[2 * q] = make_float2(w.x, w.y);
      c[2 * q + 1] = make_float2(w.z, w.w);
    }
#pragma unroll
    for (int hb = 0; hb < kHeads; ++hb) {
      const int row0 = w0 + hb * kHd;
      if (row0 >= N) break;
      const vec16 lo_v = *reinterpret_cast<const vec16*>(tile.slot(row, (hb * kHd + i) * 2));
      const vec16 hi_v = *reinterpret_cast<const vec16*>(tile.slot(row, (hb * kHd + kHalf + i) * 2));
      if (row0 >= r.q_dim + kv_dim) {
        elem_t* dst = r.view.values + r.view.offset<kPaged>((row0 - r.q_dim - kv_dim) / kHd, position) + i;
        store16(dst, lo_v);
        store16(dst + kHalf, hi_v);
        continue;
      }
      float lo[8], hi[8];
      unpack8(lo_v, lo);
      unpack8(hi_v, hi);
      vec16 a, b;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float2 r0 = rope_rotate(lo[2 * v], hi[2 * v], c[2 * v]);
        const float2 r1 = rope_rotate(lo[2 * v + 1], hi[2 * v + 1], c[2 * v + 1]);
        a.w[v] = pack_elems(r0.x, r1.x);
        b.w[v] = pack_elems(r0.y, r1.y);
      }
      elem_t* dst = row0 < r.q_dim
                        ? r.q_heads + (static_cast<size_t>(row0 / kHd) * T + t) * kHd + i
                        : r.view.keys + r.view.offset<kPaged>((row0 - r.q_dim) / kHd, position) + i;
      store16(dst, a);
      store16(dst + kHalf, b);
    }
  }
}

// The ring tile's store through LDS (see StagedTile): gated tiles write
// act[t][f] = SwiGLU of fragments 2m and 2m + 1, split tiles their fp32
// partial products, others Y in the output type. `lds` holds kLdsBytes.
template <int BW, int BT, int FW, int FT, int kThreads, int kLdsBytes, bool kFp32Out>
__device__ __forceinline__ void store_ring_tile_staged(const mfma_acc4 (&acc)[FW][FT], void* Y, float* partial,
                                                       int T, int N, const GemmGrid& grid, int t0, int w0, int wt,
                                                       int ww, int col, int grp, char* lds) {
  const int ffn = grid.ffn;
  const int rows_left = T - t0;
  if (ffn > 0 && partial == nullptr) {
    constexpr int kRowBytes = BW / 2 * static_cast<int>(sizeof(elem_t));
    static_assert(BT * kRowBytes <= kLdsBytes, "gated tile fits the ring");
    const StagedTile<kRowBytes, BT> tile{lds};
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FT; ++j) {
      const int r = wt + 16 * j + col;
#pragma unroll
      for (int m = 0; m < FW / 2; ++m) {
        const int fl = (ww + 32 * m) / 2 + 4 * grp;
        uint2 packed;
        packed.x = pack_elems(swiglu_rounded(acc[2 * m][j][0], acc[2 * m + 1][j][0]),
                              swiglu_rounded(acc[2 * m][j][1], acc[2 * m + 1][j][1]));
        packed.y = pack_elems(swiglu_rounded(acc[2 * m][j][2], acc[2 * m + 1][j][2]),
                              swiglu_rounded(acc[2 * m][j][3], acc[2 * m + 1][j][3]));
        *reinterpret_cast<uint2*>(tile.slot(r, fl * static_cast<int>(sizeof(elem_t)))) = packed;
      }
    }
    __syncthreads();
    const int f0 = w0 / 2;
    tile.template copy_out<kThreads>(
        reinterpret_cast<char*>(static_cast<elem_t*>(Y) + static_cast<size_t>(t0) * ffn + f0),
        static_cast<size_t>(ffn) * sizeof(elem_t), rows_left, (ffn - f0) * static_cast<int>(sizeof(elem_t)));
    return;
  }
  if (kFp32Out || partial != nullptr) {
    constexpr int kRowBytes = BW * 4;
    constexpr int kRowsPerPass = (BT * kRowBytes <= kLdsBytes) ? BT : kLdsBytes / kRowBytes;
    static_assert(kRowsPerPass % 16 == 0 && BT % kRowsPerPass == 0, "passes of whole fragments");
    const StagedTile<kRowBytes, kRowsPerPass> tile{lds};
    float* out = partial != nullptr ? partial : static_cast<float*>(Y);
#pragma unroll
    for (int pass = 0; pass < BT / kRowsPerPass; ++pass) {
      __syncthreads();
#pragma unroll
      for (int j = 0; j < FT; ++j) {
        const int r = wt + 16 * j + col - pass * kRowsPerPass;
        if (wt + 16 * j < pass * kRowsPerPass || wt + 16 * j >= (pass + 1) * kRowsPerPass) continue;
#pragma unroll
        for (int i = 0; i < FW; ++i) {
          *reinterpret_cast<float4*>(tile.slot(r, (ww + 16 * i + 4 * grp) * 4)) =
              float4{acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        }
      }
      __syncthreads();
      const int first = t0 + pass * kRowsPerPass;
      tile.template copy_out<kThreads>(reinterpret_cast<char*>(out + static_cast<size_t>(first) * N + w0),
                                       static_cast<size_t>(N) * 4, T - first, (N - w0) * 4);
    }
    return;
  }
  constexpr int kRowBytes = BW * static_cast<int>(sizeof(elem_t));
  static_assert(BT * kRowBytes <= kLdsBytes, "tile fits the ring");
  const StagedTile<kRowBytes, BT> tile{lds};
  __syncthreads();
#pragma unroll
  for (int j = 0; j < FT; ++j) {
    const int r = wt + 16 * j + col;
#pragma unroll
    for (int i = 0; i < FW; ++i) {
      uint2 packed;
      packed.x = pack_elems(acc[i][j][0], acc[i][j][1]);
      packed.y = pack_elems(acc[i][j][2], acc[i][j][3]);
      *reinterpret_cast<uint2*>(tile.slot(r, (ww + 16 * i + 4 * grp) * static_cast<int>(sizeof(elem_t)))) = packed;
    }
  }
  __syncthreads();
  if constexpr (!kFp32Out) {
    if (grid.rope.table != nullptr) {
      const GemmRope& r = grid.rope;
      if (r.view.head_dim == 64) {
        if (r.paged) {
          rope_copy_out<64, true, BW, BT, kThreads>(tile, r, T, N, t0, w0);
        } else {
          rope_copy_out<64, false, BW, BT, kThreads>(tile, r, T, N, t0, w0);
        }
      } else if constexpr (BW % 128 == 0) {  // the planner keeps 128-row heads off other tiles
        if (r.paged) {
          rope_copy_out<128, true, BW, BT, kThreads>(tile, r, T, N, t0, w0);
        } else {
          rope_copy_out<128, false, BW, BT, kThreads>(tile, r, T, N, t0, w0);
        }
      }
      return;
    }
  }
  tile.template copy_out<kThreads>(
      reinterpret_cast<char*>(static_cast<elem_t*>(Y) + static_cast<size_t>(t0) * N + w0),
      static_cast<size_t>(N) * sizeof(elem_t), rows_left, (N - w0) * static_cast<int>(sizeof(elem_t)));
}

// Block tile BW x BT (W rows x tokens) over kWavesW x kWavesT waves; each
// wave owns a (BW / kWavesW) x (BT / kWavesT) piece. Operands go global ->
// registers -> LDS, a stage of 64 K ahead, through two LDS buffers.
template <int BW, int BT, int kWavesW, int kWavesT, bool kFp32Out>
__global__ __launch_bounds__(64 * kWavesW * kWavesT) void gemm_nt_kernel(
    void* __restrict__ Y, const elem_t* __restrict__ X, const elem_t* __restrict__ W, int T, int N,
    int K, GemmGrid grid) {
  constexpr int kThreads = 64 * kWavesW * kWavesT;
  constexpr int kWaveW = BW / kWavesW, kWaveT = BT / kWavesT;
  constexpr int FW = kWaveW / 16, FT = kWaveT / 16;
  constexpr int kRowsPerPass = kThreads / 8;  // rows one pass of 16-byte chunks covers
  constexpr int kPerW = BW / kRowsPerPass, kPerT = BT / kRowsPerPass;
  static_assert(BW % kRowsPerPass == 0 && BT % kRowsPerPass == 0, "stage must split evenly");
  __shared__ __attribute__((aligned(16))) elem_t stage[2][(BW + BT) * kGemmPitch];

  GemmWork work;
  if (!gemm_work(grid, BW, BT, K, work)) return;
  const int w0 = work.w0, t0 = work.t0;

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
    wsrc[c] = W + static_cast<size_t>(weight_row(min(row, N - 1), grid.ffn)) * K + work.k_first;
  }
#pragma unroll
  for (int c = 0; c < kPerT; ++c) {
    const int row = t0 + kRowsPerPass * c + trow;
    live |= (row < T ? 1u : 0u) << (kPerW + c);
    xsrc[c] = X + static_cast<size_t>(min(row, T - 1)) * K + work.k_first;
  }
  // The loads of a stage are issued a stage ahead; the zeroing select waits
  // until the data is written to LDS, so nothing waits on the loads before
  // the matrix work of the current stage.
  const int k_len = work.k_len;
  vec16 held[kPerW + kPerT];
  uint32_t held_ok = 0;
  auto fetch = [&](int k0) {
    const int k = min(k0 + kc, k_len - 8);  // a tail stage reads in bounds; deposit zeroes it
    held_ok = k0 + kc < k_len ? live : 0u;
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
      store16(&stage[buf][(kRowsPerPass * c + trow) * kGemmPitch + (((tid & 7) ^ (trow & 7)) << 3)], v);
    }
  };

  mfma_acc4 acc[FW][FT];
#pragma unroll
  for (int i = 0; i < FW; ++i) {
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }

  const int stages = (k_len + kStageK - 1) / kStageK;
  fetch(0);
  deposit(0);
  __syncthreads();
  for (int s = 0; s < stages; ++s) {
    const int buf = s & 1;
    if (s + 1 < stages) fetch((s + 1) * kStageK);
    const elem_t* wl = &stage[buf][(ww + col) * kGemmPitch];
    const elem_t* tl = &stage[buf][(BW + wt + col) * kGemmPitch];
#pragma unroll
    for (int kk = 0; kk < kStageK; kk += 32) {
      mfma_in8 bt[FT], aw[FW];
      const int at = ((((kk >> 3) + grp) ^ (col & 7)) << 3);  // rows 16m + col: row & 7 == col & 7
#pragma unroll
      for (int j = 0; j < FT; ++j) bt[j] = lds_operand(tl + j * 16 * kGemmPitch + at);
#pragma unroll
      for (int i = 0; i < FW; ++i) aw[i] = lds_operand(wl + i * 16 * kGemmPitch + at);
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

  float* partial = grid.partial != nullptr ? grid.partial + static_cast<size_t>(work.split) * T * N : nullptr;
  store_gemm_tile<FW, FT, kFp32Out>(acc, Y, partial, T, N, t0 + wt, w0 + ww, col, grp, grid);
}

// The large-tile GEMM with a ring of kStages LDS stages of 32 K each, filled
// by direct global-to-LDS loads (global_load_lds_dwordx4: lane L's 16 bytes
// land at the wave's LDS address in M0 + 16 L), so loads run kStages - 1
// stages ahead of the matrix work without holding registers. A stage holds
// 256 W rows then 256 token rows of 32 elements (64 bytes); 16-byte chunk g
// of row r sits at position g ^ ((r >> 1) & 3), the placement that measured
// free of bank conflicts for the fragment reads of 16 consecutive rows on
// MI355X. Rows past the end read
// the last row (their outputs are not stored); K must be a multiple of 32.
//
// The loads are issued from inline assembly and the stages are fenced by
// hand: each wave waits until its loads of the stage it is about to read have
// landed (vector-memory count down to the younger stages' loads) and until
// its fragment reads of the previous stage are done, then the block meets at
// a plain s_barrier. Had the compiler seen the loads as LDS writes, it would
// drain every load in flight at each barrier and the ring would be one stage
// deep. Loads the compiler does not count can only make its own in-order
// count waits stricter.
constexpr int kRingK = 32;

// Wait until at most kCount vector-memory operations of this wave are in
// flight and every LDS read has returned (gfx9 encoding: vmcnt bits 3:0 and
// 15:14, expcnt 6:4 left at its maximum, lgkmcnt 11:8 zero).
template <int kCount>
__device__ __forceinline__ void wait_stage_landed() {
  static_assert(kCount >= 0 && kCount < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((kCount & 15) | ((kCount >> 4) << 14) | (7 << 4));
}

// Block tiles of BW W rows x BT tokens:
//  - 256 x 256, kWaves = 8: wave tiles of 128 W rows x 64 tokens (two waves
//    per SIMD);
//  - 256 x 256, kWaves = 4: wave tiles of 128 x 128 (one wave per SIMD, its
//    256 fp32 accumulators in the accumulation registers);
//  - 256 x 128, kWaves = 8: wave tiles of 64 x 64, for token counts whose
//    256-token tiles would leave compute units idle;
//  - 192 x 128, kWaves = 8: wave tiles of 96 x 32 (three 64-row heads per
//    block tile), so 3072 q/k/v rows and 2048 tokens make exactly 256 tiles;
//  - 128 x 128, kWaves = 8: wave tiles of 64 x 32, for projections whose
//    larger tiles would leave compute units idle (two blocks fit a CU).
// kRK: K per ring stage, 32 (64-byte rows) or 64 (128-byte rows: twice the
// products per stage barrier). Either way the products run over K in 32-wide
// MFMA steps in increasing order, so the results are the same bits.
template <int kStages, int kWaves, int BW, int BT, bool kFp32Out, int kRK = kRingK>
__global__ __launch_bounds__(64 * kWaves) void gemm_ring_kernel(void* __restrict__ Y, const elem_t* __restrict__ X,
                                                                const elem_t* __restrict__ W, int T, int N, int K,
                                                                GemmGrid grid) {
  static_assert(kRK == 32 || kRK == 64, "ring stages of 32 or 64 K");
  static_assert((BW == 256 && BT == 256 && (kWaves == 4 || kWaves == 8)) ||
                    ((BW == 256 || BW == 192 || BW == 128) && BT == 128 && kWaves == 8),
                "supported ring tiles: 256 x 256 on 4 or 8 waves, 256 x 128, 192 x 128 and 128 x 128 on 8 waves");
  // waves along W; the rest split the tokens
  constexpr int kWavesW = (BW == 128 || BW == 192 || BT == 256) ? 2 : 4;
  constexpr int kWavesT = kWaves / kWavesW;
  constexpr int FW = BW / kWavesW / 16;  // W fragments of 16 rows per wave
  constexpr int FT = BT / kWavesT / 16;      // token fragments of 16 tokens per wave
  constexpr int kRows = BW + BT;
  constexpr int kStageElems = kRows * kRK;
  constexpr int kLoadRows = 512 / kRK;              // rows of one 1 KB load: 16 or 8
  constexpr int kLanesPerRow = 64 / kLoadRows;      // 16-byte chunks per row: 4 or 8
  constexpr int kKSteps = kRK / 32;                 // MFMA k-steps per stage
  constexpr int kLoads = kRows / kLoadRows / kWaves;  // 1 KB loads per wave per stage
  static_assert(kLoads * kLoadRows * kWaves == kRows, "stage rows split evenly over the waves");
  static_assert(FW % 2 == 0, "the gated epilogue pairs fragments 2m and 2m + 1");
  __shared__ __attribute__((aligned(1024))) elem_t ring[kStages * kStageElems];

  GemmWork work;
  if (!gemm_work(grid, BW, BT, K, work)) return;
  const int w0 = work.w0, t0 = work.t0;

  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int ww = (wave / kWavesT) * (16 * FW);
  const int wt = (wave % kWavesT) * (16 * FT);

  // Chunk c of row r sits at 16-byte slot c ^ swizzle(r) of the row: for
  // 64-byte rows (r >> 1) & 3, for 128-byte rows r & 7; fragment reads of 16
  // consecutive rows are then free of bank conflicts.
  auto row_swizzle = [](int r) { return kRK == 32 ? ((r >> 1) & 3) : (r & 7); };
  // Load i of a wave fills 1 KB block kWaves * i + wave of the stage: rows
  // kLoadRows block .. + kLoadRows - 1, kLanesPerRow lanes per row; a lane
  // loads the chunk that belongs in its slot.
  const elem_t* src[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int row = kLoadRows * (kWaves * i + wave) + lane / kLanesPerRow;
    const int chunk = (lane % kLanesPerRow) ^ row_swizzle(row);
    src[i] = (row < BW ? W + static_cast<size_t>(weight_row(min(w0 + row, N - 1), grid.ffn)) * K
                           : X + static_cast<size_t>(min(t0 + row - BW, T - 1)) * K) + work.k_first + 8 * chunk;
  }
  const uint32_t ring_base = lds_address_of(ring) + static_cast<uint32_t>(wave * 1024);
  auto issue = [&](int s) {
    const uint32_t base = ring_base + static_cast<uint32_t>((s % kStages) * kStageElems * 2);
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      load_to_lds16(src[i] + s * kRK, base + static_cast<uint32_t>(i * kWaves * 1024));
    }
  };

  mfma_acc4 acc[FW][FT];
#pragma unroll
  for (int i = 0; i < FW; ++i) {
#pragma unroll
    for (int j = 0; j < FT; ++j) acc[i][j] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }
  // 16-byte slot of k-step ks's chunk of this lane's fragment rows (16 rows
  // from a multiple of 16, so the row's swizzle is that of `col`).
  auto swz = [&](int ks) { return 8 * ((4 * ks + grp) ^ row_swizzle(col)); };
  const int stages = work.k_len / kRK;
  const int ksteps = stages * kKSteps;
  // The next stage's fragments are read during the current stage's products,
  // so LDS reads overlap matrix work: its token fragments into the second of
  // two sets, and each W fragment into the registers of the current one as
  // soon as that one's products are issued. After the barrier that precedes
  // reading stage s + 1, every wave's reads of stage s have returned, and
  // stage s's buffer takes stage s + kStages.
  mfma_in8 aw[FW], bt_a[FT], bt_b[FT];
  // k-step q: stage q / kKSteps, step q % kKSteps of it.
  auto read_tokens = [&](int q, mfma_in8 (&bt)[FT]) {
    const elem_t* base = ring + ((q / kKSteps) % kStages) * kStageElems + swz(q % kKSteps);
#pragma unroll
    for (int j = 0; j < FT; ++j) bt[j] = lds_operand(base + (BW + wt + 16 * j + col) * kRK);
  };
  // Products of the stage whose fragments are in aw / bt, reading stage
  // `next` into aw / bt_next. After the last stage `next` repeats a stage
  // whose loads have all landed, and what is read goes unused.
  auto step = [&](const mfma_in8 (&bt)[FT], mfma_in8 (&bt_next)[FT], int next) {
    const elem_t* nb =
        ring + ((next / kKSteps) % kStages) * kStageElems + (ww + col) * kRK + swz(next % kKSteps);
    read_tokens(next, bt_next);
    // The wave holds issue priority over its SIMD's other wave while it runs
    // its products, so that wave's loads and LDS reads issue in the matrix
    // pipe's gaps instead of the two waves trading products (same bits;
    // 256 x 128 tiles 4-5 % faster).
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int i = 0; i < FW; ++i) {
#pragma unroll
      for (int j = 0; j < FT; ++j) acc[i][j] = mfma16x16x32(aw[i], bt[j], acc[i][j]);
      aw[i] = lds_operand(nb + 16 * i * kRK);
    }
    // keep that order: the token reads, then per W fragment its products and
    // its replacement's read
    __builtin_amdgcn_sched_group_barrier(0x100, FT, 0);
#pragma unroll
    for (int i = 0; i < FW; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, FT, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
    __builtin_amdgcn_s_setprio(0);
  };
  // Before reading stage `next`: this wave's loads of it have landed (at most
  // the loads of the stages issued after it remain) and its earlier fragment
  // reads have returned; then the block meets and the freed buffer is refilled.
  auto advance = [&](int next) {
    if (next + kStages - 2 < stages) {
      wait_stage_landed<kLoads * (kStages - 2)>();
    } else {
      wait_stage_landed<0>();
    }
    __builtin_amdgcn_s_barrier();
    if (next + kStages - 1 < stages) issue(next + kStages - 1);
  };
  for (int s = 0; s < kStages - 1 && s < stages; ++s) issue(s);
  advance(0);
  read_tokens(0, bt_a);
  {
    const elem_t* base = ring + (ww + col) * kRK + swz(0);
#pragma unroll
    for (int i = 0; i < FW; ++i) aw[i] = lds_operand(base + 16 * i * kRK);
  }
  for (int q = 0; q < ksteps; ++q) {
    // Reading k-step q + 1's fragments opens a new stage every kKSteps steps.
    if (q + 1 < ksteps && (q + 1) % kKSteps == 0) advance((q + 1) / kKSteps);
    step(bt_a, bt_b, min(q + 1, ksteps - 1));
#pragma unroll
    for (int j = 0; j < FT; ++j) bt_a[j] = bt_b[j];
  }

  float* partial = grid.partial != nullptr ? grid.partial + static_cast<size_t>(work.split) * T * N : nullptr;
  if (staged_store_ok(grid, Y, partial, kFp32Out, N)) {
    store_ring_tile_staged<BW, BT, FW, FT, 64 * kWaves, kStages * kStageElems * static_cast<int>(sizeof(elem_t)),
                           kFp32Out>(acc, Y, partial, T, N, grid, t0, w0, wt, ww, col, grp,
                                     reinterpret_cast<char*>(ring));
    return;
  }
  store_gemm_tile<FW, FT, kFp32Out>(acc, Y, partial, T, N, t0 + wt, w0 + ww, col, grp, grid);
}

constexpr int kRingStages = 4;
// Fraction of a compute unit's MFMA peak the 256 x 128 ring tile reaches
// (measured on MI355X; the plan compares it with the other shapes').
constexpr double kRing256x128Efficiency = 0.30;
// 64 K per stage, three stages (144 KiB of LDS): half the stage barriers of 32
// K per stage, the same bits; prefill 2.415 -> 2.356 ms at 512 tokens (with
// the 128 x 128 tile below as well: 2.328 ms, and 6.231 -> 6.115 ms at 2048).
constexpr int kRing256x128K = 64;
constexpr int kRing256x128Stages = 3;
// The 128 x 128 ring tile: o_proj at 2048 tokens (one tile per compute unit)
// takes 24.2 us, 0.28 of a compute unit's peak, against 34-36 us for the
// register-staged 128 x 128 kernel.
constexpr double kRing128x128Efficiency = 0.28;
// The 192 x 128 ring tile: three stages of 64 K (120 KiB of LDS).
constexpr double kRing192x128Efficiency = 0.29;
constexpr int kRing192x128K = 64;
constexpr int kRing192x128Stages = 3;
constexpr int kRing128x128K = 64;  // 64 K per stage, four stages (128 KiB of LDS)
constexpr int kRing128x128Stages = 4;
// Waves per ring block. Eight (two per SIMD) measured faster than four with
// 128 x 128 wave tiles: 143 against 176 us for T = 2048, N = 16384, K = 2048;
// one wave per SIMD leaves the LDS and barrier latencies uncovered.
constexpr int kRingWaves = 8;

// act[t][f] = SwiGLU of the summed gate and up partial products (logical
// columns 32 (f / 16) + f % 16 and that + 16), for gated split launches.
__global__ __launch_bounds__(256) void gemm_reduce_swiglu_kernel(elem_t* __restrict__ act,
                                                                 const float* __restrict__ partial, int splits,
                                                                 int T, int ffn) {
  const size_t i = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;  // act element, f % 4 == 0
  if (i >= static_cast<size_t>(T) * ffn) return;
  const int t = static_cast<int>(i / ffn);
  const int f = static_cast<int>(i % ffn);
  const size_t n = 2 * static_cast<size_t>(ffn);
  const size_t count = static_cast<size_t>(T) * n;
  const size_t g_at = static_cast<size_t>(t) * n + ((f >> 4) << 5) + (f & 15);
  float4 g = *reinterpret_cast<const float4*>(partial + g_at);
  float4 u = *reinterpret_cast<const float4*>(partial + g_at + 16);
  for (int s = 1; s < splits; ++s) {
    const float4 gs = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(s) * count + g_at);
    const float4 us = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(s) * count + g_at + 16);
    g.x += gs.x; g.y += gs.y; g.z += gs.z; g.w += gs.w;
    u.x += us.x; u.y += us.y; u.z += us.z; u.w += us.w;
  }
  uint2 packed;
  packed.x = pack_elems(swiglu_rounded(g.x, u.x), swiglu_rounded(g.y, u.y));
  packed.y = pack_elems(swiglu_rounded(g.z, u.z), swiglu_rounded(g.w, u.w));
  *reinterpret_cast<uint2*>(act + i) = packed;
}

// Split projection launches with RoPE: one thread per (token, head, four
// pairs) sums the slices of its four low and four high outputs in slice
// order, then rounds, rotates and writes them as the unsplit epilogue does.
template <bool kPaged>
__global__ __launch_bounds__(256) void gemm_reduce_rope_kernel(const float* __restrict__ partial, int splits,
                                                               int T, int N, GemmRope r) {
  const int head_dim = r.view.head_dim;
  const int half = head_dim >> 1;
  const int quads = half >> 2;
  const int heads = N / head_dim;
  const size_t u = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
  if (u >= static_cast<size_t>(T) * heads * quads) return;
  const int q = static_cast<int>(u % quads);
  const size_t rest = u / quads;
  const int h = static_cast<int>(rest % heads);
  const int t = static_cast<int>(rest / heads);
  const size_t count = static_cast<size_t>(T) * N;
  const size_t at = static_cast<size_t>(t) * N + static_cast<size_t>(h) * head_dim + 4 * q;
  float4 lo = *reinterpret_cast<const float4*>(partial + at);
  float4 hi = *reinterpret_cast<const float4*>(partial + at + half);
  for (int s = 1; s < splits; ++s) {
    const float4 ls = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(s) * count + at);
    const float4 hs = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(s) * count + at + half);
    lo.x += ls.x; lo.y += ls.y; lo.z += ls.z; lo.w += ls.w;
    hi.x += hs.x; hi.y += hs.y; hi.z += hs.z; hi.w += hs.w;
  }
  const float l[4] = {round_to_elem(lo.x), round_to_elem(lo.y), round_to_elem(lo.z), round_to_elem(lo.w)};
  const float hh[4] = {round_to_elem(hi.x), round_to_elem(hi.y), round_to_elem(hi.z), round_to_elem(hi.w)};
  emit_rope_quad<kPaged>(r, T, t, h * head_dim, 4 * q, head_dim, l, hh);
}

// The residual add and RMSNorm that follow a projection (x += Y, out =
// RMSNorm(x) * weight) on a split launch: one 256-thread block per token row
// sums each chunk's slices in slice order and rounds it to the element type,
// as the reduction's output, then runs the norm row on it: bit for bit the
// reduction followed by the residual RMSNorm kernel.
struct GemmNorm {
  elem_t* out;
  elem_t* x;
  const elem_t* weight;
  float eps;
};

template <int kChunks>
__global__ __launch_bounds__(kNormThreads) void gemm_reduce_norm_kernel(const float* __restrict__ partial, int splits,
                                                                        int T, int dim, GemmNorm n) {
  __shared__ float scratch[9];
  const size_t base = static_cast<size_t>(blockIdx.x) * dim;
  const size_t count = static_cast<size_t>(T) * dim;
  norm_row_vec<true, kChunks>(
      n.out + base, n.x + base, n.weight, dim, n.eps,
      [&](int c, float* df) {
        const float* p = partial + base + 8 * c;
        float4 a = *reinterpret_cast<const float4*>(p);
        float4 b = *reinterpret_cast<const float4*>(p + 4);
        for (int sl = 1; sl < splits; ++sl) {
          const float4 sa = *reinterpret_cast<const float4*>(p + static_cast<size_t>(sl) * count);
          const float4 sb = *reinterpret_cast<const float4*>(p + static_cast<size_t>(sl) * count + 4);
          a.x += sa.x; a.y += sa.y; a.z += sa.z; a.w += sa.w;
          b.x += sb.x; b.y += sb.y; b.z += sb.z; b.w += sb.w;
        }
        df[0] = round_to_elem(a.x); df[1] = round_to_elem(a.y); df[2] = round_to_elem(a.z);
        df[3] = round_to_elem(a.w); df[4] = round_to_elem(b.x); df[5] = round_to_elem(b.y);
        df[6] = round_to_elem(b.z); df[7] = round_to_elem(b.w);
      },
      scratch);
}

// Y = sum over slices of the fp32 partial products, in slice order.
template <bool kFp32Out>
__global__ __launch_bounds__(256) void gemm_reduce_kernel(void* __restrict__ Y, const float* __restrict__ partial,
                                                          int splits, size_t count) {
  const size_t i = (static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i >= count) return;
  if (i + 4 <= count) {
    float4 sum = *reinterpret_cast<const float4*>(partial + i);
    for (int s = 1; s < splits; ++s) {
      const float4 v = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(s) * count + i);
      sum.x += v.x;
      sum.y += v.y;
      sum.z += v.z;
      sum.w += v.w;
    }
    if (kFp32Out) {
      *reinterpret_cast<float4*>(static_cast<float*>(Y) + i) = sum;
    } else {
      uint2 packed;
      packed.x = pack_elems(sum.x, sum.y);
      packed.y = pack_elems(sum.z, sum.w);
      *reinterpret_cast<uint2*>(static_cast<elem_t*>(Y) + i) = packed;
    }
    return;
  }
  for (size_t e = i; e < count; ++e) {
    float sum = partial[e];
    for (int s = 1; s < splits; ++s) sum += partial[static_cast<size_t>(s) * count + e];
    if (kFp32Out) {
      static_cast<float*>(Y)[e] = sum;
    } else {
      static_cast<elem_t*>(Y)[e] = float_to_elem(sum);
    }
  }
}

enum class GemmShape { kRing256x256, kRing256x128, kRing192x128, kRing128x128, k256x256, k256x128, k128x128 };

struct GemmPlan {
  GemmShape shape;
  int bw, bt;
  int splits;
  int k_chunk;
  size_t workspace_bytes;
};

// The plan with the least estimated time. Work units (tile x K slice) run in
// whole rounds over the compute units; a unit costs its flops at the shape's
// measured fraction of a compute unit's MFMA peak. Splitting K is considered
// only when the tiles alone leave compute units idle, and costs the fp32
// partials' round trip through memory plus a launch. Each slice keeps at
// least 256 K and is a whole number of the shape's K stages. With
// wide_waves, an unsplit plan uses only shapes whose waves own 128 W rows
// (the RoPE epilogue for 128-row heads). The 192-row tile is for unsplit
// plans, and without narrow_ok for none (its RoPE epilogue needs the staged
// store).
GemmPlan plan_gemm(int T, int N, int K, int cus, size_t workspace_bytes, bool wide_waves = false,
                   bool narrow_ok = true) {
  struct Option {
    GemmShape shape;
    int bw, bt, stage_k;
    double efficiency;  // fraction of a compute unit's MFMA peak, measured on MI355X
  };
  // A ring shape needs K in whole ring stages of its depth.
  const bool ring = K % kRingK == 0;
  const bool ring256x128 = K % kRing256x128K == 0;
  const bool ring128x128 = K % kRing128x128K == 0;
  const bool ring192x128 = K % kRing192x128K == 0;
  const Option options[] = {
      {ring ? GemmShape::kRing256x256 : GemmShape::k256x256, 256, 256, ring ? kRingK : kStageK, ring ? 0.37 : 0.31},
      {ring256x128 ? GemmShape::kRing256x128 : GemmShape::k256x128, 256, 128,
       ring256x128 ? kRing256x128K : kStageK, ring256x128 ? kRing256x128Efficiency : 0.23},
      {ring128x128 ? GemmShape::kRing128x128 : GemmShape::k128x128, 128, 128,
       ring128x128 ? kRing128x128K : kStageK, ring128x128 ? kRing128x128Efficiency : 0.20},
      // ring only: the register-staged kernel has no 192-row tile
      {GemmShape::kRing192x128, 192, 128, kRing192x128K, ring192x128 ? kRing192x128Efficiency : 0.0}};
  constexpr double kCuPeak = 9.8e12;     // bf16 dense flop/s per compute unit
  constexpr double kBandwidth = 5.0e12;  // sustained bytes/s for the partials' round trip
  constexpr double kLaunch = 4e-6;
  GemmPlan best{GemmShape::k128x128, 128, 128, 1, K, 0};
  double best_time = -1.0;
  for (const Option& o : options) {
    if (o.efficiency <= 0.0) continue;
    const long long tiles = static_cast<long long>((N + o.bw - 1) / o.bw) * ((T + o.bt - 1) / o.bt);
    for (int splits = 1; splits <= 16; splits *= 2) {
      if (splits > 1 && tiles * (splits / 2) >= cus) break;  // already enough units
      const int k_chunk = ((K + splits - 1) / splits + o.stage_k - 1) / o.stage_k * o.stage_k;
      if (splits > 1 && k_chunk < 256) break;
      const int used = (K + k_chunk - 1) / k_chunk;
      if (wide_waves && used == 1 && o.bt != 256) continue;
      // 192-row tiles unsplit only: split four ways for q/k/v at 512 tokens
      // they measured slower than 128 x 128 tiles split in two
      if (o.bw == 192 && (used > 1 || !narrow_ok)) continue;
      const size_t bytes = used > 1 ? static_cast<size_t>(used) * T * N * sizeof(float) : 0;
      if (bytes > workspace_bytes) break;
      const long long rounds = (tiles * used + cus - 1) / cus;
      double time = static_cast<double>(rounds) * 2.0 * o.bw * o.bt * k_chunk / (o.efficiency * kCuPeak);
      if (used > 1) time += (static_cast<double>(bytes) + static_cast<double>(T) * N * 4.0) / kBandwidth + kLaunch;
      if (best_time < 0.0 || time < best_time) {
        best = GemmPlan{o.shape, o.bw, o.bt, used, k_chunk, bytes};
        best_time = time;
      }
    }
  }
  return best;
}

template <int BW, int BT, int kWavesW, int kWavesT>
void launch_gemm_tiles(void* Y, bool fp32_out, const elem_t* X, const elem_t* W, int T, int N, int K,
                       const GemmGrid& grid, hipStream_t s) {
  const int units = grid.tiles_t * grid.tiles_w * grid.splits;
  const unsigned blocks = static_cast<unsigned>(((units + 7) / 8) * 8);
  constexpr unsigned kThreads = 64u * kWavesW * kWavesT;
  if (fp32_out) {
    gemm_nt_kernel<BW, BT, kWavesW, kWavesT, true><<<blocks, kThreads, 0, s>>>(Y, X, W, T, N, K, grid);
  } else {
    gemm_nt_kernel<BW, BT, kWavesW, kWavesT, false><<<blocks, kThreads, 0, s>>>(Y, X, W, T, N, K, grid);
  }
}

template <int BW, int BT, int kWaves, int kStages, int kRK = kRingK>
void launch_gemm_ring(void* Y, bool fp32_out, const elem_t* X, const elem_t* W, int T, int N, int K,
                      const GemmGrid& grid, hipStream_t s) {
  const int units = grid.tiles_t * grid.tiles_w * grid.splits;
  const unsigned blocks = static_cast<unsigned>(((units + 7) / 8) * 8);
  if (fp32_out) {
    gemm_ring_kernel<kStages, kWaves, BW, BT, true, kRK><<<blocks, 64 * kWaves, 0, s>>>(Y, X, W, T, N, K, grid);
  } else {
    gemm_ring_kernel<kStages, kWaves, BW, BT, false, kRK><<<blocks, 64 * kWaves, 0, s>>>(Y, X, W, T, N, K, grid);
  }
}

// Returns whether the residual RMSNorm `norm` was applied (a split plan whose
// rows the fused reduction covers); otherwise Y holds the projection.
bool run_gemm(void* Y, bool fp32_out, const elem_t* X, const elem_t* W, int T, int N, int K, void* workspace,
              size_t workspace_bytes, int ffn, hipStream_t s, const GemmRope* rope = nullptr,
              const GemmNorm* norm = nullptr) {
  const bool wide_waves = rope != nullptr && rope->view.head_dim == 128;
  // The staged RoPE epilogue's conditions (staged_store_ok), known here.
  const bool narrow_ok =
      rope == nullptr ||
      (rope->view.head_dim == 64 &&
       ((reinterpret_cast<uintptr_t>(rope->q_heads) | reinterpret_cast<uintptr_t>(rope->view.keys) |
         reinterpret_cast<uintptr_t>(rope->view.values)) & 15u) == 0 &&
       rope->view.page_stride % 8 == 0 && rope->view.head_stride % 8 == 0);
  const GemmPlan plan = plan_gemm(T, N, K, device_compute_units(), workspace != nullptr ? workspace_bytes : 0,
                                  wide_waves, narrow_ok);
  GemmGrid grid{(T + plan.bt - 1) / plan.bt, (N + plan.bw - 1) / plan.bw, plan.splits, plan.k_chunk,
                plan.splits > 1 ? static_cast<float*>(workspace) : nullptr, ffn,
                rope != nullptr ? *rope : GemmRope{}};
  switch (plan.shape) {
    case GemmShape::kRing256x256:
      launch_gemm_ring<256, 256, kRingWaves, kRingStages>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::kRing256x128:
      launch_gemm_ring<256, 128, 8, kRing256x128Stages, kRing256x128K>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::kRing128x128:
      launch_gemm_ring<128, 128, 8, kRing128x128Stages, kRing128x128K>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::kRing192x128:
      launch_gemm_ring<192, 128, 8, kRing192x128Stages, kRing192x128K>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::k256x256:
      launch_gemm_tiles<256, 256, 2, 4>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::k256x128:
      launch_gemm_tiles<256, 128, 4, 2>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
    case GemmShape::k128x128:
      launch_gemm_tiles<128, 128, 2, 2>(Y, fp32_out, X, W, T, N, K, grid, s);
      break;
  }
  const int norm_chunks = (N / 8 + kNormThreads - 1) / kNormThreads;
  if (plan.splits > 1 && norm != nullptr && N % 8 == 0 && norm_chunks <= 4 &&
      ((reinterpret_cast<uintptr_t>(norm->out) | reinterpret_cast<uintptr_t>(norm->x) |
        reinterpret_cast<uintptr_t>(norm->weight)) & 15u) == 0) {
    const unsigned rows = static_cast<unsigned>(T);
    if (norm_chunks == 1) {
      gemm_reduce_norm_kernel<1><<<rows, kNormThreads, 0, s>>>(grid.partial, plan.splits, T, N, *norm);
    } else if (norm_chunks == 2) {
      gemm_reduce_norm_kernel<2><<<rows, kNormThreads, 0, s>>>(grid.partial, plan.splits, T, N, *norm);
    } else {
      gemm_reduce_norm_kernel<4><<<rows, kNormThreads, 0, s>>>(grid.partial, plan.splits, T, N, *norm);
    }
    return true;
  }
  if (plan.splits > 1 && rope != nullptr) {
    const size_t threads = static_cast<size_t>(T) * (N / rope->view.head_dim) * (rope->view.head_dim / 8);
    const unsigned blocks = static_cast<unsigned>((threads + 255) / 256);
    if (rope->paged) {
      gemm_reduce_rope_kernel<true><<<blocks, 256, 0, s>>>(grid.partial, plan.splits, T, N, *rope);
    } else {
      gemm_reduce_rope_kernel<false><<<blocks, 256, 0, s>>>(grid.partial, plan.splits, T, N, *rope);
    }
  } else if (plan.splits > 1 && ffn > 0) {
    const size_t count = static_cast<size_t>(T) * ffn;
    gemm_reduce_swiglu_kernel<<<static_cast<unsigned>((count + 1023) / 1024), 256, 0, s>>>(
        static_cast<elem_t*>(Y), grid.partial, plan.splits, T, ffn);
  } else if (plan.splits > 1) {
    const size_t count = static_cast<size_t>(T) * N;
    const unsigned blocks = static_cast<unsigned>((count + 1023) / 1024);
    if (fp32_out) {
      gemm_reduce_kernel<true><<<blocks, 256, 0, s>>>(Y, grid.partial, plan.splits, count);
    } else {
      gemm_reduce_kernel<false><<<blocks, 256, 0, s>>>(Y, grid.partial, plan.splits, count);
    }
  }
  return false;
}

// ---------------------------------------------------------------------------
// Prefill attention (MFMA, flash-style)
// ---------------------------------------------------------------------------

// Eight waves: the four query heads of one kv head, each over two key groups
// (the even and the odd 64-key tiles), so a block walks its keys in half the
// steps; the two groups merge their statistics and their outputs at fixed
// points, group 0 first.
constexpr int kFlashThreads = 512;
constexpr int kFlashKeys = 64;      // keys per tile; two tiles are staged per step
constexpr int kKeyGroups = 2;

// Key rows are head_dim elements with 16-byte chunk c at position
// c ^ key_swizzle(key), so the fragment reads of 16 consecutive keys are free
// of bank conflicts (measured on MI355X for 128-byte rows; 256-byte rows
// spread 16 rows over all 16 chunk positions).
template <int kHeadDim>
__device__ __forceinline__ int key_swizzle(int key) {
  return kHeadDim == 64 ? (key & 7) : (key & 15);
}

// Value rows are kept as they are in the cache (key-major) with chunk c at
// c ^ value_swizzle(key). The P.V operand is assembled by transposing reads
// (ds_read_b64_tr_b16): in each 16-lane group, lane 4k + q names 8 bytes (4
// dims) of one key row and lane 4q + c receives dim c of those 8 bytes from
// the rows named by lanes 4k + q, k = 0..3. One read covers 16 rows x 32
// bytes; with an even swizzle that takes each value twice over the rows of
// one bank half, every bank serves the same number of dwords.
template <int kHeadDim>
__device__ __forceinline__ int value_swizzle(int key) {
  return kHeadDim == 64 ? (key & 6) : ((key & 7) << 1);
}

template <int kHeadDim, int kRows>
struct FlashShared {
  static constexpr int kKeyPitch = kHeadDim;
  elem_t keys[2][kKeyGroups * kFlashKeys * kKeyPitch];    // two tiles per buffer
  elem_t values[2][kKeyGroups * kFlashKeys * kHeadDim];   // the same keys' values
  float stats[kFlashThreads / 64][kRows][2];              // per wave: row max, row sum
};

typedef short lds_v4i16 __attribute__((ext_vector_type(4)));

template <bool kPaged, int kHeadDim, int kRF>
__global__ __launch_bounds__(kFlashThreads, kHeadDim == 64 ? 4 : 2) void flash_prefill_kernel(
    elem_t* __restrict__ out, const elem_t* __restrict__ q_heads, KvCacheView view, int num_heads,
    int group, int tokens, int start_position, float scale_log2e) {
  constexpr int kRows = 16 * kRF;                         // query positions per block
  constexpr int kSteps = kHeadDim / 32;                   // MFMA k-steps over head_dim
  constexpr int kDFrags = kHeadDim / 16;                  // output fragments over head_dim
  constexpr int kPairKeys = kKeyGroups * kFlashKeys;      // keys staged per step
  constexpr int kKeyPitch = FlashShared<kHeadDim, kRows>::kKeyPitch;
  constexpr int kRowChunks = kHeadDim / 8;                // 16-byte chunks per key row
  constexpr int kLoadRows = 64 / kRowChunks;              // rows of one 1 KiB direct load
  constexpr int kWaveLoads = kPairKeys / kLoadRows / (kFlashThreads / 64);  // per wave, K or V
  static_assert(kWaveLoads * kLoadRows * (kFlashThreads / 64) == kPairKeys, "a step splits over the waves");
  static_assert(kKeyGroups * 4 == kFlashThreads / 64, "one wave per (head, key group)");
  __shared__ __attribute__((aligned(1024))) FlashShared<kHeadDim, kRows> sh;

  // XCD-aware order: XCD x (block id mod 8) takes the contiguous run of units
  // [x * per, (x + 1) * per) of the kv-head-major order, so one XCD's L2 holds
  // the keys and values of few kv heads (one, for 8 kv heads); within a head,
  // the longest rows start first.
  const int row_blocks = (tokens + kRows - 1) / kRows;
  const int units = row_blocks * view.num_kv_heads;
  const int per_xcd = (units + 7) / 8;
  const int u = static_cast<int>(blockIdx.x % 8u) * per_xcd + static_cast<int>(blockIdx.x / 8u);
  if (u >= units) return;  // the whole block: no barrier has been met
  const int kv = u / row_blocks;
  const int r0 = (row_blocks - 1 - u % row_blocks) * kRows;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int lane = lane_id();
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int kg = wave >> 2;  // key group: tiles kg, kg + 2, ...
  const int g = blockIdx.z * 4 + (wave & 3);
  const bool active = g < group;
  const int head = kv * group + (active ? g : 0);

  const int last_key = start_position + tokens - 1;
  const int block_keys = start_position + min(r0 + kRows, tokens);
  const int tiles = (block_keys + kFlashKeys - 1) / kFlashKeys;
  const int steps = (tiles + kKeyGroups - 1) / kKeyGroups;

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

  // Step `step` stages tiles 2 step and 2 step + 1 (keys 128 step .. +127)
  // by direct global-to-LDS loads, no registers between: load n of a wave
  // fills rows kLoadRows (8 n + wave) .. + kLoadRows - 1, lane i writing slot
  // i % kRowChunks of row i / kRowChunks, so the lane loads the chunk whose
  // swizzled position that slot is. Keys past the last position repeat it (the
  // scores mask them).
  const int load_row = lane / kRowChunks;
  const int load_slot = lane % kRowChunks;
  auto issue = [&](int step, int buf, bool with_values) {
#pragma unroll
    for (int n = 0; n < kWaveLoads; ++n) {
      const int block_row = kLoadRows * (8 * n + wave);
      const int row = block_row + load_row;
      const size_t at = view.offset<kPaged>(kv, min(step * kPairKeys + row, last_key));
      load_to_lds16(view.keys + at + 8 * (load_slot ^ key_swizzle<kHeadDim>(row)),
                    lds_address_of(&sh.keys[buf][block_row * kKeyPitch]));
      if (with_values) {
        load_to_lds16(view.values + at + 8 * (load_slot ^ value_swizzle<kHeadDim>(row)),
                      lds_address_of(&sh.values[buf][block_row * kHeadDim]));
      }
    }
  };
  // The A operand of O^T += V^T . P^T for dims 16 df .. + 15 and the 32 keys
  // of half `half` of this wave's tile, in the order the P^T fragments hold
  // them: k-slot 8 grp + j is key 32 half + 4 grp + j (j < 4) or
  // 32 half + 16 + 4 grp + (j - 4). Two transposing reads, one per group of
  // four keys; this lane names row 4 grp + col / 4 (+ 16) at dims
  // 16 df + 4 (col % 4) .. + 3.
  auto value_operand = [&](const elem_t* tile, int half, int df) {
    typedef __attribute__((address_space(3))) lds_v4i16* lds_v4i16_ptr;
    const int r0 = 32 * half + 4 * grp + (col >> 2);
    const int c = 2 * df + ((col & 3) >> 1);
    const int within = (col & 1) * 4;
    const int r1 = r0 + 16;
    const elem_t* p0 = tile + r0 * kHeadDim + ((c ^ value_swizzle<kHeadDim>(r0)) << 3) + within;
    const elem_t* p1 = tile + r1 * kHeadDim + ((c ^ value_swizzle<kHeadDim>(r1)) << 3) + within;
    const lds_v4i16 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(p0));
    const lds_v4i16 y = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16_ptr)(p1));
    typedef short v8i16 __attribute__((ext_vector_type(8)));
    const v8i16 both = __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(mfma_in8, both);
  };
  // Scores q . k of this wave's tile of a staged step, transposed:
  // s[rf][kf][v] is row 16rf + col against key 16kf + 4grp + v of tile
  // `tile`; keys past a row's position are -inf. The scale (in base-2 units,
  // scale * log2(e)) is applied inside the exponentials, as one fma with the
  // row max: exp2(c s - c m).
  auto scores = [&](int buf, int tile, mfma_acc4 (&s)[kRF][4]) {
    const elem_t* kb = &sh.keys[buf][kg * kFlashKeys * kKeyPitch];
#pragma unroll
    for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) s[rf][kf] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kSteps; ++ks) {
        const mfma_in8 a = lds_operand(
            kb + (kf * 16 + col) * kKeyPitch + (((ks * 4 + grp) ^ key_swizzle<kHeadDim>(col)) << 3));
#pragma unroll
        for (int rf = 0; rf < kRF; ++rf) s[rf][kf] = mfma16x16x32(a, qf[rf][ks], s[rf][kf]);
      }
    }
    const int key0 = tile * kFlashKeys;
    if (key0 + kFlashKeys - 1 > start_position + r0) {  // a tile that crosses the diagonal
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) {
        const int over = key0 + 4 * grp - (start_position + r0 + rf * 16 + col);  // key - last visible key
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            if (over + kf * 16 + v > 0) s[rf][kf][v] = -__builtin_huge_valf();
          }
        }
      }
    }
  };

  // Pass 1: per key group, row max m and sum l of exp(s - m), keys only; the
  // sum is kept per lane against a running max and rescaled when it grows.
  float m[kRF], l[kRF];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    m[rf] = -__builtin_huge_valf();
    l[rf] = 0.0f;
  }
  issue(0, 0, false);
  wait_stage_landed<0>();
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    // buf ^ 1 was last read in the previous step, before its closing barrier
    if (step + 1 < steps) issue(step + 1, buf ^ 1, false);
    const int tile = kKeyGroups * step + kg;
    if (active && tile < tiles) {
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
        // Until a row has seen a visible key in this group (group 1's first
        // tiles can be fully masked for the early rows) its max is -inf; the
        // exponentials are then taken against 0, all of them are 0, and l
        // stays 0.
        const float neg_base = m_new == -__builtin_huge_valf() ? 0.0f : -m_new * scale_log2e;
        float sum = 0.0f;
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
#pragma unroll
          for (int v = 0; v < 4; ++v) sum += __builtin_amdgcn_exp2f(__builtin_fmaf(s[rf][kf][v], scale_log2e, neg_base));
        }
        l[rf] = m[rf] == m_new ? l[rf] + sum
                               : __builtin_fmaf(l[rf], __builtin_amdgcn_exp2f(__builtin_fmaf(m[rf], scale_log2e, neg_base)), sum);
        m[rf] = m_new;
      }
    }
    wait_stage_landed<0>();
    __syncthreads();
  }
  // Merge the two key groups, group 0 first: M = max(m0, m1),
  // L = l0 exp(m0 - M) + l1 exp(m1 - M). Group 0 holds key 0, visible to every
  // row, so M is finite; a group with no visible key has m = -inf and
  // contributes 0.
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    float total = l[rf];
    total += xor_lane<16>(total);
    total += xor_lane<32>(total);
    if (grp == 0) {
      sh.stats[wave][rf * 16 + col][0] = m[rf];
      sh.stats[wave][rf * 16 + col][1] = total;
    }
  }
  __syncthreads();
  float inv[kRF];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    const int h = wave & 3;
    const float m0 = sh.stats[h][rf * 16 + col][0], l0 = sh.stats[h][rf * 16 + col][1];
    const float m1 = sh.stats[h + 4][rf * 16 + col][0], l1 = sh.stats[h + 4][rf * 16 + col][1];
    const float M = fmaxf(m0, m1);
    const float L = __builtin_fmaf(l1, __builtin_amdgcn_exp2f((m1 - M) * scale_log2e),
                                   l0 * __builtin_amdgcn_exp2f((m0 - M) * scale_log2e));
    m[rf] = -M * scale_log2e;  // pass 2 takes exp2(c s - c M) as one fma
    inv[rf] = 1.0f / L;
  }

  // Pass 2: p = exp(s - M) * (1/L) rounded to the element type, where the
  // reference rounds its probability buffer, then O^T += V^T . P^T in fp32 per
  // key group; the groups' outputs add at the end, group 0 first.
  mfma_acc4 o[kRF][kDFrags];
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
#pragma unroll
    for (int df = 0; df < kDFrags; ++df) o[rf][df] = mfma_acc4{0.f, 0.f, 0.f, 0.f};
  }
  issue(0, 0, true);
  wait_stage_landed<0>();
  __syncthreads();
  for (int step = 0; step < steps; ++step) {
    const int buf = step & 1;
    if (step + 1 < steps) issue(step + 1, buf ^ 1, true);
    const int tile = kKeyGroups * step + kg;
    if (active && tile < tiles) {
      mfma_acc4 s[kRF][4];
      scores(buf, tile, s);
      const elem_t* vt = &sh.values[buf][kg * kFlashKeys * kHeadDim];
#pragma unroll
      for (int rf = 0; rf < kRF; ++rf) {
        uint32_t pk[4][2];
#pragma unroll
        for (int kf = 0; kf < 4; ++kf) {
          float pr[4];
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            pr[v] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[rf][kf][v], scale_log2e, m[rf])) * inv[rf];
          }
          pk[kf][0] = pack_rounded(pr[0], pr[1]);
          pk[kf][1] = pack_rounded(pr[2], pr[3]);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          const vec16 pw{{pk[2 * half][0], pk[2 * half][1], pk[2 * half + 1][0], pk[2 * half + 1][1]}};
          const mfma_in8 b = as_operand(pw);
#pragma unroll
          for (int df = 0; df < kDFrags; ++df) {
            o[rf][df] = mfma16x16x32(value_operand(vt, half, df), b, o[rf][df]);
          }
        }
      }
    }
    wait_stage_landed<0>();
    __syncthreads();
  }

  // Group 1 hands its partial output to group 0 through the (now free) key
  // buffers; group 0 adds it to its own and stores.
  float* handoff = reinterpret_cast<float*>(&sh.keys[0][0]);
  static_assert(sizeof(sh.keys) >= 4 * kRF * kDFrags * 4 * 64 * sizeof(float), "handoff must fit");
  if (kg == 1) {
#pragma unroll
    for (int rf = 0; rf < kRF; ++rf) {
#pragma unroll
      for (int df = 0; df < kDFrags; ++df) {
#pragma unroll
        for (int v = 0; v < 4; ++v) handoff[((((wave & 3) * kRF + rf) * kDFrags + df) * 4 + v) * 64 + lane] = o[rf][df][v];
      }
    }
  }
  __syncthreads();
  if (!active || kg == 1) return;
  // o[rf][df][v] = O[row 16rf + col][dim 16df + 4grp + v]
#pragma unroll
  for (int rf = 0; rf < kRF; ++rf) {
    const int row = r0 + rf * 16 + col;
    if (row >= tokens) continue;
    elem_t* dst = out + static_cast<size_t>(row) * num_heads * kHeadDim +
                  static_cast<size_t>(head) * kHeadDim + 4 * grp;
#pragma unroll
    for (int df = 0; df < kDFrags; ++df) {
      float r[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) r[v] = o[rf][df][v] + handoff[((((wave & 3) * kRF + rf) * kDFrags + df) * 4 + v) * 64 + lane];
      uint2 packed;
      packed.x = pack_elems(r[0], r[1]);
      packed.y = pack_elems(r[2], r[3]);
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
  const float scale_log2e = static_cast<float>(static_cast<double>(scale) * 1.4426950408889634);
  const unsigned zs = static_cast<unsigned>((group + 3) / 4);
  // One row fragment (16 positions) per wave: more, lighter blocks (two per
  // compute unit) measured faster than two fragments per wave at every T.
  const int units = (tokens + 15) / 16 * v.num_kv_heads;
  const dim3 grid(static_cast<unsigned>((units + 7) / 8 * 8), 1u, zs);
  flash_prefill_kernel<kPaged, kHeadDim, 1><<<grid, kFlashThreads, 0, s>>>(o, q, v, num_heads, group, tokens,
                                                                          start_position, scale_log2e);
}

}  // namespace
}  // namespace lcr

using namespace lcr;

static int gemm_checks(const void* Y, const void* X, const void* W, int T, int N, int K) {
  CAPI_CHECK(T >= 0 && N >= 0 && K >= 0, "gemm needs non-negative sizes");
  if (T == 0 || N == 0) return LCR_OK;
  CAPI_CHECK(K > 0 && K % 8 == 0, "gemm needs K to be a positive multiple of 8, got " << K);
  CAPI_CHECK((reinterpret_cast<uintptr_t>(X) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(W) & 15u) == 0 &&
                 (reinterpret_cast<uintptr_t>(Y) & 15u) == 0,
             "gemm needs 16-byte aligned operands");
  return LCR_OK;
}

extern "C" int lcr_gemm(void* Y, int y_fp32, const void* X, const void* W, int T, int N, int K,
                        void* stream) {
  const int status = gemm_checks(Y, X, W, T, N, K);
  if (status != LCR_OK || T == 0 || N == 0) return status;
  run_gemm(Y, y_fp32 != 0, static_cast<const elem_t*>(X), static_cast<const elem_t*>(W), T, N, K, nullptr, 0, 0,
           static_cast<hipStream_t>(stream));
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" size_t lcr_gemm_workspace_bytes(int T, int N, int K) {
  if (T <= 0 || N <= 0 || K <= 0 || K % 8 != 0) return 0;
  return plan_gemm(T, N, K, device_compute_units(), static_cast<size_t>(-1)).workspace_bytes;
}

extern "C" int lcr_gemm_ws(void* Y, int y_fp32, const void* X, const void* W, int T, int N, int K,
                           void* workspace, size_t workspace_bytes, void* stream) {
  const int status = gemm_checks(Y, X, W, T, N, K);
  if (status != LCR_OK || T == 0 || N == 0) return status;
  CAPI_CHECK(workspace != nullptr || workspace_bytes == 0, "gemm workspace of " << workspace_bytes
                                                                               << " bytes has no pointer");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "gemm workspace must be 16-byte aligned");
  run_gemm(Y, y_fp32 != 0, static_cast<const elem_t*>(X), static_cast<const elem_t*>(W), T, N, K, workspace,
           workspace_bytes, 0, static_cast<hipStream_t>(stream));
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_gemm_swiglu_ws(void* act, const void* X, const void* W_gate_up, int T, int ffn, int K,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  CAPI_CHECK(ffn >= 0, "gemm_swiglu needs a non-negative ffn width");
  CAPI_CHECK(ffn % 16 == 0, "gemm_swiglu needs ffn to be a multiple of 16, got " << ffn);
  const int status = gemm_checks(act, X, W_gate_up, T, 2 * ffn, K);
  if (status != LCR_OK || T == 0 || ffn == 0) return status;
  CAPI_CHECK(workspace != nullptr || workspace_bytes == 0, "gemm workspace of " << workspace_bytes
                                                                               << " bytes has no pointer");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "gemm workspace must be 16-byte aligned");
  run_gemm(act, false, static_cast<const elem_t*>(X), static_cast<const elem_t*>(W_gate_up), T, 2 * ffn, K,
           workspace, workspace_bytes, ffn, static_cast<hipStream_t>(stream));
  CAPI_LAUNCHED();
  return LCR_OK;
}

extern "C" int lcr_gemm_residual_rmsnorm_ws(void* out, void* x, void* delta, const void* X, const void* W,
                                            const void* weight, int T, int N, int K, float eps, void* workspace,
                                            size_t workspace_bytes, void* stream) {
  const int status = gemm_checks(delta, X, W, T, N, K);
  if (status != LCR_OK || T == 0 || N == 0) return status;
  CAPI_CHECK(out != nullptr && x != nullptr && weight != nullptr,
             "gemm_residual_rmsnorm needs the output, the residual and the norm weight");
  CAPI_CHECK(workspace != nullptr || workspace_bytes == 0, "gemm workspace of " << workspace_bytes
                                                                               << " bytes has no pointer");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "gemm workspace must be 16-byte aligned");
  const GemmNorm norm{static_cast<elem_t*>(out), static_cast<elem_t*>(x), static_cast<const elem_t*>(weight), eps};
  const bool fused = run_gemm(delta, false, static_cast<const elem_t*>(X), static_cast<const elem_t*>(W), T, N, K,
                              workspace, workspace_bytes, 0, static_cast<hipStream_t>(stream), nullptr, &norm);
  CAPI_LAUNCHED();
  if (fused) return LCR_OK;
  return lcr_add_residual_rmsnorm(out, x, delta, weight, T, N, eps, stream);
}

extern "C" int lcr_gemm_qkv_rope_ws(void* q_heads, const lcr_kv_view* view, const void* X, const void* W_qkv,
                                    const float* rope_table, int T, int num_heads, int K, int start_position,
                                    int paged, void* workspace, size_t workspace_bytes, void* stream) {
  CAPI_CHECK(view != nullptr, "gemm_qkv_rope needs a cache view");
  CAPI_CHECK(num_heads >= 0 && view->num_kv_heads >= 0 && start_position >= 0,
             "gemm_qkv_rope needs non-negative head counts and start position");
  const int head_dim = view->head_dim;
  CAPI_CHECK(head_dim == 64 || head_dim == 128, "gemm_qkv_rope supports head_dim 64 or 128, got " << head_dim);
  const long long n = static_cast<long long>(num_heads + 2 * view->num_kv_heads) * head_dim;
  CAPI_CHECK(n <= INT32_MAX, "gemm_qkv_rope output width " << n << " is too large");
  const int N = static_cast<int>(n);
  const int status = gemm_checks(q_heads, X, W_qkv, T, N, K);
  if (status != LCR_OK || T == 0 || N == 0) return status;
  CAPI_CHECK(rope_table != nullptr && (reinterpret_cast<uintptr_t>(rope_table) & 15u) == 0,
             "gemm_qkv_rope needs a 16-byte aligned RoPE table");
  CAPI_CHECK(view->num_kv_heads == 0 ||
                 (view->keys != nullptr && view->values != nullptr &&
                  (reinterpret_cast<uintptr_t>(view->keys) & 7u) == 0 &&
                  (reinterpret_cast<uintptr_t>(view->values) & 7u) == 0),
             "gemm_qkv_rope needs 8-byte aligned cache keys and values");
  CAPI_CHECK(view->page_stride % 4 == 0 && view->head_stride % 4 == 0,
             "gemm_qkv_rope needs cache strides in whole 8-byte groups");
  CAPI_CHECK(!paged || view->page_table != nullptr, "a paged cache view needs a page table");
  CAPI_CHECK(!paged || view->page_size > 0, "a paged cache view needs a positive page size");
  CAPI_CHECK(workspace != nullptr || workspace_bytes == 0, "gemm workspace of " << workspace_bytes
                                                                               << " bytes has no pointer");
  CAPI_CHECK((reinterpret_cast<uintptr_t>(workspace) & 15u) == 0, "gemm workspace must be 16-byte aligned");
  GemmRope rope{};
  rope.table = reinterpret_cast<const float2*>(rope_table);
  rope.q_heads = static_cast<elem_t*>(q_heads);
  rope.view = KvCacheView::from_c(*view);
  rope.start_position = start_position;
  rope.q_dim = num_heads * head_dim;
  rope.paged = paged != 0 ? 1 : 0;
  run_gemm(nullptr, false, static_cast<const elem_t*>(X), static_cast<const elem_t*>(W_qkv), T, N, K, workspace,
           workspace_bytes, 0, static_cast<hipStream_t>(stream), &rope);
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
