// Split-K GQA decode attention for one query token, as a device routine shared
// by the standalone launcher and the fused decode step.
//
// Work split. One 512-thread block (8 waves) per (split, query heads): either
// one query head (short contexts: the most, lightest blocks) or the whole GQA
// group sharing a kv head (long contexts: each key/value loaded once for all
// the group's heads). Split s covers positions
// [s*chunk, min(seq_len, (s+1)*chunk)) with chunk = ceil(seq_len / splits), as
// in the reference (src/kernels/attention.cu:129-133). The range is cut into
// tiles of 64 positions; wave w takes tiles w, w+8, w+16, ... . Every value
// below belongs to one query head and no operation mixes heads, so how heads
// are grouped into blocks cannot change a result.
//
// Tile layout. A position's key (or value) is head_dim/8 = P chunks of 16
// bytes. Lane L holds chunk j = L % P of positions i*(64/P) + L/P for
// i = 0..P-1, so each load instruction of the wave reads 64 consecutive chunks
// (1 KiB contiguous in the contiguous layout, whole 16-position page runs in
// the paged one). A wave requests its next tile before it works on the current
// one (positions past the range are clamped to the last valid one for the
// address and zeroed before use), so at most one load latency is exposed.
//
// Arithmetic, in this exact order (the CPU oracle repeats it):
//  1. q is multiplied by `scale` in fp32 (the reference folds the scale into q,
//     attention.cu:138-145).
//  2. Partial dot of lane L for position i: d = sum over the 8 elements of its
//     chunk, d = fma(q, k, d) from d = 0.
//  3. The P partials of a position are added by a butterfly over the P lanes
//     holding it (offsets P/2, ..., 1), run as a reduce-scatter: afterwards lane
//     L owns the score of position index (L % P)*(64/P) + L/P of the tile.
//     Positions past the end of the range get score -FLT_MAX.
//  4. Per tile: M = max(m, max over the wave of the scores); r = exp(m - M);
//     p = exp(s - M) for the owned position; l_lane = fma(l_lane, r, p); m = M.
//  5. The p of the tile go through LDS so lane L reads the P probabilities of
//     the positions it holds values for, and for each element e:
//     acc = acc * r, then acc = fma(p_i, v_i[e], acc) for i = 0..P-1.
//  6. After its last tile a wave adds acc over the lanes holding the same chunk
//     (butterfly offsets 32, ..., P) and l over all 64 lanes (offsets 32..1).
//  7. The 8 waves merge max first: M = max of the wave maxima m_w,
//     c_w = exp(m_w - M), L = sum over w = 0..7 of fma(l_w, c_w, L) and
//     acc = sum over w of fma(c_w, acc_w, acc), both from 0 in wave order.
//     (The reference folds the waves one at a time with softmax_combine,
//     reduce.cuh:45-52; taking the maximum first gives the same value with one
//     exponential per wave instead of a dependent chain.)
//  8. splits == 1: out = rne(acc * (1 / L)). Otherwise the block writes
//     (M, L, acc[head_dim]) to partials[head][split] and the merge combines the
//     splits 0..splits-1 the same way as step 7: M = max m_s, c_s = exp(m_s - M),
//     L and sum accumulated in split order, out = rne(sum * (1 / L)).
#pragma once

#include <type_traits>

#include "../kv_cache.h"
#include "device_common.h"
#include "exchange.h"

namespace lcr {

constexpr int kAttnWaves = 8;
constexpr int kAttnThreads = 64 * kAttnWaves;
constexpr int kAttnTile = 64;
constexpr int kPartialHeader = 2;
constexpr int kMaxSplits = 64;

// Softmax combine of the reference (reduce.cuh:45-52) with the product order
// fixed: l = fma(l, exp(m - M), other_l * exp(other_m - M)). Used by the
// prefill-side causal softmax.
__host__ __device__ __forceinline__ void softmax_combine(float* m, float* l, float other_m,
                                                         float other_l) {
  const float merged = fmaxf(*m, other_m);
  *l = __builtin_fmaf(*l, lcr_expf(*m - merged), other_l * lcr_expf(other_m - merged));
  *m = merged;
}

// Positions whose cache addresses a block of the paged layout keeps in LDS
// (16 KiB): a split longer than this is walked in windows of that many
// positions (64 tiles, so every wave keeps its tiles and their order).
constexpr int kAttnPositionTable = 4096;

template <bool kPaged, int kHeadDim, int kHeads>
struct AttnShared {
  float probs[kAttnWaves][64 * kHeads];
  float wave_m[kAttnWaves][kHeads];
  float wave_l[kAttnWaves][kHeads];
  float wave_acc[kAttnWaves][kHeads][kHeadDim];
  // Paged layout: the 16-byte-chunk index of position begin + i of the
  // block's range (chunk 0 of that position's key and value rows).
  uint32_t chunks[kPaged ? kAttnPositionTable : 1];
};

// What a block that runs inside the q/k/v projection's grid takes from it
// (exchange.h): its queries and, when its range holds the new position
// (take_kv), that position's key and value; plus LDS for them once taken.
//  - consume words (one head, one split): 3 * head_dim words (query, key,
//    value) at `words`, one reader each, cleared when read;
//  - broadcast words (`broadcast`; any split, one head or the whole group):
//    the queries of the block's heads at q_words (head after head), the key
//    at k_words and the value at v_words, tagged `tag`.
template <int kHeadDim>
struct AttnExchange {
  unsigned long long* words;
  bool broadcast;
  unsigned long long* q_words;
  unsigned long long* k_words;
  unsigned long long* v_words;
  bool take_kv;
  int spins;
  int* status;
  float* q_lds;                  // [heads][kHeadDim] LDS
  // Take the queries before requesting the first tiles rather than after:
  // for a block that computed q/k/v rows first, whose queries are mostly
  // published by then. Loads complete in issue order, so a wait issued behind
  // both of a wave's tiles holds every wave until both have landed; taken
  // first, the wave starts on its first tile while the second is in flight.
  bool early_wait = false;
  elem_t* kv_lds;                // [2][kHeadDim] LDS, 16-byte aligned
  // When set, the head's output also goes out as broadcast words, two
  // elements each (element 2i in the low half), tagged `tag`, at
  // out_words[(head * kHeadDim) / 2 + i]: for the o_proj blocks of the grid.
  unsigned long long* out_words;
  uint32_t tag;
};

// No prologue work.
struct NoPreWait {
  __device__ void operator()() const {}
};

// Step 3's reduce-scatter: at offset O the lane keeps the half of its N values
// whose position-index bit matches its own lane bit and adds the partner's
// copy of that half.
template <int O, int N>
__device__ __forceinline__ void reduce_scatter(float* vals, int lane) {
  const bool upper = (lane & O) != 0;
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const float lo = vals[k];
    const float hi = vals[k + N / 2];
    const float send = upper ? lo : hi;
    const float keep = upper ? hi : lo;
    vals[k] = keep + xor_lane<O>(send);
  }
  if constexpr (O > 1) reduce_scatter<O / 2, N / 2>(vals, lane);
}

// Step 6's sum over the lanes holding the same chunk: offsets 32, 16, ..., P.
template <int P>
__device__ __forceinline__ float sum_over_groups(float v) {
  v += xor_lane<32>(v);
  if constexpr (P <= 16) v += xor_lane<16>(v);
  if constexpr (P <= 8) v += xor_lane<8>(v);
  return v;
}

template <bool B>
using attn_flag = std::integral_constant<bool, B>;

// One block: query heads head0 .. head0 + kHeads - 1 (all reading kv head
// `kv_head`) over split `split` of `splits` (split < splits). One head per
// block gives short contexts the most blocks; a whole GQA group per block
// loads each key/value once for all its heads, which is what long contexts,
// bound by the cache bytes, need. `q` holds num_heads * kHeadDim elements
// (head h at h * kHeadDim). Writes out (splits == 1) or partials[head][split].
//
// Addressing. A lane's key and value chunks of a position share one 16-byte
// index (32 bits: a layer view spans at most 64 GiB), computed once per tile
// for both. In the paged layout the block first stores the index of every
// position of its range (or of the current window of it) in LDS, one
// page-table read and division per position, all issued together, so no tile
// waits on a page-table load: loads return in issue order, and a table load
// issued after a tile's keys would hold the next tile's requests until those
// keys were in. Tiles whose 64 positions are all in range skip the masking
// selects.
//
// kExchange: the block runs inside the q/k/v projection's grid. Its queries
// and the new position's key and value are not in memory yet. It first runs
// `prologue` (work of its own for the grid, every thread, before its own
// registers fill), issues its first tiles' cache loads, then takes the
// queries and the new key and value from exchange words (`x`), and uses the
// taken key and value in place of the cache's for position seq_len - 1. The
// arithmetic is unchanged.
template <bool kPaged, int kHeadDim, int kHeads, bool kExchange = false, typename Prologue = NoPreWait>
__device__ __forceinline__ void decode_attention_block(
    AttnShared<kPaged, kHeadDim, kHeads>& sh, elem_t* __restrict__ out,
    float* __restrict__ partials, const elem_t* __restrict__ q, const KvCacheView& view,
    int kv_head, int head0, int split, int splits, int seq_len, float scale,
    const AttnExchange<kHeadDim>* x = nullptr, Prologue prologue = Prologue{}) {
  constexpr int P = kHeadDim / 8;   // chunks per position
  constexpr int Q = 64 / P;         // positions per load instruction
  constexpr int G = kHeads;
  static_assert(!kExchange || P <= 8, "exchange blocks take head_dim <= 64");
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const int j = lane % P;
  const int a = lane / P;

  if constexpr (kExchange) prologue();
  const int chunk = (seq_len + splits - 1) / splits;
  const int begin = split * chunk;
  const int end = min(seq_len, begin + chunk);
  const int length = max(0, end - begin);
  // Positions [begin + window, begin + window + window_len) are addressed
  // through the table.
  // One thread per page of the window: a single page-table read, then the
  // index of each of the page's positions in the window.
  auto fill_table = [&](int window) {
    const int window_len = min(kAttnPositionTable, length - window);
    if (window_len <= 0) return;  // an empty split reads no page-table entry
    const int first = begin + window;                      // first position of the window
    const int first_page = first / view.page_size;
    const int pages = (first + window_len - 1) / view.page_size - first_page + 1;
    const uint32_t head_chunk8 = static_cast<uint32_t>(
        (static_cast<size_t>(kv_head) * static_cast<size_t>(view.head_stride)) / 8);
    for (int pi = static_cast<int>(threadIdx.x); pi < pages; pi += kAttnThreads) {
      const int page = first_page + pi;
      const uint32_t base = static_cast<uint32_t>(
          (static_cast<size_t>(view.page_table[page]) * static_cast<size_t>(view.page_stride)) / 8) +
          head_chunk8;
      const int lo = max(page * view.page_size, first);
      const int hi = min((page + 1) * view.page_size, first + window_len);
      for (int pos = lo; pos < hi; ++pos) {
        sh.chunks[pos - first] =
            base + static_cast<uint32_t>(pos - page * view.page_size) * static_cast<uint32_t>(P);
      }
    }
  };
  if constexpr (kPaged) fill_table(0);

  float qv[G][8];
  if constexpr (!kExchange) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const vec16 raw = load16(q + static_cast<size_t>(head0 + g) * kHeadDim + 8 * j);
      unpack8(raw, qv[g]);
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[g][e] *= scale;
    }
  }
  // kExchange: wave 0 takes the query and the new key and value from the
  // exchange words into LDS; after the barrier every lane reads its query
  // chunk. Every wave calls this exactly once: after its first tile's loads,
  // or before them with x->early_wait.
  auto exchange_wait = [&]() {
    if constexpr (kExchange) {
      static_assert(kHeadDim % 64 == 0, "exchange blocks take whole waves of words");
      // Word i of what wave 0 takes: the queries, then the key, then the value.
      auto keep = [&](int i, float v) {
        if (i < G * kHeadDim) {
          x->q_lds[i] = v;
        } else {
          x->kv_lds[i - G * kHeadDim] = float_to_elem(v);
        }
      };
      if (wave == 0) {
        if (!x->broadcast) {
          constexpr int N = 3 * kHeadDim / 64;
          float vals[N];
          exchange_take<N>(x->words, vals, x->spins, x->status);
#pragma unroll
          for (int k = 0; k < N; ++k) keep(lane + 64 * k, vals[k]);
        } else {
          constexpr int NQ = G * kHeadDim / 64;
          constexpr int NKV = 2 * kHeadDim / 64;
          auto address = [&](int k) {
            const int i = lane + 64 * k;
            return i < G * kHeadDim ? x->q_words + i
                                    : (i < G * kHeadDim + kHeadDim ? x->k_words + (i - G * kHeadDim)
                                                                   : x->v_words + (i - G * kHeadDim - kHeadDim));
          };
          if (x->take_kv) {
            uint32_t bits[NQ + NKV];
            exchange_wait_tagged_at<NQ + NKV>(address, x->tag, bits, x->spins, x->status);
#pragma unroll
            for (int k = 0; k < NQ + NKV; ++k) keep(lane + 64 * k, __uint_as_float(bits[k]));
          } else {
            uint32_t bits[NQ];
            exchange_wait_tagged_at<NQ>(address, x->tag, bits, x->spins, x->status);
#pragma unroll
            for (int k = 0; k < NQ; ++k) keep(lane + 64 * k, __uint_as_float(bits[k]));
          }
        }
      }
      __syncthreads();
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[g][e] = x->q_lds[g * kHeadDim + 8 * j + e] * scale;
      }
    }
  };
  // kExchange: position seq_len - 1 comes from the exchange, not from the
  // cache, whose copy its producer may not have written yet. It is the last
  // position of the range of the block that takes it (take_kv): the lanes
  // holding it overwrite their chunk of the tile that contains it (the last
  // tile of the range, the last one its wave processes, so no later load of
  // that wave is still in flight).
  auto patch_new = [&](int tile, vec16 (&kr)[P], vec16 (&vr)[P]) {
    if constexpr (kExchange) {
      const int idx = length - 1;
      if (!x->take_kv || tile != idx / kAttnTile) return;
      const int in_tile = idx % kAttnTile;
#pragma unroll
      for (int i = 0; i < P; ++i) {
        if (i * Q + a == in_tile) {
          kr[i] = load16(x->kv_lds + 8 * j);
          vr[i] = load16(x->kv_lds + kHeadDim + 8 * j);
        }
      }
    }
  };

  float m[G], l_lane[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = kSoftmaxIdentity;
    l_lane[g] = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.0f;
  }
  if constexpr (kPaged) __syncthreads();

  // 16-byte index of this lane's chunk of the P positions it holds in tile
  // `tile` (positions past the range are clamped to the last valid one, so
  // every tile issues the same loads); `window` is the table's first position.
  const uint32_t head_chunk = kPaged ? 0u : static_cast<uint32_t>(
      (static_cast<size_t>(kv_head) * static_cast<size_t>(view.head_stride)) / 8);
  auto tile_chunks = [&](int tile, int window, uint32_t (&o)[P]) {
    const int tile_begin = tile * kAttnTile;
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const int idx = min(tile_begin + i * Q + a, length - 1);
      uint32_t c;
      if constexpr (kPaged) {
        c = sh.chunks[idx - window];
      } else {
        c = head_chunk + static_cast<uint32_t>(begin + idx) * P;
      }
      o[i] = c + static_cast<uint32_t>(j);
    }
  };
  // A block serving the whole GQA group reads each key and value once, so
  // those loads are marked non-temporal (32768 positions: 25.5 -> 23.4 us per
  // layer); per-head blocks share them through L2 and keep plain loads.
  auto load_chunks = [&](const elem_t* base, const uint32_t (&o)[P], vec16 (&r)[P]) {
#pragma unroll
    for (int i = 0; i < P; ++i) {
      if constexpr (G > 1) {
        r[i] = load16_stream(base + 8 * static_cast<size_t>(o[i]));
      } else {
        r[i] = load16(base + 8 * static_cast<size_t>(o[i]));
      }
    }
  };

  // Steps 2-4 for one tile: scores, the online softmax update, and the
  // probabilities into LDS; leaves r[] for step 5.
  float r[G];
  auto score_tile = [&](int count, const vec16 (&kr)[P], auto full) {
    constexpr bool kFull = decltype(full)::value;
    // Step 2: partial dots (positions past the range contribute zeros), value
    // index i * G + g.
    float vals[P * G];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool keep = kFull || i * Q + a < count;
      float kf[8];
      unpack8(kr[i], kf);
      if constexpr (!kFull) {
#pragma unroll
        for (int e = 0; e < 8; ++e) kf[e] = keep ? kf[e] : 0.0f;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float d = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d = __builtin_fmaf(qv[g][e], kf[e], d);
        vals[i * G + g] = d;
      }
    }
    // Step 3.
    reduce_scatter<P / 2, P * G>(vals, lane);
    const int own = j * Q + a;  // owned position index within the tile
    // Step 4.
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = (kFull || own < count) ? vals[g] : kSoftmaxIdentity;
      const float mnew = fmaxf(m[g], wave_max(s));
      r[g] = lcr_expf(m[g] - mnew);
      const float p = lcr_expf(s - mnew);
      l_lane[g] = __builtin_fmaf(l_lane[g], r[g], p);
      m[g] = mnew;
      sh.probs[wave][lane * G + g] = p;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // Step 5 for one tile.
  auto value_tile = [&](int count, const vec16 (&vr)[P], auto full) {
    constexpr bool kFull = decltype(full)::value;
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[g][e] = acc[g][e] * r[g];
    }
    const float* pr = &sh.probs[wave][a * P * G];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool keep = kFull || i * Q + a < count;
      float vf[8];
      unpack8(vr[i], vf);
      if constexpr (!kFull) {
#pragma unroll
        for (int e = 0; e < 8; ++e) vf[e] = keep ? vf[e] : 0.0f;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float pi = pr[i * G + g];
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[g][e] = __builtin_fmaf(pi, vf[e], acc[g][e]);
      }
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  // The single-head tile, steps 2-5 in one pass (the same arithmetic as
  // score_tile + value_tile, in the instruction order that runs fastest for
  // the latency-bound short-context case).
  auto process_tile = [&](int count, const vec16 (&kr)[P], const vec16 (&vr)[P], auto full) {
    constexpr bool kFull = decltype(full)::value;
    float vals[P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool keep = kFull || i * Q + a < count;
      float kf[8];
      unpack8(kr[i], kf);
      float d = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e) d = __builtin_fmaf(qv[0][e], keep ? kf[e] : 0.0f, d);
      vals[i] = d;
    }
    reduce_scatter<P / 2, P>(vals, lane);
    const int own = j * Q + a;
    const float s = (kFull || own < count) ? vals[0] : kSoftmaxIdentity;
    const float mnew = fmaxf(m[0], wave_max(s));
    const float rr = lcr_expf(m[0] - mnew);
    const float p = lcr_expf(s - mnew);
    l_lane[0] = __builtin_fmaf(l_lane[0], rr, p);
    m[0] = mnew;
    sh.probs[wave][lane] = p;
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[0][e] = acc[0][e] * rr;
    const float* pr = &sh.probs[wave][a * P];
#pragma unroll
    for (int i = 0; i < P; ++i) {
      const bool keep = kFull || i * Q + a < count;
      float vf[8];
      unpack8(vr[i], vf);
      const float pi = pr[i];
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[0][e] = __builtin_fmaf(pi, keep ? vf[e] : 0.0f, acc[0][e]);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  auto tile_count = [&](int tile) { return min(kAttnTile, length - tile * kAttnTile); };

  // Tiles wave, wave + 8, ... of the window [first_tile, last_tile). Up to
  // two heads per block with head_dim <= 64: two register sets, the next
  // tile's loads in flight while the current one is processed. Four heads
  // per block need their registers for the heads (and head_dim 128 needs
  // them for its tile), so they keep one set and refill the keys as soon as
  // the scores are taken and the values as soon as they are used.
  // `waits` (compile-time): this window is the first, whose tiles take the
  // exchange wait (a separate instance, so later windows hold nothing for it).
  auto run_tiles = [&](int first_tile, int last_tile, int window, auto waits) {
    constexpr bool kWaits = decltype(waits)::value;
    if (first_tile + wave >= last_tile) {
      if constexpr (kWaits) exchange_wait();
      return;
    }
    if constexpr (G <= 2 && P <= 8) {
      auto process = [&](int tile, const vec16 (&kr)[P], const vec16 (&vr)[P]) {
        const int count = tile_count(tile);
        if constexpr (G == 1) {
          if (count == kAttnTile) {
            process_tile(count, kr, vr, attn_flag<true>{});
          } else {
            process_tile(count, kr, vr, attn_flag<false>{});
          }
        } else if (count == kAttnTile) {
          score_tile(count, kr, attn_flag<true>{});
          value_tile(count, vr, attn_flag<true>{});
        } else {
          score_tile(count, kr, attn_flag<false>{});
          value_tile(count, vr, attn_flag<false>{});
        }
      };
      vec16 ka[P], va[P], kb[P], vb[P];
      uint32_t o[P];
      int tile = first_tile + wave;
      bool first = kWaits;
      if constexpr (kWaits) {
        if (x->early_wait) {
          exchange_wait();
          first = false;
        }
      }
      tile_chunks(tile, window, o);
      load_chunks(view.keys, o, ka);
      load_chunks(view.values, o, va);
      while (true) {
        const int t1 = tile + kAttnWaves;
        const bool more1 = t1 < last_tile;
        if (more1) {
          tile_chunks(t1, window, o);
          load_chunks(view.keys, o, kb);
          load_chunks(view.values, o, vb);
        }
        if (first) {
          exchange_wait();
          first = false;
        }
        patch_new(tile, ka, va);
        process(tile, ka, va);
        if (!more1) break;
        const int t2 = t1 + kAttnWaves;
        const bool more2 = t2 < last_tile;
        if (more2) {
          tile_chunks(t2, window, o);
          load_chunks(view.keys, o, ka);
          load_chunks(view.values, o, va);
        }
        patch_new(t1, kb, vb);
        process(t1, kb, vb);
        if (!more2) break;
        tile = t2;
      }
    } else {
      vec16 kr[P], vr[P];
      uint32_t o[P];
      int tile = first_tile + wave;
      if constexpr (kWaits) {
        if (x->early_wait) exchange_wait();
      }
      tile_chunks(tile, window, o);
      load_chunks(view.keys, o, kr);
      load_chunks(view.values, o, vr);
      if constexpr (kWaits) {
        if (!x->early_wait) exchange_wait();
      }
      while (true) {
        const int next = tile + kAttnWaves;
        const bool more = next < last_tile;
        const int count = tile_count(tile);
        const bool full = count == kAttnTile;
        patch_new(tile, kr, vr);
        if (full) {
          score_tile(count, kr, attn_flag<true>{});
        } else {
          score_tile(count, kr, attn_flag<false>{});
        }
        if (more) {
          tile_chunks(next, window, o);
          load_chunks(view.keys, o, kr);
        }
        if (full) {
          value_tile(count, vr, attn_flag<true>{});
        } else {
          value_tile(count, vr, attn_flag<false>{});
        }
        if (!more) break;
        // head_dim 128 recomputes the indices rather than keeping 16 of them
        // live across the value products
        if constexpr (P > 8) tile_chunks(next, window, o);
        load_chunks(view.values, o, vr);
        tile = next;
      }
    }
  };
  const int tiles = (length + kAttnTile - 1) / kAttnTile;
  if constexpr (kPaged) {
    constexpr int kWindowTiles = kAttnPositionTable / kAttnTile;
    if (tiles > 0) run_tiles(0, min(tiles, kWindowTiles), 0, attn_flag<kExchange>{});
    for (int first = kWindowTiles; first < tiles; first += kWindowTiles) {
      __syncthreads();  // every wave is done with the previous window's table
      fill_table(first * kAttnTile);
      __syncthreads();
      run_tiles(first, min(tiles, first + kWindowTiles), first * kAttnTile, attn_flag<false>{});
    }
  } else {
    run_tiles(0, tiles, 0, attn_flag<kExchange>{});
  }

  // Step 6.
#pragma unroll
  for (int g = 0; g < G; ++g) {
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = sum_over_groups<P>(acc[g][e]);
    l_lane[g] = wave_sum(l_lane[g]);
  }
  if (lane < P) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) sh.wave_acc[wave][g][8 * lane + e] = acc[g][e];
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      sh.wave_m[wave][g] = m[g];
      sh.wave_l[wave][g] = l_lane[g];
    }
  }
  __syncthreads();

  // Step 7, inside each wave: a head's outputs are whole waves (kHeadDim is
  // a multiple of 64), and every lane of such a wave takes the maximum of the
  // head's wave maxima; lane w computes c_w, which the wave's lanes read by
  // readlane. No barrier separates the factors from the outputs.
  static_assert(kHeadDim % 64 == 0 && kAttnWaves <= 64, "a head's outputs are whole waves");
  for (int idx = threadIdx.x; idx < G * kHeadDim; idx += kAttnThreads) {
    const int g = idx / kHeadDim;
    const int d = idx % kHeadDim;
    float tm = sh.wave_m[0][g];
#pragma unroll
    for (int v = 1; v < kAttnWaves; ++v) tm = fmaxf(tm, sh.wave_m[v][g]);
    const float c_lane = lcr_expf(sh.wave_m[lane % kAttnWaves][g] - tm);
    float tl = 0.0f, merged = 0.0f;
#pragma unroll
    for (int w = 0; w < kAttnWaves; ++w) {
      const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(c_lane), w));
      tl = __builtin_fmaf(sh.wave_l[w][g], c, tl);
      merged = __builtin_fmaf(c, sh.wave_acc[w][g][d], merged);
    }
    const int head = head0 + g;
    if (splits == 1) {
      const elem_t e = float_to_elem(merged * (1.0f / tl));
      out[static_cast<size_t>(head) * kHeadDim + d] = e;
      if constexpr (kExchange) {
        // kHeadDim is a multiple of 64, so a lane and its odd neighbour hold
        // outputs d and d + 1 of the same wave.
        const uint32_t bits = e.bits;
        // lane + 1's bits (DPP row_shl:1; the even lanes that use it read
        // inside their row of 16)
        const uint32_t next = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(0, static_cast<int>(bits), 0x101, 0xF, 0xF, true));
        if (x->out_words != nullptr && (d & 1) == 0) {
          exchange_put_tagged(x->out_words + (static_cast<size_t>(head) * kHeadDim + d) / 2, x->tag,
                              bits | (next << 16));
        }
      }
    } else {
      float* slot = partials + (static_cast<size_t>(head) * splits + split) * (kPartialHeader + kHeadDim);
      if (d == 0) {
        slot[0] = tm;
        slot[1] = tl;
      }
      slot[kPartialHeader + d] = merged;
    }
  }
}

// Merge of the split partials of one query head (step 8), by a block of
// exactly kMergeThreads threads. The partials are first copied into LDS with every
// thread loading (they come from other XCDs' writes, so each load is a trip to
// the memory side; issued together they cost one such trip, not one per
// split), then folded from LDS in split order.
constexpr int kMergeThreads = 256;
constexpr int kMaxHeadDim = 128;
constexpr int kMergeLdsFloats = kMaxSplits * (kPartialHeader + kMaxHeadDim) + kMaxSplits;
static_assert(kMaxSplits <= 64, "the merge takes the maximum over the splits in one wave");

//
// A block of more than kMergeThreads threads may run it: the others only pass
// the barriers and take part in the output loop. With `out_words`, the output
// also goes out as broadcast words, two elements each, tagged `tag`, at
// out_words[(head * head_dim) / 2 + i] (head_dim a multiple of 64).
__device__ __forceinline__ void merge_split_partials(elem_t* __restrict__ out,
                                                     const float* __restrict__ partials, int head,
                                                     int splits, int head_dim, float* lds,
                                                     unsigned long long* out_words = nullptr, uint32_t tag = 0) {
  const int stride = kPartialHeader + head_dim;
  const float* base = partials + static_cast<size_t>(head) * splits * stride;
  const int n = splits * stride;
  // Every load is issued before the first LDS store: a loop of load-then-
  // store would wait out one memory round trip per iteration.
  constexpr int kPer = (kMaxSplits * (kPartialHeader + kMaxHeadDim) + kMergeThreads - 1) / kMergeThreads;
  if (threadIdx.x < kMergeThreads) {
    float staged[kPer];
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = static_cast<int>(threadIdx.x) + k * kMergeThreads;
      staged[k] = i < n ? base[i] : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < kPer; ++k) {
      const int i = static_cast<int>(threadIdx.x) + k * kMergeThreads;
      if (i < n) lds[i] = staged[k];
    }
  }
  __syncthreads();
  float* c = lds + kMaxSplits * (kPartialHeader + kMaxHeadDim);
  if (threadIdx.x < 64) {
    // The maximum over the splits by one wave (splits <= 64; a maximum does
    // not depend on the order it is taken in).
    const int s = threadIdx.x;
    const float ms = s < splits ? lds[s * stride] : kSoftmaxIdentity;
    const float tm = wave_max(ms);
    if (s < splits) c[s] = lcr_expf(ms - tm);
  }
  __syncthreads();
  for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
    float tl = 0.0f, sum = 0.0f;
#pragma unroll 8
    for (int s = 0; s < splits; ++s) {
      tl = __builtin_fmaf(lds[s * stride + 1], c[s], tl);
      sum = __builtin_fmaf(c[s], lds[s * stride + kPartialHeader + d], sum);
    }
    const elem_t e = float_to_elem(sum * (1.0f / tl));
    out[static_cast<size_t>(head) * head_dim + d] = e;
    if (out_words != nullptr) {
      // d and d + 1 are neighbouring lanes of one wave (whole waves of d).
      const uint32_t bits = e.bits;
      const uint32_t next = static_cast<uint32_t>(
          __builtin_amdgcn_update_dpp(0, static_cast<int>(bits), 0x101, 0xF, 0xF, true));  // lane + 1 (row_shl:1)
      if ((d & 1) == 0) {
        exchange_put_tagged(out_words + (static_cast<size_t>(head) * head_dim + d) / 2, tag, bits | (next << 16));
      }
    }
  }
  __syncthreads();
}

}  // namespace lcr
