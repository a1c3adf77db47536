// The fused decode step (see decode_step.h for what is fused and why the
// results equal the unfused sequence bit for bit).
#include <algorithm>
#include <cmath>

#include "../hip_utils.h"
#include "attention_decode.h"
#include "decode_step.h"
#include "exchange.h"
#include "gemv_core.h"
#include "row_norm.h"
#include "sampling.h"

namespace lcr {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kLmHeadMaxBlocks = 1024;
// Output-head grids of up to this many blocks fold the argmax into block 0.
constexpr int kLmHeadFoldMaxBlocks = 256;
constexpr int kLmHeadRows = 2;  // rows per wave per group
// Waves per output-head block (at least kThreads / 64: the norm's threads).
// Measured on the whole step (two rounds): 4 waves 0.5245 / 0.5246 ms (lm_head
// 76.0 / 75.9 us), 8 waves 0.5324 / 0.5326 (81.2 / 81.1 us), 16 waves 0.5301 /
// 0.5299 (79.3 / 78.9 us).
constexpr int kLmHeadWaves = 4;
constexpr int kOProjWaves = 4;  // waves (rows) per o_proj block
// Waves (rows) per down block. Measured on the whole step (255 graph-replayed
// greedy steps, two rounds): 1 wave 0.5276 / 0.5281 ms, 2 waves 0.5244 /
// 0.5246, 4 waves 0.5252 / 0.5254, 8 waves 0.5267, 16 waves 0.565. Staging
// the activation in LDS once per block instead of every wave reading it from
// the cache measured slower at 2, 4 and 8 waves (0.5294-0.5307 ms).
constexpr int kDownWaves = 2;
constexpr int kQkvRowsPerWave = 2;   // rows per qkv wave (separate kernel and split grid)
#ifndef LCR_EXCHANGE_QKV_ROWS
#define LCR_EXCHANGE_QKV_ROWS 2
#endif
#ifndef LCR_EXCHANGE_OPROJ_ROWS
#define LCR_EXCHANGE_OPROJ_ROWS 2
#endif
// Rows per wave of the one-split exchange grid's q/k/v blocks and of the
// exchange grids' o_proj blocks. Two: the q/k/v projection is the start of
// the grid's dependency chain and streams fastest spread over the most
// compute units (192 blocks of 16 rows; 96 blocks of 32 rows measured
// 9.7 -> 11.2 us for the grid).
constexpr int kExchangeQkvRows = LCR_EXCHANGE_QKV_ROWS;
// Ticks of the 100 MHz realtime counter (1 us) that the one-split grid's
// o_proj blocks wait before requesting their weight rows. The blocks that
// are dispatched with the first wave of the grid (the grid has more blocks
// than compute units) would otherwise stream their rows beside the q/k/v
// rows at the head of the grid's dependency chain; their output is needed
// only after attention, about 7 us in. Measured in one session: 0.5344 ms
// per token without the wait, 0.5317 with it (0.5322 when only blocks that
// can be in the first wave wait; 2 us: slower).
constexpr unsigned kOProjStartDelay = 100;
constexpr int kOProjRowsPerWave = LCR_EXCHANGE_OPROJ_ROWS;
constexpr int kGateUpActsPerWave = 1;  // activations (gate + up row pairs) per gate_up wave
// Waves per gate_up block (at least kThreads / 64: the norm's threads). Each
// block repeats the norm, so fewer, larger blocks would repeat it less; the
// whole step measured slower with them (two rounds): 4 waves 0.5221 / 0.5226
// ms, 8 waves 0.5265 / 0.5267, 16 waves 0.5309 / 0.5306, and two activations
// per wave at 4 waves 0.5322 / 0.5324.
constexpr int kGateUpWaves = 4;
// Query heads per block in the long-context attention launch (with fewer
// than G, the heads of one kv head are spread over G / kLongContextHeads
// blocks on one XCD, which share its keys and values in L2). The whole group
// of four measured fastest at 32768 positions: 27.0 us at 32 splits, against
// 28.3 us for two heads per block at their best count (16 splits), although
// two heads leave the registers for two key/value tiles in flight per wave.
constexpr int kLongContextHeads = 4;
// From this many splits on (the model's policy gives them to contexts of 16384
// and more) attention runs kLongContextHeads query heads per block.
constexpr int kGroupedMinSplits = 16;

__device__ __forceinline__ float silu(float v) { return lcr_silu(v); }

// RMSNorm of the residual sum v into LDS as elements:
//   normed = rne((f(rne(v)) * scale) * f(w)),  scale from sum(v^2).
// Split in two so a kernel can issue the norm's loads (v and w, 12 KiB) before
// its weight stream: loads return in issue order, so inputs fetched after the
// weight tile would make the norm wait for the whole tile.
// Thread t handles chunks t, t+256, ... as the fixed norm order requires.
template <int NCH>
struct NormInput {
  static constexpr int kPer = NCH / 4;  // chunks per thread (H / 8 / 256)
  float v[kPer][8];
  vec16 w[kPer];
};

// `load_chunk(c, out8)` yields the 8 floats of chunk c of v.
// Threads from kThreads on (blocks of more than kThreads threads) take no part.
template <int NCH, typename LoadChunk>
__device__ __forceinline__ void norm_load(NormInput<NCH>& in, LoadChunk load_chunk,
                                          const elem_t* __restrict__ w) {
  const int t = threadIdx.x;
  if (t >= kThreads) return;
#pragma unroll
  for (int c = 0; c < NormInput<NCH>::kPer; ++c) {
    const int chunk = t + c * kThreads;
    load_chunk(chunk, in.v[c]);
    in.w[c] = load16(w + 8 * chunk);
  }
}

// Finishes the norm into `xs` (all threads; two barriers, the first inside
// the sum of squares; `scratch` is used once per kernel and holds one float
// per 32 threads of the block). When `resid_out` is set, the thread also
// stores its v chunks there (layer 0 seeding the residual sum with the
// embedding row). Threads from kThreads on contribute nothing.
template <int NCH>
__device__ __forceinline__ void norm_finish(elem_t* xs, const NormInput<NCH>& in, float eps,
                                            float* scratch, float* resid_out) {
  constexpr int H = NCH * 512;
  const int t = threadIdx.x;
  const bool active = t < kThreads;
  float s = 0.0f;
  if (active) {
#pragma unroll
    for (int c = 0; c < NormInput<NCH>::kPer; ++c) {
#pragma unroll
      for (int j = 0; j < 8; ++j) s = __builtin_fmaf(in.v[c][j], in.v[c][j], s);
    }
  }
  const float scale = norm_scale(block_norm_total_once(s, scratch), H, eps);
#pragma unroll
  for (int c = 0; c < NormInput<NCH>::kPer; ++c) {
    if (!active) break;
    const int chunk = t + c * kThreads;
    const float* v = in.v[c];
    if (resid_out != nullptr) {
      *reinterpret_cast<float4*>(resid_out + 8 * chunk) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(resid_out + 8 * chunk + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
    vec16 out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x0 = elem_to_float(float_to_elem(v[2 * i]));
      const float x1 = elem_to_float(float_to_elem(v[2 * i + 1]));
      out.w[i] = pack_elems((x0 * scale) * elem_lo(in.w[c].w[i]),
                            (x1 * scale) * elem_hi(in.w[c].w[i]));
    }
    store16(xs + 8 * chunk, out);
  }
  __syncthreads();
}

template <int NCH>
__device__ __forceinline__ void load_x_lds(vec16 (&xv)[NCH], const elem_t* xs, int lane) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) xv[c] = load16(xs + c * 512 + lane * kGemvChunk);
}

template <int NCH>
__device__ __forceinline__ void load_x_global(vec16 (&xv)[NCH], const elem_t* x, int lane) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) xv[c] = load16(x + c * 512 + lane * kGemvChunk);
}

__device__ __forceinline__ void load_resid_chunk(const float* resid, int chunk, float* out) {
  const float4 a = *reinterpret_cast<const float4*>(resid + 8 * chunk);
  const float4 b = *reinterpret_cast<const float4*>(resid + 8 * chunk + 4);
  out[0] = a.x; out[1] = a.y; out[2] = a.z; out[3] = a.w;
  out[4] = b.x; out[5] = b.y; out[6] = b.z; out[7] = b.w;
}

// ---------------------------------------------------------------------------
// 1. QKV projection + RoPE + KV append
// ---------------------------------------------------------------------------

// LDS of a q/k/v block with `PAIRS` rotation pairs.
template <int NCH, int PAIRS>
struct QkvShared {
  __attribute__((aligned(16))) elem_t xs[NCH * 512];
  float scratch[16];
  float rowv[2 * PAIRS];
};

// Block `block` of the q/k/v projection, with WAVES waves of RW rows each.
// It serves PAIRS = WAVES / 2 * RW rotation pairs (i, i + head_dim / 2) of one
// head: the first WAVES / 2 waves take the first rows of the pairs, the others
// the second ones. With kPublish the rotated query and key values and the
// value rows also go out as exchange words (exchange.h) for the attention
// blocks of the same grid:
//  - kPublishConsume: 3 * HD consume words per query head h: its query at
//    x[3 h HD + i], and the key and value of its kv head at x[3 h HD + HD + i]
//    and x[3 h HD + 2 HD + i] (a kv head's once for each of its G query heads);
//  - kPublishBroadcast: broadcast words tagged `tag`, in the projection's row
//    order (queries, keys, values, head after head) from
//    exchange_qkv_word().
//
// At layer 0 block 0 also seeds the residual sum with the embedding row,
// unless `seed` is false (the exchange grid with o_proj blocks, which read
// the embedding row themselves: a seed written from one XCD's L2 and joins
// written from others could be written back in either order).
constexpr int kPublishNone = 0;
constexpr int kPublishConsume = 1;
constexpr int kPublishBroadcast = 2;

// `after_load` runs right after the block's weight loads are issued (the layer
// grid issues the loads of its later phases there).
template <int NCH, int HD, bool kPaged, int WAVES, int RW, int G, int kPublish, typename AfterLoad = NoPreWait>
__device__ __forceinline__ void qkv_block(const DecodeStepArgs& a, const LayerDevicePtrs& w,
                                          const KvCacheView& view, int layer, int block,
                                          QkvShared<NCH, WAVES / 2 * RW>& sh, bool seed = true, uint32_t tag = 0,
                                          AfterLoad after_load = AfterLoad{}) {
  constexpr int H = NCH * 512;
  constexpr int HALF = HD / 2;
  constexpr int PAIRS = WAVES / 2 * RW;  // rotation pairs per block
  constexpr int BLOCKS_PER_HEAD = HALF / PAIRS;
  static_assert(HALF % PAIRS == 0, "head_dim / 2 must be a multiple of the pairs per block");

  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int head = block / BLOCKS_PER_HEAD;
  const int i0 = (block % BLOCKS_PER_HEAD) * PAIRS;
  const int r0 = i0 + (wave % (WAVES / 2)) * RW + ((wave / (WAVES / 2)) ? HALF : 0);  // row within the head

  // Everything the prologue and epilogue read is requested before the weight
  // tile, so its latency hides under the stream: the position, the rotation
  // (cos, sin) of this position from the precomputed table, and the norm
  // inputs.
  const int pos = *a.position;
  const float2 rot = a.rope_table[static_cast<size_t>(pos) * HALF + i0 + (threadIdx.x % PAIRS)];
  NormInput<NCH> nin;
  if (layer == 0) {
    const elem_t* erow = a.embedding + static_cast<size_t>(*a.token) * H;
    norm_load<NCH>(nin, [&](int chunk, float* out) { unpack8(load16(erow + 8 * chunk), out); },
                   w.input_norm);
  } else {
    norm_load<NCH>(nin, [&](int chunk, float* out) { load_resid_chunk(a.resid, chunk, out); },
                   w.input_norm);
  }

  GemvTile<RW, NCH> tile;
  {
    const elem_t* rows[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) rows[r] = w.qkv + static_cast<size_t>(head * HD + r0 + r) * H;
    tile.load(rows, lane);
  }
  after_load();

  norm_finish<NCH>(sh.xs, nin, a.eps, sh.scratch, (seed && layer == 0 && block == 0) ? a.resid : nullptr);

  vec16 xv[NCH];
  load_x_lds<NCH>(xv, sh.xs, lane);
  float out[RW];
  tile.dot(out, xv);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RW; ++r) sh.rowv[wave * RW + r] = elem_to_float(float_to_elem(out[r]));
  }
  __syncthreads();

  if (static_cast<int>(threadIdx.x) < PAIRS) {
    const int k = threadIdx.x;
    const int i = i0 + k;
    const float lo = sh.rowv[k];
    const float hi = sh.rowv[PAIRS + k];
    unsigned long long* xw = a.exchange;
    if constexpr (kPublish == kPublishBroadcast) {
      // Published first, in row order: the rotated or copied values below,
      // as floats of their element values.
      unsigned long long* dst = xw + exchange_qkv_word(a.num_heads, HD) + static_cast<size_t>(head) * HD;
      float lo_out = lo, hi_out = hi;
      if (head < a.num_heads + a.num_kv_heads) {
        lo_out = elem_to_float(float_to_elem(lo * rot.x - hi * rot.y));
        hi_out = elem_to_float(float_to_elem(hi * rot.x + lo * rot.y));
      } else {
        lo_out = elem_to_float(float_to_elem(lo));
        hi_out = elem_to_float(float_to_elem(hi));
      }
      exchange_put_tagged(dst + i, tag, __float_as_uint(lo_out));
      exchange_put_tagged(dst + i + HALF, tag, __float_as_uint(hi_out));
    }
    if (head < a.num_heads + a.num_kv_heads) {
      const float ra = lo * rot.x - hi * rot.y;
      const float rb = hi * rot.x + lo * rot.y;
      const elem_t ea = float_to_elem(ra);
      const elem_t eb = float_to_elem(rb);
      if (head < a.num_heads) {
        a.q[head * HD + i] = ea;
        a.q[head * HD + i + HALF] = eb;
        if constexpr (kPublish == kPublishConsume) {
          unsigned long long* dst = xw + static_cast<size_t>(3 * head) * HD;
          exchange_put(dst + i, elem_to_float(ea));
          exchange_put(dst + i + HALF, elem_to_float(eb));
        }
      } else {
        const int kvh = head - a.num_heads;
        const size_t off = view.offset<kPaged>(kvh, pos);
        view.keys[off + i] = ea;
        view.keys[off + i + HALF] = eb;
        if constexpr (kPublish == kPublishConsume) {
#pragma unroll
          for (int g = 0; g < G; ++g) {
            unsigned long long* dst = xw + static_cast<size_t>(3 * (kvh * G + g) + 1) * HD;
            exchange_put(dst + i, elem_to_float(ea));
            exchange_put(dst + i + HALF, elem_to_float(eb));
          }
        }
      }
    } else {
      const int kvh = head - a.num_heads - a.num_kv_heads;
      const size_t off = view.offset<kPaged>(kvh, pos);
      const elem_t ea = float_to_elem(lo);
      const elem_t eb = float_to_elem(hi);
      view.values[off + i] = ea;
      view.values[off + i + HALF] = eb;
      if constexpr (kPublish == kPublishConsume) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
          unsigned long long* dst = xw + static_cast<size_t>(3 * (kvh * G + g) + 2) * HD;
          exchange_put(dst + i, elem_to_float(ea));
          exchange_put(dst + i + HALF, elem_to_float(eb));
        }
      }
    }
  }
}

template <int NCH, int HD, bool kPaged>
__global__ __launch_bounds__(kThreads) void qkv_rope_kernel(DecodeStepArgs a, LayerDevicePtrs w,
                                                            KvCacheView view, int layer) {
  __shared__ QkvShared<NCH, kWaves / 2 * kQkvRowsPerWave> sh;
  qkv_block<NCH, HD, kPaged, kWaves, kQkvRowsPerWave, 1, kPublishNone>(a, w, view, layer, blockIdx.x, sh);
}

// ---------------------------------------------------------------------------
// 2. Attention (split-K; a second kernel merges the splits)
// ---------------------------------------------------------------------------

// Block b of a grid with `group` blocks per (kv head, split) unit: up to 16K
// positions one block per (query head, split), four times the blocks of a
// per-kv-head grid with a quarter of the arithmetic each, which is what the
// latency-bound shorter contexts need; beyond, one block per pair of query
// heads. The blocks of one unit are numbered so they land on the same XCD
// (consecutive block ids go round robin over the 8 XCDs), where they share
// the key/value lines in that XCD's L2. The results equal a per-kv-head
// grid's bit for bit: no arithmetic mixes heads.
__device__ __forceinline__ void attention_block_coords(int b, int units, int group, int* unit,
                                                       int* g) {
  constexpr int kXcds = 8;
  const int full = (units / kXcds) * kXcds * group;  // blocks in whole rounds of 8 units
  if (b < full) {
    const int round = b / (kXcds * group);
    const int rem = b % (kXcds * group);
    *g = rem / kXcds;
    *unit = round * kXcds + rem % kXcds;
  } else {
    const int tail = units % kXcds;
    const int r = b - full;
    *g = r / tail;
    *unit = (units / kXcds) * kXcds + r % tail;
  }
}

// kHeads query heads per block (1 or kLongContextHeads), G / kHeads blocks
// per (kv head, split), numbered so the blocks of a kv head share an XCD.
template <bool kPaged, int HD, int G, int kHeads>
__global__ __launch_bounds__(kAttnThreads) void attention_step_kernel(DecodeStepArgs a,
                                                                      KvCacheView view,
                                                                      float scale) {
  __shared__ AttnShared<kPaged, HD, kHeads> sh;
  constexpr int kBlocksPerGroup = G / kHeads;
  const int seq_len = *a.position + 1;
  const int splits = min(a.splits, seq_len);
  int unit, g = 0;
  if (kBlocksPerGroup > 1) {
    attention_block_coords(blockIdx.x, a.num_kv_heads * a.splits, kBlocksPerGroup, &unit, &g);
  } else {
    unit = blockIdx.x;
  }
  const int kv_head = unit / a.splits;
  const int split = unit % a.splits;
  // A graph captured for more splits than this position can use: the extra
  // blocks have no range and must not touch the partials of other heads.
  if (split >= splits) return;
  decode_attention_block<kPaged, HD, kHeads>(sh, a.attn, a.partials, a.q, view, kv_head,
                                             kv_head * G + g * kHeads, split, splits, seq_len, scale);
}

// q/k/v projection and single-split attention in one grid (exchange.h). The
// first qkv_blocks blocks are the projection (kAttnWaves waves of
// kExchangeQkvRows rows) and publish what they compute; the
// last num_heads blocks are the attention, one query head each, numbered as
// attention_step_kernel numbers them (qkv_blocks is a multiple of the eight
// XCDs, so each kv head's blocks still share one XCD). An attention block
// issues its first cache tiles while the projection streams its weights, then
// takes its query and the new key and value from the exchange words. Same
// arithmetic, same bits as qkv_rope_kernel followed by attention_step_kernel.
template <int NCH, int HD, bool kPaged>
struct ExchangeStepShared {
  union {
    QkvShared<NCH, kAttnWaves / 2 * kExchangeQkvRows> qkv;
    struct {
      AttnShared<kPaged, HD, 1> attn;
      float q[HD];
      __attribute__((aligned(16))) elem_t kv[2 * HD];
    } at;
    __attribute__((aligned(16))) elem_t ox[NCH * 512];  // o_proj blocks: the attention output
  };
};

// Block `ob` of the o_proj projection inside the exchange grid: kAttnWaves
// waves of kOProjRowsPerWave rows. Its weight rows and residual entries are
// requested first; then each wave waits for its share of the attention
// output's broadcast words (two elements per word), the block assembles the
// whole vector in LDS, and finishes as proj_residual_kernel does (same
// products in the same order, same residual join).
//
// At layer 0 (`first`) the residual sum before the join is the embedding row,
// read from the embedding (the q/k/v blocks of this grid do not seed it).
template <int NCH>
__device__ __forceinline__ void oproj_block(const DecodeStepArgs& a, const elem_t* __restrict__ W,
                                            unsigned long long* words, uint32_t tag, int ob, elem_t* xs,
                                            bool first, unsigned start_delay = 0) {
  constexpr int K = NCH * 512;
  constexpr int RW = kOProjRowsPerWave;
  constexpr int PER = K / 2 / kAttnThreads;  // words per lane
  static_assert(PER * 2 * kAttnThreads == K, "the block's lanes take the words evenly");
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  const int row0 = (ob * kAttnWaves + wave) * RW;
  if (start_delay > 0) {
    // Wait start_delay ticks of the 100 MHz realtime counter before
    // requesting the weight rows (see kOProjStartDelay).
    const unsigned long long t0 = wall_clock64();
    while (wall_clock64() - t0 < start_delay) __builtin_amdgcn_s_sleep(2);
  }
  GemvTile<RW, NCH> tile;
  {
    const elem_t* rows[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) rows[r] = W + static_cast<size_t>(row0 + r) * K;
    tile.load(rows, lane);
  }
  float vold[RW];
  const elem_t* erow = a.embedding + static_cast<size_t>(*a.token) * a.hidden;
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    vold[r] = first ? elem_to_float(erow[row0 + r]) : a.resid[row0 + r];
    hold_value(vold[r]);
  }
  uint32_t payload[PER];
  exchange_wait_tagged<PER>(words + wave * 64 * PER, tag, payload, a.exchange_spins, a.exchange_status);
  uint32_t* xs32 = reinterpret_cast<uint32_t*>(xs);
#pragma unroll
  for (int k = 0; k < PER; ++k) xs32[wave * 64 * PER + lane + 64 * k] = payload[k];
  __syncthreads();
  vec16 xv[NCH];
  load_x_lds<NCH>(xv, xs, lane);
  float out[RW];
  tile.dot(out, xv);
  if (lane == 0) {
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const float proj = elem_to_float(float_to_elem(out[r]));
      const float xold = elem_to_float(float_to_elem(vold[r]));
      a.resid[row0 + r] = xold + proj;
    }
  }
}

//
// kOProj: the o_proj projection with its residual join joins the grid as its
// last hidden / (kAttnWaves * kOProjRowsPerWave) blocks (oproj_block), fed
// by the attention blocks' broadcast words. Their tag is
// epoch * kExchangeTagSlots + tag_slot + 1: `tag_slot` is the launch's place
// in its graph (the layer in a decode step), `epoch` the count of completed
// steps, which only grows.
template <int NCH, int HD, bool kPaged, int G, bool kOProj>
__global__ __launch_bounds__(kAttnThreads) void qkv_attention_kernel(DecodeStepArgs a, LayerDevicePtrs w,
                                                                     KvCacheView view, int layer,
                                                                     int qkv_blocks, float scale, int tag_slot) {
  __shared__ ExchangeStepShared<NCH, HD, kPaged> sh;
  const int b = static_cast<int>(blockIdx.x);
  if (b < qkv_blocks) {
    qkv_block<NCH, HD, kPaged, kAttnWaves, kExchangeQkvRows, G, kPublishConsume>(a, w, view, layer, b, sh.qkv,
                                                                                 !kOProj);
    return;
  }
  const size_t broadcast = 3 * static_cast<size_t>(a.num_heads) * HD;  // first broadcast word
  const uint32_t tag = (*a.epoch) * static_cast<uint32_t>(kExchangeTagSlots) + static_cast<uint32_t>(tag_slot) + 1u;
  if constexpr (kOProj) {
    if (b >= qkv_blocks + a.num_heads) {
      oproj_block<NCH>(a, w.o, a.exchange + a.exchange_read_offset + broadcast, tag, b - qkv_blocks - a.num_heads,
                       sh.ox, layer == 0, kOProjStartDelay);
      return;
    }
  }
  int unit, g = 0;
  if (G > 1) {
    attention_block_coords(b - qkv_blocks, a.num_kv_heads, G, &unit, &g);
  } else {
    unit = b - qkv_blocks;
  }
  const int kv_head = unit;
  const int head = kv_head * G + g;
  AttnExchange<HD> x;
  x.words = a.exchange + a.exchange_read_offset + static_cast<size_t>(3 * head) * HD;
  x.broadcast = false;
  x.take_kv = true;
  x.spins = a.exchange_spins;
  x.status = a.exchange_status;
  x.q_lds = sh.at.q;
  x.kv_lds = sh.at.kv;
  x.out_words = kOProj ? a.exchange + broadcast : nullptr;
  x.tag = tag;
  const int seq_len = *a.position + 1;
  decode_attention_block<kPaged, HD, 1, true>(sh.at.attn, a.attn, a.partials, nullptr, view, kv_head, head,
                                              0, 1, seq_len, scale, &x);
}

// q/k/v projection and split attention in one grid (splits > 1). Every block
// is an attention block, numbered as attention_step_kernel numbers them; the
// first qkv_blocks of them also compute 16 q/k/v rows (kAttnWaves waves of
// kQkvRowsPerWave rows), after issuing their first cache tiles and before
// they wait, and publish them as broadcast words for every attention block.
// All blocks fit on the device at once (the host checks), and each does its
// own q/k/v rows before it waits, so every wait is eventually served. The
// split partials go to memory for the merge, as attention_step_kernel's do.
template <int NCH, int HD, bool kPaged, int G, int kHeads>
__global__ __launch_bounds__(kAttnThreads) void split_exchange_kernel(DecodeStepArgs a, LayerDevicePtrs w,
                                                                      KvCacheView view, int layer, int qkv_blocks,
                                                                      float scale, int tag_slot) {
  __shared__ AttnShared<kPaged, HD, kHeads> ash;
  __shared__ QkvShared<NCH, kAttnWaves / 2 * kQkvRowsPerWave> qsh;
  __shared__ float q_lds[kHeads * HD];
  __shared__ __attribute__((aligned(16))) elem_t kv_lds[2 * HD];
  constexpr int kBlocksPerGroup = G / kHeads;
  const int b = static_cast<int>(blockIdx.x);
  const uint32_t tag = (*a.epoch) * static_cast<uint32_t>(kExchangeTagSlots) + static_cast<uint32_t>(tag_slot) + 1u;
  auto project = [&]() {
    if (b < qkv_blocks) {
      qkv_block<NCH, HD, kPaged, kAttnWaves, kQkvRowsPerWave, G, kPublishBroadcast>(a, w, view, layer, b, qsh, true,
                                                                                     tag);
    }
  };
  const int seq_len = *a.position + 1;
  const int splits = min(a.splits, seq_len);
  int unit, g = 0;
  if (kBlocksPerGroup > 1) {
    attention_block_coords(b, a.num_kv_heads * a.splits, kBlocksPerGroup, &unit, &g);
  } else {
    unit = b;
  }
  const int kv_head = unit / a.splits;
  const int split = unit % a.splits;
  if (split >= splits) {
    // No range at this position (a graph captured for more splits): only the
    // projection rows, if the block has any.
    project();
    return;
  }
  const int head0 = kv_head * G + g * kHeads;
  unsigned long long* words = a.exchange + a.exchange_read_offset + exchange_qkv_word(a.num_heads, HD);
  AttnExchange<HD> x;
  x.words = nullptr;
  x.broadcast = true;
  x.q_words = words + static_cast<size_t>(head0) * HD;
  x.k_words = words + static_cast<size_t>(a.num_heads + kv_head) * HD;
  x.v_words = words + static_cast<size_t>(a.num_heads + a.num_kv_heads + kv_head) * HD;
  // The split whose range holds the new position (splits past the end of the
  // sequence have empty ranges, so it need not be the last one).
  const int chunk = (seq_len + splits - 1) / splits;
  x.take_kv = split == (seq_len - 1) / chunk;
  x.spins = a.exchange_spins;
  x.status = a.exchange_status;
  x.q_lds = q_lds;
  x.kv_lds = kv_lds;
  x.out_words = nullptr;
  x.tag = tag;
  // 8192 positions: 0.697 -> 0.688 ms per token; 32768: 0.855 -> 0.835.
  x.early_wait = b < qkv_blocks;
  decode_attention_block<kPaged, HD, kHeads, true>(ash, a.attn, a.partials, nullptr, view, kv_head, head0, split,
                                                   splits, seq_len, scale, &x, project);
}

// The split merge and o_proj in one grid: blocks 0 .. num_heads - 1 merge one
// query head's split partials (from memory, written by the previous kernel),
// as attention_merge_step_kernel does, and publish the output as broadcast
// words; the rest are the exchange grid's o_proj blocks.
template <int NCH, int HD>
__global__ __launch_bounds__(kAttnThreads) void merge_oproj_kernel(DecodeStepArgs a, LayerDevicePtrs w,
                                                                   int tag_slot) {
  __shared__ float lds[kMergeLdsFloats];
  __shared__ __attribute__((aligned(16))) elem_t xs[NCH * 512];
  const int b = static_cast<int>(blockIdx.x);
  const uint32_t tag = (*a.epoch) * static_cast<uint32_t>(kExchangeTagSlots) + static_cast<uint32_t>(tag_slot) + 1u;
  const size_t attn_words = exchange_attn_out_word(a.num_heads, HD);
  if (b >= a.num_heads) {
    oproj_block<NCH>(a, w.o, a.exchange + a.exchange_read_offset + attn_words, tag, b - a.num_heads, xs, false);
    return;
  }
  const int splits = min(a.splits, *a.position + 1);
  merge_split_partials(a.attn, a.partials, b, splits, HD, lds, a.exchange + attn_words, tag);
}

// ---------------------------------------------------------------------------
// The layer grid: a whole layer in one grid (one split)
// ---------------------------------------------------------------------------
//
// One 512-thread block per compute unit, kLayerBlocks of them, all resident
// at once (the host checks), each taking several roles in turn:
//   Q  blocks 0 .. qkv_blocks - 1: 16 q/k/v rows each (qkv_block), publishing
//      the query and the new key and value to the attention blocks (consume
//      words); 192 blocks for Llama-3.2-1B;
//   A  the next num_heads blocks: attention for one query head (as in
//      qkv_attention_kernel), publishing its output as tagged words;
//   O  every block: one o_proj row per wave, joining the residual, and
//      publishing the joined value of its row as a tagged word;
//   G  every block: four gate/up activation pairs per wave, after the norm of
//      the whole residual (read from the O words), publishing the SwiGLU
//      activations as tagged words (two elements each);
//   D  every block: one down row per wave over all activations (read from the
//      G words), joining the residual into memory for the next layer.
// A block issues the weight loads of O and G before it waits for anything
// (Q blocks right after their own q/k/v loads; attention blocks, whose own
// registers are full, after the attention), so the o_proj and gate/up
// weights stream while the q/k/v -> attention -> o_proj chain runs; the down
// loads are issued once G has consumed its registers. The arithmetic of every
// row is the separate kernels' (same tiles, same orders, same rounding
// points), so the results are theirs bit for bit.
//
// Word regions (exchange.h, X = num_heads * head_dim): the one-split grid's
// consume words [0, 3X) and attention words [3X, 3.5X); then the O words
// (hidden of them) and the G words (ffn / 2) from 3.5X.
constexpr int kLayerBlocks = 256;
constexpr int kLayerActsPerWave = 4;   // gate/up activation pairs per wave
// Of those, the ones whose rows a block requests before it waits for the
// attention output (the rest after o_proj). Every variant measured on
// MI355X for the Llama-3.2-1B step (1 to 4 early activations, the down row
// requested before or after the residual wait, the quiet or the direct wait)
// took 32-35 us per layer, against 28.4 us for the exchange grid, gate_up and
// down kernels, which is why the model leaves this grid off by default.
constexpr int kLayerEarlyActs = 2;

__host__ __device__ inline size_t layer_resid_word(int num_heads, int head_dim) {
  return exchange_qkv_word(num_heads, head_dim);
}
__host__ __device__ inline size_t layer_act_word(int num_heads, int head_dim, int hidden) {
  return exchange_qkv_word(num_heads, head_dim) + static_cast<size_t>(hidden);
}

// Every wave of the block waits for N tagged words per lane at address(k):
// first lane 0 alone polls one of the wave's words (one small read per poll
// instead of the wave's whole set, while the producers still stream their
// weights), then the wave takes them all.
template <int N, typename Address>
__device__ __forceinline__ void wait_tagged_quietly(Address address, uint32_t tag, uint32_t (&out)[N], int spins,
                                                    int* status) {
  const int lane = lane_id();
  int polls = 0;
  while (true) {
    uint32_t seen = 0;
    if (lane == 0) seen = static_cast<uint32_t>(exchange_peek(address(0)) >> 32);
    seen = __builtin_amdgcn_readfirstlane(seen);
    if (seen == tag) break;
    if (++polls >= spins) break;  // the full wait below gives up and reports
  }
  exchange_wait_tagged_at<N>(address, tag, out, spins, status);
}

template <int NCH, int NCH_F, int HD, bool kPaged, int G>
struct LayerShared {
  union {
    QkvShared<NCH, kAttnWaves / 2 * kQkvRowsPerWave> qkv;
    struct {
      AttnShared<kPaged, HD, 1> attn;
      float q[HD];
      __attribute__((aligned(16))) elem_t kv[2 * HD];
    } at;
    struct {
      __attribute__((aligned(16))) elem_t xs[NCH * 512];  // o_proj input, then the normed residual
      float scratch[16];
    } og;
    __attribute__((aligned(16))) elem_t act[NCH_F * 512];  // down input
  };
  float resid[NCH * 512];  // the residual after o_proj (G's norm input, D's join)
  // Words the block publishes (its o_proj rows' joined residual, then its
  // activation pairs), gathered so that one wave writes them with one store
  // instruction: every 64-byte line of words has one writer instruction, as
  // in the other exchange grids.
  uint32_t publish[2 * kAttnWaves];
};

// The gate and up rows of activations first .. first + R/2 - 1, as pairs.
template <int R, int NCH>
__device__ __forceinline__ void load_gate_up_rows(GemvTile<R, NCH>& tile, const elem_t* __restrict__ gate_up,
                                                  int first, int ffn, int lane) {
  constexpr int H = NCH * 512;
  const elem_t* rows[R];
#pragma unroll
  for (int k = 0; k < R / 2; ++k) {
    rows[2 * k] = gate_up + static_cast<size_t>(first + k) * H;
    rows[2 * k + 1] = gate_up + static_cast<size_t>(ffn + first + k) * H;
  }
  tile.load(rows, lane);
}

template <int NCH, int NCH_F, int HD, bool kPaged, int G>
__global__ __launch_bounds__(kAttnThreads) void layer_grid_kernel(DecodeStepArgs a, LayerDevicePtrs w,
                                                                  KvCacheView view, int layer, int qkv_blocks,
                                                                  float scale, int tag_slot) {
  constexpr int H = NCH * 512;
  constexpr int F = NCH_F * 512;
  constexpr int A = kLayerActsPerWave;
  constexpr int E = kLayerEarlyActs;
  static_assert(H / kLayerBlocks == kAttnWaves, "one o_proj and one down row per wave");
  static_assert(F / kLayerBlocks == kAttnWaves * A, "four activations per wave");
  static_assert(E >= 0 && E <= A, "early activations are a part of the wave's");
  __shared__ LayerShared<NCH, NCH_F, HD, kPaged, G> sh;
  const int b = static_cast<int>(blockIdx.x);
  const int lane = lane_id();
  const int wave = static_cast<int>(threadIdx.x) >> 6;
  const uint32_t tag = (*a.epoch) * static_cast<uint32_t>(kExchangeTagSlots) + static_cast<uint32_t>(tag_slot) + 1u;
  unsigned long long* const attn_words = a.exchange + exchange_attn_out_word(a.num_heads, HD);
  unsigned long long* const resid_words = a.exchange + layer_resid_word(a.num_heads, HD);
  unsigned long long* const act_words = a.exchange + layer_act_word(a.num_heads, HD, H);
  const int rd = a.exchange_read_offset;

  const int row = b * kAttnWaves + wave;  // this wave's o_proj and down row
  const int act0 = row * A;               // its first activation
  GemvTile<1, NCH> wo;
  GemvTile<2 * (E > 0 ? E : 1), NCH> wg_early;
  GemvTile<2 * (A - E > 0 ? A - E : 1), NCH> wg_late;
  float vold = 0.0f;  // the residual entry of `row` before the o_proj join
  // Loads return in issue order, so a wait also waits for every load issued
  // before it: a block requests only what arrives before the words it waits
  // for next. During the q/k/v -> attention chain: the o_proj row, and (q/k/v
  // and idle blocks) the gate/up rows of the first E activations; after
  // o_proj: the other gate/up rows (the attention blocks' E as well: theirs
  // would arrive after the attention output) and the down row, which streams
  // behind them while G waits and runs.
  const bool attention_role = b >= qkv_blocks && b < qkv_blocks + a.num_heads;
  auto issue_early = [&]() {
    vold = layer == 0 ? elem_to_float(a.embedding[static_cast<size_t>(*a.token) * H + row]) : a.resid[row];
    const elem_t* orow[1] = {w.o + static_cast<size_t>(row) * H};
    wo.load(orow, lane);
    if constexpr (E > 0) {
      if (!attention_role) load_gate_up_rows(wg_early, w.gate_up, act0, F, lane);
    }
  };

  if (b < qkv_blocks) {
    // Q: its q/k/v rows; the residual is not seeded here (the O role reads
    // the embedding row at layer 0 itself).
    qkv_block<NCH, HD, kPaged, kAttnWaves, kQkvRowsPerWave, G, kPublishConsume>(a, w, view, layer, b, sh.qkv, false);
  } else if (attention_role) {
    // A: attention for one query head, numbered as qkv_attention_kernel
    // numbers its attention blocks (the q/k/v blocks are a multiple of the
    // eight XCDs).
    int unit, g = 0;
    if (G > 1) {
      attention_block_coords(b - qkv_blocks, a.num_kv_heads, G, &unit, &g);
    } else {
      unit = b - qkv_blocks;
    }
    const int head = unit * G + g;
    AttnExchange<HD> x;
    x.words = a.exchange + rd + static_cast<size_t>(3 * head) * HD;
    x.broadcast = false;
    x.take_kv = true;
    x.spins = a.exchange_spins;
    x.status = a.exchange_status;
    x.q_lds = sh.at.q;
    x.kv_lds = sh.at.kv;
    x.out_words = attn_words;
    x.tag = tag;
    decode_attention_block<kPaged, HD, 1, true>(sh.at.attn, a.attn, a.partials, nullptr, view, unit, head, 0, 1,
                                                *a.position + 1, scale, &x);
  }
  issue_early();
  __syncthreads();  // the Q and A roles are done with the LDS union

  // O: the attention output (two elements per word) into LDS, the row's dot,
  // the residual join, published.
  {
    constexpr int PER = H / 2 / kAttnThreads;
    uint32_t payload[PER];
    unsigned long long* mine = attn_words + rd + wave * 64 * PER;
    wait_tagged_quietly<PER>([&](int k) { return mine + lane + 64 * k; }, tag, payload, a.exchange_spins,
                             a.exchange_status);
    uint32_t* xs32 = reinterpret_cast<uint32_t*>(sh.og.xs);
#pragma unroll
    for (int k = 0; k < PER; ++k) xs32[wave * 64 * PER + lane + 64 * k] = payload[k];
    __syncthreads();
    vec16 xv[NCH];
    load_x_lds<NCH>(xv, sh.og.xs, lane);
    float out[1];
    wo.dot(out, xv);
    if (lane == 0) {
      const float proj = elem_to_float(float_to_elem(out[0]));
      const float xold = elem_to_float(float_to_elem(vold));
      sh.publish[wave] = __float_as_uint(xold + proj);
    }
    __syncthreads();
    if (wave == 0 && lane < kAttnWaves) {
      exchange_put_tagged(resid_words + b * kAttnWaves + lane, tag, sh.publish[lane]);
    }
  }
  if constexpr (E > 0) {
    if (attention_role) load_gate_up_rows(wg_early, w.gate_up, act0, F, lane);
  }
  if constexpr (A - E > 0) load_gate_up_rows(wg_late, w.gate_up, act0 + E, F, lane);
  GemvTile<1, NCH_F> wd;
  {
    const elem_t* drow[1] = {w.down + static_cast<size_t>(row) * F};
    wd.load(drow, lane);
  }

  // G: the norm of the whole joined residual (threads below kThreads read
  // chunk t of it, 8 words, as norm_load would from memory), the gate/up rows,
  // SwiGLU, the activations published two to a word.
  {
    NormInput<NCH> nin;
    static_assert(NormInput<NCH>::kPer == 1, "one norm chunk per thread");
    if (static_cast<int>(threadIdx.x) < kThreads) {
      uint32_t bits[8];
      unsigned long long* mine = resid_words + rd + 8 * threadIdx.x;
      wait_tagged_quietly<8>([&](int k) { return mine + k; }, tag, bits, a.exchange_spins, a.exchange_status);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        nin.v[0][j] = __uint_as_float(bits[j]);
        sh.resid[8 * threadIdx.x + j] = nin.v[0][j];
      }
      nin.w[0] = load16(w.post_norm + 8 * threadIdx.x);
    }
    __syncthreads();  // O's LDS reads are done before the norm overwrites it
    norm_finish<NCH>(sh.og.xs, nin, a.eps, sh.og.scratch, nullptr);
    vec16 xv[NCH];
    load_x_lds<NCH>(xv, sh.og.xs, lane);
    float out[2 * A];
    if constexpr (E > 0) {
      float part[2 * (E > 0 ? E : 1)];
      wg_early.dot(part, xv);
#pragma unroll
      for (int k = 0; k < 2 * E; ++k) out[k] = part[k];
    }
    if constexpr (A - E > 0) {
      float part[2 * (A - E > 0 ? A - E : 1)];
      wg_late.dot(part, xv);
#pragma unroll
      for (int k = 0; k < 2 * (A - E); ++k) out[2 * E + k] = part[k];
    }
    uint32_t pairs[A / 2];
#pragma unroll
    for (int k = 0; k < A / 2; ++k) {
      const float g0 = elem_to_float(float_to_elem(out[4 * k]));
      const float u0 = elem_to_float(float_to_elem(out[4 * k + 1]));
      const float g1 = elem_to_float(float_to_elem(out[4 * k + 2]));
      const float u1 = elem_to_float(float_to_elem(out[4 * k + 3]));
      pairs[k] = static_cast<uint32_t>(float_to_elem_bits(silu(g0) * u0)) |
                 (static_cast<uint32_t>(float_to_elem_bits(silu(g1) * u1)) << 16);
    }
    static_assert(A / 2 * kAttnWaves <= 2 * kAttnWaves, "the block's activation words fit the staging");
    if (lane == 0) {
#pragma unroll
      for (int k = 0; k < A / 2; ++k) sh.publish[wave * (A / 2) + k] = pairs[k];
    }
    __syncthreads();
    if (wave == 0 && lane < A / 2 * kAttnWaves) {
      exchange_put_tagged(act_words + b * (A / 2) * kAttnWaves + lane, tag, sh.publish[lane]);
    }
  }

  // D: all activations into LDS, the dot with the down row, the join.
  {
    constexpr int PER = F / 2 / kAttnThreads;
    uint32_t payload[PER];
    unsigned long long* mine = act_words + rd + PER * threadIdx.x;
    wait_tagged_quietly<PER>([&](int k) { return mine + k; }, tag, payload, a.exchange_spins, a.exchange_status);
    __syncthreads();  // G's LDS reads are done before the union is reused
    uint32_t* act32 = reinterpret_cast<uint32_t*>(sh.act);
#pragma unroll
    for (int k = 0; k < PER; ++k) act32[PER * threadIdx.x + k] = payload[k];
    __syncthreads();
    vec16 xv[NCH_F];
    load_x_lds<NCH_F>(xv, sh.act, lane);
    float out[1];
    wd.dot(out, xv);
    if (lane == 0) {
      const float proj = elem_to_float(float_to_elem(out[0]));
      const float xmid = elem_to_float(float_to_elem(sh.resid[row]));
      a.resid[row] = xmid + proj;
    }
  }
}

// Split merge (splits > 1 only), one kMergeThreads-thread block per query head.
__global__ __launch_bounds__(kMergeThreads) void attention_merge_step_kernel(DecodeStepArgs a,
                                                                            int head_dim) {
  __shared__ float lds[kMergeLdsFloats];
  const int splits = min(a.splits, *a.position + 1);
  if (splits <= 1) {
    // The attention blocks wrote the output directly. (The merge of one split
    // would give the same bits; there is nothing to do.)
    return;
  }
  merge_split_partials(a.attn, a.partials, blockIdx.x, splits, head_dim, lds);
}

// ---------------------------------------------------------------------------
// 3 / 5. Projection + residual join (o_proj, down)
// ---------------------------------------------------------------------------

// One row per wave (WAVES waves per block): the shape that streams these
// matrices fastest on MI355X (more, smaller waves than two rows per wave).
// The compiler's own interleaving of the weight and x loads with the
// multiplies is kept: holding all of a row's loads in flight (x first, then
// the weights, no multiply before the last load) measured slower for down,
// 7.75 -> 9.05 us.
template <int NCH, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void proj_residual_kernel(DecodeStepArgs a,
                                                                   const elem_t* __restrict__ W,
                                                                   const elem_t* __restrict__ x) {
  constexpr int K = NCH * 512;
  const int lane = lane_id();
  const int row = blockIdx.x * WAVES + (threadIdx.x >> 6);
  GemvTile<1, NCH> tile;
  const elem_t* rows[1] = {W + static_cast<size_t>(row) * K};
  tile.load(rows, lane);
  // The residual entry this wave finishes, fetched while the weights stream
  // (held: the compiler would otherwise load it after the products, in the
  // lane-0 branch, a round trip of its own: down 7.41 -> 7.0 us when held).
  const float vold = a.resid[row];
  vec16 xv[NCH];
  load_x_global<NCH>(xv, x, lane);
  hold_value(vold);
  float out[1];
  tile.dot(out, xv);
  if (lane == 0) {
    const float proj = elem_to_float(float_to_elem(out[0]));
    const float xold = elem_to_float(float_to_elem(vold));
    a.resid[row] = xold + proj;
  }
}

// ---------------------------------------------------------------------------
// 4. gate/up projection + SwiGLU
// ---------------------------------------------------------------------------

template <int NCH>
__global__ __launch_bounds__(kGateUpWaves * 64) void gate_up_kernel(DecodeStepArgs a, LayerDevicePtrs w) {
  static_assert(kGateUpWaves * 64 >= kThreads, "the norm takes the block's first kThreads threads");
  constexpr int H = NCH * 512;
  __shared__ __attribute__((aligned(16))) elem_t xs[H];
  __shared__ float scratch[kGateUpWaves * 2 + 1];  // one float per 32 threads
  constexpr int A = kGateUpActsPerWave;
  const int lane = lane_id();
  // First activation index of this wave.
  const int i = (blockIdx.x * kGateUpWaves + (threadIdx.x >> 6)) * A;
  NormInput<NCH> nin;
  norm_load<NCH>(nin, [&](int chunk, float* out) { load_resid_chunk(a.resid, chunk, out); },
                 w.post_norm);
  GemvTile<2 * A, NCH> tile;
  const elem_t* rows[2 * A];
#pragma unroll
  for (int k = 0; k < A; ++k) {
    rows[2 * k] = w.gate_up + static_cast<size_t>(i + k) * H;
    rows[2 * k + 1] = w.gate_up + static_cast<size_t>(a.ffn + i + k) * H;
  }
  tile.load(rows, lane);
  norm_finish<NCH>(xs, nin, a.eps, scratch, nullptr);
  vec16 xv[NCH];
  load_x_lds<NCH>(xv, xs, lane);
  float out[2 * A];
  tile.dot(out, xv);
  if (lane == 0) {
#pragma unroll
    for (int k = 0; k < A; ++k) {
      const float g = elem_to_float(float_to_elem(out[2 * k]));
      const float u = elem_to_float(float_to_elem(out[2 * k + 1]));
      a.act[i + k] = float_to_elem(silu(g) * u);
    }
  }
}

// ---------------------------------------------------------------------------
// 6. Output head: final norm, fp32 logits, argmax partials
// ---------------------------------------------------------------------------

// kFold: the step's argmax runs in block 0 of this grid instead of in
// argmax_step_kernel. Every block publishes its key as two tagged words (its
// high and low halves, written by two lanes with one store instruction);
// block 0's first wave waits for all of them (bounded; every block of the
// grid is resident at once, one per compute unit, and only block 0 waits),
// takes the maximum and does argmax_step_kernel's writes. The words are in
// the q/k/v broadcast region, under the step's last tag slot, which no layer
// of a step uses.
constexpr int kHeadTagSlot = kExchangeTagSlots - 1;

template <int NCH, bool kFold>
__global__ __launch_bounds__(kLmHeadWaves * 64) void lm_head_kernel(DecodeStepArgs a) {
  static_assert(kLmHeadWaves * 64 >= kThreads && kLmHeadWaves <= 16, "the norm takes the first kThreads threads");
  constexpr int H = NCH * 512;
  constexpr int GROUP_ROWS = kLmHeadWaves * kLmHeadRows;
  __shared__ __attribute__((aligned(16))) elem_t xs[H];
  __shared__ float scratch[kLmHeadWaves * 2 + 1];  // one float per 32 threads
  __shared__ unsigned long long lds_best[16];
  const int lane = lane_id();
  const int wave = threadIdx.x >> 6;
  // kFold: the epoch read here tags the words and is advanced at the end
  // without a second read. (Reading the position here as well measured 10 us
  // slower per step: it moved the register allocation of the streaming loop
  // below, and the compiler then placed a wait for every load in flight
  // inside that loop.)
  uint32_t tag = 0, epoch0 = 0;
  if constexpr (kFold) {
    epoch0 = *a.epoch;
    tag = epoch0 * static_cast<uint32_t>(kExchangeTagSlots) + kHeadTagSlot + 1u;
  }
  const int groups = (a.vocab + GROUP_ROWS - 1) / GROUP_ROWS;
  const int stride = gridDim.x;

  auto row_ptrs = [&](int g, const elem_t* (&rows)[kLmHeadRows]) {
#pragma unroll
    for (int r = 0; r < kLmHeadRows; ++r) {
      const int row = min(g * GROUP_ROWS + wave * kLmHeadRows + r, a.vocab - 1);
      rows[r] = a.lm_head + static_cast<size_t>(row) * H;
    }
  };

  // The tile loads stay conditional. Unconditional ones (clamped rows) let
  // the compiler keep the next tile's loads in flight during the current
  // tile's multiplies, and measured slower: 84.6 -> 90.0 us.
  NormInput<NCH> nin;
  norm_load<NCH>(nin, [&](int chunk, float* out) { load_resid_chunk(a.resid, chunk, out); },
                 a.final_norm);
  GemvTile<kLmHeadRows, NCH> t0, t1;
  int g = blockIdx.x;
  if (g < groups) {
    const elem_t* rows[kLmHeadRows];
    row_ptrs(g, rows);
    t0.load(rows, lane);
  }
  norm_finish<NCH>(xs, nin, a.eps, scratch, nullptr);
  vec16 xv[NCH];
  load_x_lds<NCH>(xv, xs, lane);

  unsigned long long best = 0;
  auto finish = [&](const GemvTile<kLmHeadRows, NCH>& t, int grp) {
    float out[kLmHeadRows];
    t.dot(out, xv);
#pragma unroll
    for (int r = 0; r < kLmHeadRows; ++r) {
      const int row = grp * GROUP_ROWS + wave * kLmHeadRows + r;
      if (lane == r && row < a.vocab) {
        a.logits[row] = out[r];
        best = umax64(best, argmax_key(out[r], static_cast<uint32_t>(row)));
      }
    }
  };

  for (; g < groups; g += 2 * stride) {
    const int g1 = g + stride;
    if (g1 < groups) {
      const elem_t* rows[kLmHeadRows];
      row_ptrs(g1, rows);
      t1.load(rows, lane);
    }
    finish(t0, g);
    const int g2 = g + 2 * stride;
    if (g2 < groups) {
      const elem_t* rows[kLmHeadRows];
      row_ptrs(g2, rows);
      t0.load(rows, lane);
    }
    if (g1 < groups) finish(t1, g1);
  }
  best = block_max_u64(best, lds_best);
  if (threadIdx.x == 0) a.argmax_partials[blockIdx.x] = best;
  if constexpr (kFold) {
    unsigned long long* words = a.exchange + exchange_qkv_word(a.num_heads, a.head_dim);
    if (threadIdx.x < 2) {
      exchange_put_tagged(words + 2 * blockIdx.x + threadIdx.x, tag,
                          threadIdx.x == 0 ? static_cast<uint32_t>(best >> 32) : static_cast<uint32_t>(best));
    }
    if (blockIdx.x == 0 && wave == 0) {
      constexpr int kPer = 2 * kLmHeadFoldMaxBlocks / 64;  // words per lane
      const int n = 2 * static_cast<int>(gridDim.x);
      unsigned long long* read = words + a.exchange_read_offset;
      uint32_t bits[kPer];
      exchange_wait_tagged_at<kPer>(
          [&](int k) {
            const int i = lane + 64 * k;
            return read + (i < n ? i : 0);
          },
          tag, bits, a.exchange_spins, a.exchange_status);
      // From this block's own key, so that a wait that gave up (its words then
      // hold anything) still leaves a real key in the maximum.
      unsigned long long key = best;
#pragma unroll
      for (int k = 0; k < kPer; ++k) {
        // Word 2b is block b's high half, 2b + 1 its low half: lane + 1's word.
        const uint32_t low = static_cast<uint32_t>(
            __builtin_amdgcn_update_dpp(0, static_cast<int>(bits[k]), 0x101, 0xF, 0xF, true));  // row_shl:1
        if ((lane & 1) == 0 && lane + 64 * k < n) {
          key = umax64(key, (static_cast<unsigned long long>(bits[k]) << 32) | low);
        }
      }
      key = wave_max_u64(key);
      if (lane == 0) {
        // The next step reads the embedding row of this id: after a wait that
        // gave up (the step is reported as failed) the id must still be a row.
        const int32_t id = static_cast<int32_t>(
            min(static_cast<uint32_t>(argmax_id(key)), static_cast<uint32_t>(a.vocab - 1)));
        const int pos = *a.position;
        const int want_host = *a.want_host_id;  // beside the position: one round trip
        *a.sampled = id;
        if (want_host != 0) __hip_atomic_store(a.sampled_host, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        *a.next_token = id;
        if (pos + 1 < a.history_len) a.history[pos + 1] = id;
        *a.position = pos + 1;
        *a.epoch = epoch0 + 1u;
      }
    }
  }
}

// The block maxima are reduced by a separate one-block kernel rather than by
// the last lm_head block: that would need a device-scope release fence in
// every block (an L2 write-back on each of the eight XCDs), which measured
// 2.8x slower for the whole head than this extra launch.
__global__ __launch_bounds__(kThreads) void argmax_step_kernel(DecodeStepArgs a, int blocks) {
  __shared__ unsigned long long lds_best[16];
  unsigned long long best = 0;
  for (int i = threadIdx.x; i < blocks; i += kThreads) best = umax64(best, a.argmax_partials[i]);
  best = block_max_u64(best, lds_best);
  if (threadIdx.x == 0) {
    const int32_t id = argmax_id(best);
    const int pos = *a.position;
    const int want_host = *a.want_host_id;
    *a.sampled = id;
    if (want_host != 0) __hip_atomic_store(a.sampled_host, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    *a.next_token = id;
    if (pos + 1 < a.history_len) a.history[pos + 1] = id;
    *a.position = pos + 1;
    if (a.epoch != nullptr) *a.epoch = *a.epoch + 1u;
  }
}

template <int NCH, int NCH_F, int HD, bool kPaged, int G>
void enqueue_layer_typed(const DecodeStepArgs& a, const LayerDevicePtrs& w, const KvCacheView& view,
                         int layer, hipStream_t s, unsigned mask, int tag_slot) {
  const int qkv_rows = (a.num_heads + 2 * a.num_kv_heads) * HD;
  if (a.exchange != nullptr && a.layer_grid && a.splits == 1 && mask == kDecodeAll) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(HD));
    layer_grid_kernel<NCH, NCH_F, HD, kPaged, G><<<kLayerBlocks, kAttnThreads, 0, s>>>(
        a, w, view, layer, qkv_rows / (kAttnWaves * kQkvRowsPerWave), scale, tag_slot);
    HIP_CHECK_LAUNCH();
    return;
  }
  if (a.exchange != nullptr && a.exchange_single && a.splits == 1 && (mask & kDecodeQkv) &&
      (mask & kDecodeAttention)) {
    const int qkv_blocks = qkv_rows / (kAttnWaves * kExchangeQkvRows);
    const float scale = 1.0f / std::sqrt(static_cast<float>(HD));
    if (a.exchange_oproj && (mask & kDecodeOProj)) {
      const int oproj_blocks = a.hidden / (kAttnWaves * kOProjRowsPerWave);
      qkv_attention_kernel<NCH, HD, kPaged, G, true><<<qkv_blocks + a.num_heads + oproj_blocks, kAttnThreads, 0, s>>>(
          a, w, view, layer, qkv_blocks, scale, tag_slot);
      mask &= ~kDecodeOProj;
    } else {
      qkv_attention_kernel<NCH, HD, kPaged, G, false>
          <<<qkv_blocks + a.num_heads, kAttnThreads, 0, s>>>(a, w, view, layer, qkv_blocks, scale, tag_slot);
    }
    HIP_CHECK_LAUNCH();
    mask &= ~(kDecodeQkv | kDecodeAttention);
  }
  if (a.exchange != nullptr && a.exchange_split && a.splits > 1 && (mask & kDecodeQkv) && (mask & kDecodeAttention)) {
    constexpr int kGroupHeads = G <= kLongContextHeads ? G : (G % kLongContextHeads == 0 ? kLongContextHeads : 1);
    const bool grouped = a.splits >= kGroupedMinSplits && kGroupHeads > 1;
    const int units = a.num_kv_heads * a.splits * (grouped ? G / kGroupHeads : G);
    const int qkv_blocks = qkv_rows / (kAttnWaves * kQkvRowsPerWave);
    if (units >= qkv_blocks && units <= a.exchange_slots) {
      const float scale = 1.0f / std::sqrt(static_cast<float>(HD));
      if (grouped) {
        split_exchange_kernel<NCH, HD, kPaged, G, kGroupHeads>
            <<<units, kAttnThreads, 0, s>>>(a, w, view, layer, qkv_blocks, scale, tag_slot);
      } else {
        split_exchange_kernel<NCH, HD, kPaged, G, 1><<<units, kAttnThreads, 0, s>>>(a, w, view, layer, qkv_blocks,
                                                                                   scale, tag_slot);
      }
      HIP_CHECK_LAUNCH();
      if (a.exchange_oproj && (mask & kDecodeOProj)) {
        merge_oproj_kernel<NCH, HD><<<a.num_heads + a.hidden / (kAttnWaves * kOProjRowsPerWave), kAttnThreads, 0, s>>>(
            a, w, tag_slot);
        mask &= ~kDecodeOProj;
      } else {
        attention_merge_step_kernel<<<a.num_heads, kMergeThreads, 0, s>>>(a, HD);
      }
      HIP_CHECK_LAUNCH();
      mask &= ~(kDecodeQkv | kDecodeAttention);
    }
  }
  if (mask & kDecodeQkv) {
    qkv_rope_kernel<NCH, HD, kPaged><<<qkv_rows / (kWaves * kQkvRowsPerWave), kThreads, 0, s>>>(a, w, view, layer);
    HIP_CHECK_LAUNCH();
  }
  if (mask & kDecodeAttention) {
    const float scale = 1.0f / std::sqrt(static_cast<float>(HD));
    constexpr int kHeads = G <= kLongContextHeads ? G : (G % kLongContextHeads == 0 ? kLongContextHeads : 1);
    if (a.splits >= kGroupedMinSplits && kHeads > 1) {
      attention_step_kernel<kPaged, HD, G, kHeads>
          <<<a.num_kv_heads * a.splits * (G / kHeads), kAttnThreads, 0, s>>>(a, view, scale);
    } else {
      attention_step_kernel<kPaged, HD, G, 1>
          <<<a.num_kv_heads * a.splits * G, kAttnThreads, 0, s>>>(a, view, scale);
    }
    HIP_CHECK_LAUNCH();
    if (a.splits > 1) {
      attention_merge_step_kernel<<<a.num_heads, kMergeThreads, 0, s>>>(a, HD);
      HIP_CHECK_LAUNCH();
    }
  }
  if (mask & kDecodeOProj) {
    proj_residual_kernel<NCH, kOProjWaves><<<a.hidden / kOProjWaves, kOProjWaves * 64, 0, s>>>(a, w.o, a.attn);
    HIP_CHECK_LAUNCH();
  }
  if (mask & kDecodeGateUp) {
    gate_up_kernel<NCH><<<a.ffn / (kGateUpWaves * kGateUpActsPerWave), kGateUpWaves * 64, 0, s>>>(a, w);
    HIP_CHECK_LAUNCH();
  }
  if (mask & kDecodeDown) {
    proj_residual_kernel<NCH_F, kDownWaves><<<a.hidden / kDownWaves, kDownWaves * 64, 0, s>>>(a, w.down, a.act);
    HIP_CHECK_LAUNCH();
  }
}

}  // namespace

bool decode_step_supported(int hidden, int ffn, int num_heads, int num_kv_heads, int head_dim) {
  if (hidden != 2048 || ffn != 8192 || head_dim != 64) return false;
  if (num_kv_heads <= 0 || num_heads % num_kv_heads != 0) return false;
  if (num_heads * head_dim != hidden) return false;  // o_proj input width == hidden
  const int g = num_heads / num_kv_heads;
  return g == 1 || g == 2 || g == 4 || g == 8;
}

// The q/k/v + attention grid must fit on the device at once. With o_proj
// blocks (with_oproj) it need not: the blocks that wait (attention and
// o_proj) must leave room for at least one more block, so a block that never
// waits (q/k/v) can always run and every wait is eventually served.
bool decode_exchange_fits(int num_heads, int num_kv_heads, int head_dim, int hidden, bool paged,
                          int compute_units, bool with_oproj) {
  if (head_dim != 64 || num_kv_heads <= 0) return false;
  const int g = num_heads / num_kv_heads;
  const int qkv_rows = (num_heads + 2 * num_kv_heads) * head_dim;
  if (qkv_rows % (kAttnWaves * kExchangeQkvRows) != 0) return false;
  const int qkv_blocks = qkv_rows / (kAttnWaves * kExchangeQkvRows);
  if (qkv_blocks % 8 != 0) return false;  // the attention blocks' XCD numbering
  if (with_oproj && (hidden % (kAttnWaves * kOProjRowsPerWave) != 0 || num_heads * head_dim != 2048)) return false;
  int per_cu = 0;
  const void* fn = nullptr;
#define LCR_EXCHANGE_FN(G_)                                                                                    \
  case G_:                                                                                                     \
    if (with_oproj) {                                                                                          \
      fn = paged ? reinterpret_cast<const void*>(&qkv_attention_kernel<4, 64, true, G_, true>)                 \
                 : reinterpret_cast<const void*>(&qkv_attention_kernel<4, 64, false, G_, true>);              \
    } else {                                                                                                   \
      fn = paged ? reinterpret_cast<const void*>(&qkv_attention_kernel<4, 64, true, G_, false>)                \
                 : reinterpret_cast<const void*>(&qkv_attention_kernel<4, 64, false, G_, false>);             \
    }                                                                                                          \
    break;
  switch (g) {
    LCR_EXCHANGE_FN(1)
    LCR_EXCHANGE_FN(2)
    LCR_EXCHANGE_FN(4)
    LCR_EXCHANGE_FN(8)
    default:
      return false;
  }
#undef LCR_EXCHANGE_FN
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kAttnThreads, 0) != hipSuccess) return false;
  const long slots = static_cast<long>(per_cu) * compute_units;
  if (!with_oproj) return slots >= qkv_blocks + num_heads;
  const int waiting = num_heads + hidden / (kAttnWaves * kOProjRowsPerWave);
  return slots >= qkv_blocks + num_heads && slots > waiting;
}

// The layer grid runs when its work divides as the kernel assumes (one o_proj
// and one down row per wave, four activations per wave, 16 q/k/v rows per
// block, the attention blocks after them on whole rounds of the eight XCDs)
// and all kLayerBlocks blocks are resident at once: every block waits for
// words of the others.
bool decode_layer_grid_fits(int hidden, int ffn, int num_heads, int num_kv_heads, int head_dim, bool paged,
                            int compute_units) {
  if (hidden != 2048 || ffn != 8192 || head_dim != 64 || num_kv_heads <= 0) return false;
  if (num_heads * head_dim != hidden || num_heads % num_kv_heads != 0) return false;
  const int qkv_rows = (num_heads + 2 * num_kv_heads) * head_dim;
  if (qkv_rows % (kAttnWaves * kQkvRowsPerWave) != 0) return false;
  const int qkv_blocks = qkv_rows / (kAttnWaves * kQkvRowsPerWave);
  if (qkv_blocks % 8 != 0 || qkv_blocks + num_heads > kLayerBlocks) return false;
  if (exchange_attn_out_word(num_heads, head_dim) + num_heads * head_dim / 2 > layer_resid_word(num_heads, head_dim) ||
      layer_act_word(num_heads, head_dim, hidden) + ffn / 2 > exchange_written_words(num_heads, head_dim)) {
    return false;
  }
  const void* fn = nullptr;
#define LCR_LAYER_FN(G_)                                                                              \
  case G_:                                                                                            \
    fn = paged ? reinterpret_cast<const void*>(&layer_grid_kernel<4, 16, 64, true, G_>)               \
               : reinterpret_cast<const void*>(&layer_grid_kernel<4, 16, 64, false, G_>);             \
    break;
  switch (num_heads / num_kv_heads) {
    LCR_LAYER_FN(1)
    LCR_LAYER_FN(2)
    LCR_LAYER_FN(4)
    LCR_LAYER_FN(8)
    default:
      return false;
  }
#undef LCR_LAYER_FN
  int per_cu = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kAttnThreads, 0) != hipSuccess) return false;
  return static_cast<long>(per_cu) * compute_units >= kLayerBlocks;
}

// Blocks of the split exchange grid the device holds at once (the fewest over
// its variants for this geometry), or 0 when it has none.
int decode_split_exchange_slots(int num_heads, int num_kv_heads, int head_dim, bool paged, int compute_units) {
  if (head_dim != 64 || num_kv_heads <= 0 || num_heads * head_dim != 2048) return 0;
  const int g = num_heads / num_kv_heads;
  const int qkv_rows = (num_heads + 2 * num_kv_heads) * head_dim;
  if (qkv_rows % (kAttnWaves * kQkvRowsPerWave) != 0) return 0;
  int fewest = 1 << 30;
  auto consider = [&](const void* fn) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kAttnThreads, 0) != hipSuccess) per_cu = 0;
    fewest = std::min(fewest, per_cu * compute_units);
  };
#define LCR_SPLIT_FNS(G_)                                                                                      \
  case G_: {                                                                                                   \
    constexpr int kGH = G_ <= kLongContextHeads ? G_ : (G_ % kLongContextHeads == 0 ? kLongContextHeads : 1); \
    if (paged) {                                                                                               \
      consider(reinterpret_cast<const void*>(&split_exchange_kernel<4, 64, true, G_, 1>));                    \
      consider(reinterpret_cast<const void*>(&split_exchange_kernel<4, 64, true, G_, kGH>));                  \
    } else {                                                                                                   \
      consider(reinterpret_cast<const void*>(&split_exchange_kernel<4, 64, false, G_, 1>));                   \
      consider(reinterpret_cast<const void*>(&split_exchange_kernel<4, 64, false, G_, kGH>));                 \
    }                                                                                                          \
    consider(reinterpret_cast<const void*>(&merge_oproj_kernel<4, 64>));                                       \
    break;                                                                                                     \
  }
  switch (g) {
    LCR_SPLIT_FNS(1)
    LCR_SPLIT_FNS(2)
    LCR_SPLIT_FNS(4)
    LCR_SPLIT_FNS(8)
    default:
      return 0;
  }
#undef LCR_SPLIT_FNS
  return fewest == (1 << 30) ? 0 : fewest;
}

// One block per compute unit, each taking the same number of row groups
// (measured on MI355X: 255 blocks of 63 groups stream the 525 MB head in
// 85 us; 1024 blocks of 15-16 groups take 91 us, and grids that leave some
// compute units with two blocks and others with one are slower still).
int lm_head_blocks(int vocab, int compute_units) {
  const int groups = (vocab + kLmHeadWaves * kLmHeadRows - 1) / (kLmHeadWaves * kLmHeadRows);
  const int cus = std::max(1, std::min(compute_units, kLmHeadMaxBlocks));
  const int per_block = (groups + cus - 1) / cus;
  return std::max(1, (groups + per_block - 1) / per_block);
}

void enqueue_decode_layer(const DecodeStepArgs& a, const LayerDevicePtrs& w,
                          const KvCacheView& view, int layer, hipStream_t s, unsigned mask, int tag_slot) {
  const int g = a.num_heads / a.num_kv_heads;
  if (tag_slot < 0) tag_slot = layer;
  // Only the exchange grids tag words with the slot.
  if (a.exchange != nullptr && (mask & kDecodeQkv) && (mask & kDecodeAttention)) {
    LCR_CHECK(tag_slot < kExchangeTagSlots, "exchange tag slot " << tag_slot << " out of range");
  }
#define LCR_LAYER_CASE(G_)                                                                \
  case G_:                                                                                \
    if (a.paged) {                                                                        \
      enqueue_layer_typed<4, 16, 64, true, G_>(a, w, view, layer, s, mask, tag_slot);     \
    } else {                                                                              \
      enqueue_layer_typed<4, 16, 64, false, G_>(a, w, view, layer, s, mask, tag_slot);    \
    }                                                                                     \
    return;
  switch (g) {
    LCR_LAYER_CASE(1)
    LCR_LAYER_CASE(2)
    LCR_LAYER_CASE(4)
    LCR_LAYER_CASE(8)
    default:
      LCR_FAIL("fused decode step has no kernels for " << g << " query heads per kv head");
  }
#undef LCR_LAYER_CASE
}

void enqueue_decode_head_sampled(const DecodeStepArgs& a, const SampledHead& h, hipStream_t s) {
  const int blocks = lm_head_blocks(a.vocab, a.compute_units);
  lm_head_kernel<4, false><<<blocks, kLmHeadWaves * 64, 0, s>>>(a);
  HIP_CHECK_LAUNCH();
  SampleStepState step;
  step.uniforms = h.uniforms;
  step.counter = h.counter;
  step.draws = h.draws;
  step.next_token = a.next_token;
  step.history = a.history;
  step.history_len = a.history_len;
  step.position = a.position;
  step.epoch = a.epoch;
  enqueue_sample_step(a.logits, a.vocab, h.temperature, h.top_k, h.top_p, a.argmax_partials, blocks, a.partials,
                      a.sampled, step, s);
}

void enqueue_decode_argmax(const DecodeStepArgs& a, hipStream_t s) {
  argmax_step_kernel<<<1, kThreads, 0, s>>>(a, lm_head_blocks(a.vocab, a.compute_units));
  HIP_CHECK_LAUNCH();
}

void enqueue_decode_head(const DecodeStepArgs& a, hipStream_t s, bool with_argmax) {
  const int blocks = lm_head_blocks(a.vocab, a.compute_units);
  // With the one-split exchange grid's words (the model's geometry and device
  // run it), the argmax folds into the head's grid.
  if (with_argmax && a.exchange_head && a.exchange != nullptr && a.epoch != nullptr &&
      blocks <= kLmHeadFoldMaxBlocks && blocks <= a.compute_units) {
    lm_head_kernel<4, true><<<blocks, kLmHeadWaves * 64, 0, s>>>(a);
    HIP_CHECK_LAUNCH();
    return;
  }
  lm_head_kernel<4, false><<<blocks, kLmHeadWaves * 64, 0, s>>>(a);
  HIP_CHECK_LAUNCH();
  if (!with_argmax) return;
  argmax_step_kernel<<<1, kThreads, 0, s>>>(a, blocks);
  HIP_CHECK_LAUNCH();
}

}  // namespace lcr
