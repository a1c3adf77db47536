// The fused decode step: five kernels per layer (three where the device runs
// q/k/v, attention and o_proj as one exchange grid, exchange.h) plus the
// output head, every one reading the position and token id from device memory
// so the whole step can be captured once in a hipGraph and replayed.
//
// The arithmetic is exactly that of the reference's unfused sequence
// (src/model.cu:370-484): every bf16 rounding point of the reference is kept
// (qkv, q/k after RoPE, attention output, o_proj output, x after each residual
// join, gate and up, the SwiGLU activation, down output), and every sum uses
// the fixed orders of gemv_core.h, row_norm.h and attention_decode.h. What
// fusion changes is only where intermediate values live:
//  - the residual stream is kept as the unrounded fp32 sum v of each join
//    (x = rne(v) is what the reference stores; the next RMSNorm needs the
//    sum of v^2 over the unrounded v, src/kernels/rmsnorm.cu:86-101), so a
//    GEMV epilogue can finish the join for its own rows and the next kernel's
//    prologue can redo the norm from v;
//  - RMSNorm runs as a prologue of the GEMV that consumes it, once per block,
//    while the block's weight loads are already in flight;
//  - RoPE and the KV append run in the QKV epilogue (a block owns rows i and
//    i + head_dim/2 of a head), SwiGLU in the gate/up epilogue (a wave owns
//    gate row i and up row i), the residual join in the o_proj and down
//    epilogues;
//  - the split-K partials are merged by a separate kernel (long contexts);
//  - lm_head writes fp32 logits and per-block argmax partials.
#pragma once

#include <hip/hip_runtime.h>

#include "../kv_cache.h"

namespace lcr {

struct LayerDevicePtrs {
  const elem_t* input_norm;
  const elem_t* qkv;       // [q_dim + 2 kv_dim][hidden]
  const elem_t* o;         // [hidden][q_dim]
  const elem_t* post_norm;
  const elem_t* gate_up;   // [2 ffn][hidden]
  const elem_t* down;      // [hidden][ffn]
};

struct DecodeStepArgs {
  // model
  int hidden, ffn, num_heads, num_kv_heads, head_dim, vocab;
  float eps;
  const elem_t* embedding;
  const elem_t* final_norm;
  const elem_t* lm_head;
  const float* inv_freq;
  const float2* rope_table;  // [max_seq][head_dim / 2] (cos, sin) of position * inv_freq
  // device state
  const int32_t* token;      // [1] token id of this step
  int32_t* position;         // [1] position of this step; incremented at the end
  int32_t* sampled;          // [1] argmax of this step's logits
  int32_t* next_token;       // [1] also receives the argmax (may alias token)
  int32_t* history;          // [history_len] history[position + 1] = argmax
  int history_len;
  float* resid;              // [hidden] fp32 residual sum v
  elem_t* q;                 // [num_heads * head_dim]
  elem_t* attn;              // [num_heads * head_dim]
  elem_t* act;               // [ffn]
  float* logits;             // [vocab]
  float* partials;           // attention split partials
  unsigned long long* argmax_partials;  // [lm_head blocks]
  bool paged;
  int splits;
  int compute_units;         // of the device: sizes the output head's grid
  // In-grid exchange (exchange.h), over the words at `exchange` (null: no
  // exchange grid runs). With exchange_single and splits == 1, the q/k/v
  // projection and the attention run as one grid (with exchange_oproj, the
  // o_proj projection too); with exchange_split and splits > 1, the q/k/v
  // projection and the split attention run as one grid, and (with
  // exchange_oproj) the split merge and o_proj as another. Words: see
  // exchange_*_word() below; as many again after the written ones are never
  // written (tests of the give-up path read there).
  unsigned long long* exchange;
  bool layer_grid;           // splits == 1: the whole layer as one grid (layer_grid_kernel)
  bool exchange_single;
  bool exchange_oproj;
  bool exchange_split;
  bool exchange_head;        // the greedy step's argmax in the output head's grid
  int exchange_slots;        // blocks of the split grid the device holds at once
  int* exchange_status;      // [1] raised by a wait that gave up (host-coherent memory)
  int exchange_spins;        // polls before a wait gives up
  int exchange_read_offset;  // added to every word the grid reads (0; 3.5X in tests of the give-up path)
  uint32_t* epoch;           // [1] steps completed; advanced by the step's last kernel
  int32_t* sampled_host;     // [1] host-coherent: the greedy step's id as well, when *want_host_id
  const int32_t* want_host_id;  // [1] non-zero: write sampled_host (set by the host per call)
};

// True when the fused kernels are compiled for this geometry.
bool decode_step_supported(int hidden, int ffn, int num_heads, int num_kv_heads, int head_dim);
// True when the q/k/v + attention exchange grid is compiled for this geometry
// and all its blocks fit on the device at once.
bool decode_exchange_fits(int num_heads, int num_kv_heads, int head_dim, int hidden, bool paged,
                          int compute_units, bool with_oproj);
// True when the whole-layer grid is compiled for this geometry and all its
// blocks fit on the device at once.
bool decode_layer_grid_fits(int hidden, int ffn, int num_heads, int num_kv_heads, int head_dim, bool paged,
                            int compute_units);
// Blocks of the split exchange grid the device holds at once, 0 if none.
int decode_split_exchange_slots(int num_heads, int num_kv_heads, int head_dim, bool paged, int compute_units);

// Exchange word regions (X = num_heads * head_dim):
//  [0, 3X)     the query, key and value hand-over of one-split grids,
//              [num_heads][3][head_dim], read once and cleared;
//  [3X, 3.5X)  the attention output, two elements per word, tagged;
//  [3.5X, ...) the q/k/v projection's output in row order, tagged (at most
//              3X words: num_kv_heads <= num_heads).
__host__ __device__ inline size_t exchange_attn_out_word(int num_heads, int head_dim) {
  return 3 * static_cast<size_t>(num_heads) * static_cast<size_t>(head_dim);
}
__host__ __device__ inline size_t exchange_qkv_word(int num_heads, int head_dim) {
  return 7 * static_cast<size_t>(num_heads) * static_cast<size_t>(head_dim) / 2;
}
inline size_t exchange_written_words(int num_heads, int head_dim) {
  return 13 * static_cast<size_t>(num_heads) * static_cast<size_t>(head_dim) / 2;
}
// Exchange words of the step (see DecodeStepArgs::exchange).
inline size_t decode_exchange_words(int num_heads, int head_dim) {
  return 2 * exchange_written_words(num_heads, head_dim);
}
// Launches of one graph that exchange words through the same buffer
// (enqueue_decode_layer's tag_slot is below this).
constexpr int kExchangeTagSlots = 1024;

// The five kernels of a layer, as bits of a selection mask.
enum DecodeKernel : unsigned {
  kDecodeQkv = 1u,
  kDecodeAttention = 2u,
  kDecodeOProj = 4u,
  kDecodeGateUp = 8u,
  kDecodeDown = 16u,
  kDecodeAll = 31u,
};

// Enqueues one layer's kernels (qkv+rope+kv, attention, o_proj+residual,
// gate_up+swiglu, down+residual); `mask` selects a subset (for timing one
// kernel in isolation).
// `tag_slot` (default: the layer) tells launches of one graph apart for the
// exchange grid's broadcast words; graphs that launch one layer more than
// once give each launch its own slot, below kExchangeTagSlots.
void enqueue_decode_layer(const DecodeStepArgs& a, const LayerDevicePtrs& w,
                          const KvCacheView& view, int layer, hipStream_t stream,
                          unsigned mask = kDecodeAll, int tag_slot = -1);
// Enqueues the output head and the argmax (which also advances the position;
// leave it out only to time the head alone).
void enqueue_decode_head(const DecodeStepArgs& a, hipStream_t stream, bool with_argmax = true);
// The argmax alone: the reduction of the output head's per-block keys to the
// id, which also advances the position (timing only).
void enqueue_decode_argmax(const DecodeStepArgs& a, hipStream_t stream);

int lm_head_blocks(int vocab, int compute_units);

// A sampled step's head: the output head, then the sampler (temperature,
// top-k, top-p) with draw uniforms[*counter], which writes the id to
// `sampled`, `next_token` and history[position + 1] and advances the position
// and the counter. The sampler's scratch is `partials` (sized for both).
struct SampledHead {
  float temperature;
  int top_k;
  float top_p;
  const float* uniforms;  // device, one draw per step
  int32_t* counter;       // device, index of the step's draw
  int draws;              // entries of `uniforms` (the index is clamped to it)
};
void enqueue_decode_head_sampled(const DecodeStepArgs& a, const SampledHead& head, hipStream_t stream);

}  // namespace lcr
