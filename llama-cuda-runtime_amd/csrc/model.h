// The model: weights resident in HBM, chunked prefill, single-token decode,
// sampling. Drop-in for the reference's src/model.h:27-193 (same Options
// fields, same public methods and semantics), running on HIP kernels only.
//
// Decode is a weight stream: 2.47 GB of bf16 weights per token for
// Llama-3.2-1B, each used for one multiply-add. The decode step therefore runs
// as fused kernels (three per layer with the exchange grid, see
// kernels/decode_step.h) captured once in
// a hipGraph per attention split count and replayed, with the token id and
// position living in device memory so nothing has to be re-captured per token.
// Prefill (more than one token) is compute bound and runs the projections as
// MFMA GEMMs.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "arena.h"
#include "config.h"
#include "hip_utils.h"
#include "kv_cache.h"
#include "kernels/decode_step.h"
#include "profiler.h"
#include "safetensors.h"

namespace lcr {

struct LayerWeights {
  const elem_t* input_norm = nullptr;
  const elem_t* qkv_proj = nullptr;      // [q_dim + 2 kv_dim][hidden]: q, k, v rows
  const elem_t* o_proj = nullptr;
  const elem_t* post_attention_norm = nullptr;
  const elem_t* gate_up_proj = nullptr;  // [2 ffn][hidden]: gate rows, then up rows
  const elem_t* down_proj = nullptr;
};

struct ForwardStats {
  size_t weight_bytes_per_token = 0;
  size_t kv_bytes_per_position = 0;
  size_t kv_bytes_at(int seq_len) const {
    return static_cast<size_t>(seq_len) * kv_bytes_per_position;
  }
  double last_prefill_ms = 0.0;
  double last_decode_ms = 0.0;
};

class Model {
 public:
  struct Options {
    int device = 0;
    int max_seq = 4096;
    KvLayout kv_layout = KvLayout::kContiguous;
    int page_size = 16;
    // Tokens per prefill pass. The reference defaults to 256 to bound its
    // [heads][rows][keys] fp32 score buffer; attention here keeps scores in
    // registers, so the chunk only sizes the activation buffers, and longer
    // chunks give the GEMMs enough tiles to fill the device.
    int prefill_chunk = 2048;
    int attention_splits = 0;
    // Not in the reference:
    bool fused_decode = true;        // fused kernels when the geometry has them
    bool use_graph = true;           // replay the fused step from a hipGraph
    bool prefill_via_decode = false; // run prompts token by token through decode
    // The decode step's q/k/v projection and single-split attention in one
    // grid, handing the query and the new key and value over in-grid
    // exchange words (kernels/exchange.h), when the device holds the grid.
    bool decode_exchange = true;
    bool exchange_oproj = true;           // and the o_proj projection in the same grid
    bool exchange_split = true;           // split attention: q/k/v + attention, and merge + o_proj, as grids
    int exchange_spins = 1 << 20;         // polls before an exchange wait gives up
    bool exchange_test_unwritten = false; // tests: waits read words no block writes
    // With one attention split, each layer as one grid (kernels/k_decode.hip,
    // layer_grid_kernel) when the device holds it: the o_proj and gate/up
    // weights stream while the q/k/v -> attention -> o_proj chain runs. Off
    // by default: measured 32.8-34.5 us per layer on MI355X against 28.4 us
    // for the exchange grid, gate_up and down kernels it replaces.
    bool layer_grid = false;
    // The greedy step's argmax in the output head's grid (kernels/k_decode.hip,
    // lm_head_kernel<..., true>), when the one-split exchange grid is in use.
    bool exchange_head = true;
  };

  // Prompt chunks shorter than this run token by token through the decode
  // step (GEMV path, bit-identical to decoding them) rather than through the
  // MFMA GEMMs, which only pay off from a few tiles of tokens upward.
  static constexpr int kMinMfmaPrefillTokens = 64;

  Model(const std::string& model_dir, const Options& options);
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  const float* prefill(const std::vector<int>& tokens);
  const float* decode(int token);
  std::vector<float> logits_to_host(const float* device_logits) const;

  void reset();
  int position() const { return position_; }

  const ModelConfig& config() const { return config_; }
  const KvCache& kv_cache() const { return *kv_cache_; }
  KvCache& mutable_kv_cache() { return *kv_cache_; }
  const DeviceArena& arena() const { return arena_; }
  const ForwardStats& stats() const { return stats_; }
  size_t weight_bytes() const { return weight_bytes_; }
  int multiprocessors() const { return multiprocessors_; }
  hipStream_t stream() const { return stream_; }
  const Options& options() const { return options_; }
  bool fused() const { return fused_; }

  int sample(const float* device_logits, float temperature, int top_k, float top_p,
             float uniform);

  struct Tap {
    std::string name;
    int tokens = 0;
    int width = 0;
    std::vector<float> values;
  };
  void set_capture_activations(bool enabled) { capture_activations_ = enabled; }
  Profiler& profiler() { return profiler_; }
  const Profiler& profiler() const { return profiler_; }
  const std::vector<Tap>& activation_taps() const { return taps_; }

  // Not in the reference. Greedy generation kept on the device: decodes
  // `first_token`, then feeds each step's argmax straight into the next step
  // with no host round trip, `steps` decodes in all. Returns the generated ids
  // (the argmax after each step). Needs the fused decode path.
  std::vector<int> generate_greedy(int first_token, int steps, double* elapsed_ms);
  // Not in the reference. Sampled generation kept on the device, the
  // reference's host loop (decode(), then sample() with the next draw,
  // src/main.cu:456-466) without the host: decodes `first_token`, samples
  // the next with uniforms[0] (temperature, top_k, top_p as sample()), feeds
  // it to the next step, and so on, `steps` decodes in all. Returns the
  // sampled ids, the same as decode() + sample() would give with the same
  // draws. Needs the fused decode path.
  std::vector<int> generate_sampled(int first_token, int steps, float temperature, int top_k,
                                    float top_p, const float* uniforms, double* elapsed_ms);
  // Moves the position without running the model (the long-context stress
  // case fills the cache directly). The cache must already hold `position`.
  void set_position(int position);
  // Fills every K and V element of the pool with N(0, stddev^2) bf16 values
  // from a counter-based generator keyed by `seed` (long-context stress case).
  void fill_kv_normal(uint64_t seed, float stddev);
  // The attention split count decode uses at a given sequence length.
  int decode_splits(int seq_len) const;
  // Times one fused decode kernel in isolation: `launches` launches on this
  // model's stream, cycling through the layers so each launch streams
  // different weights, each bracketed by its own pair of hipEvents. Returns
  // the mean launch duration in ms and the algorithmic bytes one launch moves.
  // kernel: "qkv", "attention", "o_proj", "gate_up", "down", "lm_head",
  // "argmax" (the reduction of the head's per-block keys to the id alone, in
  // its own kernel), "head" (lm_head and the argmax as the step runs them:
  // the argmax folded into lm_head's grid when the step exchanges words),
  // "qkv_attention" or "qkv_attention_oproj" (the exchange grids, or the
  // kernels that run in their place), "layer" (a whole layer: the layer grid,
  // or the kernels that run in its place).
  double time_decode_kernel(const std::string& kernel, int launches, double* bytes_per_launch);
  // Whether the decode step runs q/k/v and attention as one exchange grid.
  bool decode_exchange() const { return exchange_enabled_; }
  // Non-zero when an exchange wait of a past step gave up (its results are
  // then not to be trusted); reading it synchronizes the stream. decode(),
  // prefill() and the generate_* loops check it themselves and throw.
  int exchange_status() const;
  // Clears the exchange words and the status (after a wait gave up).
  void clear_exchange();
  // Whether o_proj runs in the exchange grid too.
  bool exchange_oproj() const { return exchange_oproj_; }
  bool exchange_split() const { return exchange_split_slots_ > 0; }
  // Whether single-split decode steps run each layer as one grid.
  bool layer_grid() const { return layer_grid_enabled_; }

 private:
  void load_weights(const SafetensorsArchive& archive);
  void allocate_arena();
  size_t gemm_workspace_bytes() const;
  void run_layers(int tokens, int start_position);
  void attention_prefill(int layer, int tokens, int start_position);
  void attention_decode(int layer, int position);
  void capture(const std::string& name, const elem_t* source, int tokens, int width);
  void capture_f32_residual(const std::string& name);
  void write_step_state(int token, bool want_host_id);
  void enqueue_fused_step();
  void launch_fused_step(int seq_len);
  DecodeStepArgs step_args(int splits) const;
  void advance_epoch();

  ModelConfig config_;
  Options options_;
  int multiprocessors_ = 0;
  bool fused_ = false;
  hipStream_t stream_ = nullptr;
  // decode()'s timer, whose two events are created once with the model (on
  // its device) rather than per call.
  std::unique_ptr<GpuTimer> decode_timer_;

  elem_t* weight_block_ = nullptr;
  size_t weight_bytes_ = 0;
  const elem_t* embedding_ = nullptr;
  const elem_t* final_norm_ = nullptr;
  const elem_t* lm_head_ = nullptr;
  std::vector<LayerWeights> layers_;
  float* inv_freq_ = nullptr;
  float2* rope_table_ = nullptr;  // fused step, prefill q/k/v: [max_seq][head_dim / 2] (cos, sin)
  bool qkv_rope_ = false;         // prefill chunks rotate in the q/k/v projection's epilogue

  DeviceArena arena_;
  std::unique_ptr<KvCache> kv_cache_;

  elem_t* x_ = nullptr;           // [max_tokens][hidden]
  elem_t* normed_ = nullptr;      // [max_tokens][hidden]
  elem_t* qkv_ = nullptr;         // [max_tokens][q_dim + 2 kv_dim]
  elem_t* q_heads_ = nullptr;     // [num_heads][max_tokens][head_dim]
  elem_t* attn_out_ = nullptr;    // [max_tokens][q_dim]
  elem_t* proj_out_ = nullptr;    // [max_tokens][hidden]
  elem_t* gate_up_ = nullptr;     // [max_tokens][2 ffn]
  elem_t* act_ = nullptr;         // [max_tokens][ffn]
  float* logits_ = nullptr;       // [vocab]
  float* attention_scratch_ = nullptr;
  float* gemm_workspace_ = nullptr;  // split-K partial products of the prefill projections
  size_t gemm_workspace_size_ = 0;
  int32_t* token_ids_ = nullptr;  // [max_tokens]
  int32_t* sampled_id_ = nullptr;
  // Fused decode state.
  float* resid_ = nullptr;        // [hidden] fp32 residual sum
  // The fused step's state on the device, {token, position, want_host_id}:
  // one copy per call from pinned_state_. position_dev_ points into it.
  int32_t* step_state_ = nullptr;
  int32_t* position_dev_ = nullptr;
  unsigned long long* argmax_partials_ = nullptr;
  int32_t* history_ = nullptr;    // [max_seq + 1]
  unsigned long long* exchange_words_ = nullptr;  // decode_exchange_words(...)
  // Raised by an exchange wait that gave up. Host-coherent pinned memory the
  // kernels write directly, so the host reads it after the synchronization
  // every step ends with, at no cost to the device.
  int* exchange_status_ = nullptr;       // device address of exchange_status_host_
  int* exchange_status_host_ = nullptr;
  int32_t* step_id_ = nullptr;       // device address of step_id_host_
  int32_t* step_id_host_ = nullptr;  // host-coherent: the greedy step's id, written by its output head
  // Whether any exchange grid can run (its waits then need checking).
  bool exchange_in_use() const { return exchange_enabled_ || exchange_split_slots_ > 0 || layer_grid_enabled_; }
  bool layer_grid_enabled_ = false;
  // After a synchronization: throws lcr::Error, clearing the words and the
  // status, when a wait of the steps since the last check gave up.
  void check_exchange();
  bool exchange_enabled_ = false;
  bool exchange_oproj_ = false;
  int exchange_split_slots_ = 0;  // 0: split attention keeps separate kernels
  uint32_t* epoch_ = nullptr;     // [1] decode steps completed (exchange tags)
  int32_t* pinned_state_ = nullptr;  // host {token, position, want_host_id}

  // A captured graph and its executable, destroyed together: the graph is
  // kept for as long as the executable made from it.
  struct CapturedStep {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
  };
  static void destroy_captured(CapturedStep& c);
  // Captures what `enqueue` launches on the stream and instantiates it.
  template <typename Enqueue>
  CapturedStep capture_step(Enqueue enqueue);
  std::map<int, CapturedStep> graphs_;  // by split count
  // Sampled steps' graphs, by split count, for the parameters in
  // sampled_params_ (other parameters capture them again).
  std::map<int, CapturedStep> sampled_graphs_;
  struct SampledParams {
    float temperature = 0.0f;
    int top_k = 0;
    float top_p = 0.0f;
    bool operator==(const SampledParams& o) const {
      return temperature == o.temperature && top_k == o.top_k && top_p == o.top_p;
    }
  } sampled_params_;
  float* uniforms_ = nullptr;        // [max_seq] draws of a sampled generation
  int32_t* draw_counter_ = nullptr;  // [1]
  void launch_sampled_step(int seq_len);
  void clear_sampled_graphs();
  hipGraph_t graph_template_ = nullptr;

  int position_ = 0;
  int max_tokens_ = 0;
  ForwardStats stats_;
  bool input_norm_done_ = false;
  bool capture_activations_ = false;
  // step_id_host_ (and sampled_id_) hold the argmax of logits_: the last call
  // that wrote them was a fused decode step, whose output head reduces its
  // logits to their argmax (the greedy sample's key and tie rule) and writes
  // the id to host-coherent memory too, or a greedy sample() of logits_. A
  // greedy sample() of logits_ then reads that id: no kernel, no copy.
  bool step_argmax_ready_ = false;
  // step_state_ on the device holds {device_token_, position_, 1}: the last
  // call was a fused decode(), whose step wrote its argmax as the next token
  // and advanced the position, and nothing has moved the position since. A
  // decode() of that token then has nothing to copy. Cleared by every call
  // that writes the position or the step state.
  bool step_state_current_ = false;
  int32_t device_token_ = -1;
  std::vector<Tap> taps_;
  Profiler profiler_;
};

}  // namespace lcr
