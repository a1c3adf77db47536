#include "model.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <sstream>

#include "hip_utils.h"
#include "kernels.h"
#include "kernels/fill.h"

namespace lcr {
namespace {

// Largest split count attention ever uses, so its scratch is sized once
// (the reference's src/model.cu:23).
constexpr int kMaxAttentionSplits = 64;
constexpr int kMaxLmHeadBlocks = 1024;

}  // namespace

Model::Model(const std::string& model_dir, const Options& options) : options_(options) {
  HIP_CHECK(hipSetDevice(options.device));
  const DeviceInfo device = query_device(options.device);
  multiprocessors_ = device.multiprocessors;

  config_ = ModelConfig::load(model_dir);
  LCR_CHECK(options_.max_seq > 0, "max_seq must be positive");
  LCR_CHECK(options_.prefill_chunk > 0, "prefill chunk must be positive");
  max_tokens_ = std::min(options_.prefill_chunk, options_.max_seq);

  HIP_CHECK(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  decode_timer_ = std::make_unique<GpuTimer>();

  {
    const SafetensorsArchive archive(model_dir);
    load_weights(archive);
  }
  kv_cache_ = std::make_unique<KvCache>(config_, options_.max_seq, options_.kv_layout,
                                        options_.page_size);

  const std::vector<float> inv_freq = compute_rope_inv_freq(config_);
  HIP_CHECK(hipMalloc(&inv_freq_, inv_freq.size() * sizeof(float)));
  HIP_CHECK(hipMemcpy(inv_freq_, inv_freq.data(), inv_freq.size() * sizeof(float),
                      hipMemcpyHostToDevice));

  HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&pinned_state_), 3 * sizeof(int32_t),
                          hipHostMallocDefault));
  pinned_state_[0] = 0;
  pinned_state_[1] = 0;
  pinned_state_[2] = 0;
  // Before the arena: allocating it clears the exchange state, status included.
  HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&exchange_status_host_), sizeof(int),
                          hipHostMallocCoherent | hipHostMallocMapped));
  *exchange_status_host_ = 0;
  HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&exchange_status_), exchange_status_host_, 0));
  HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&step_id_host_), sizeof(int32_t),
                          hipHostMallocCoherent | hipHostMallocMapped));
  *step_id_host_ = 0;
  HIP_CHECK(hipHostGetDevicePointer(reinterpret_cast<void**>(&step_id_), step_id_host_, 0));
  allocate_arena();

  fused_ = options_.fused_decode &&
           decode_step_supported(config_.hidden_size, config_.intermediate_size,
                                 config_.num_heads, config_.num_kv_heads, config_.head_dim) &&
           config_.vocab_size > 0;
  {
    const bool paged = options_.kv_layout == KvLayout::kPaged;
    exchange_enabled_ = fused_ && options_.decode_exchange &&
                        decode_exchange_fits(config_.num_heads, config_.num_kv_heads, config_.head_dim,
                                             config_.hidden_size, paged, multiprocessors_, false);
    exchange_split_slots_ = fused_ && options_.decode_exchange && options_.exchange_split
                                ? decode_split_exchange_slots(config_.num_heads, config_.num_kv_heads,
                                                              config_.head_dim, paged, multiprocessors_)
                                : 0;
    exchange_oproj_ = exchange_enabled_ && options_.exchange_oproj &&
                      decode_exchange_fits(config_.num_heads, config_.num_kv_heads, config_.head_dim,
                                           config_.hidden_size, paged, multiprocessors_, true);
    layer_grid_enabled_ = fused_ && options_.decode_exchange && options_.layer_grid &&
                          decode_layer_grid_fits(config_.hidden_size, config_.intermediate_size, config_.num_heads,
                                                 config_.num_kv_heads, config_.head_dim, paged, multiprocessors_);
  }

  // The table serves the fused decode step and the prefill q/k/v projection
  // with RoPE in its epilogue.
  qkv_rope_ = config_.head_dim == 64 || config_.head_dim == 128;
  if (fused_ || qkv_rope_) {
    const int half = config_.head_dim / 2;
    HIP_CHECK(hipMalloc(&rope_table_, static_cast<size_t>(options_.max_seq) * half * sizeof(float2)));
    build_rope_table(rope_table_, inv_freq_, options_.max_seq, half, stream_);
    HIP_CHECK(hipStreamSynchronize(stream_));
  }

  stats_.kv_bytes_per_position = config_.kv_bytes_per_token(sizeof(elem_t));
  stats_.weight_bytes_per_token = weight_bytes_per_token(config_, sizeof(elem_t));
}

Model::~Model() {
  if (stream_ != nullptr) (void)hipStreamSynchronize(stream_);
  for (auto& kv : graphs_) destroy_captured(kv.second);
  for (auto& kv : sampled_graphs_) destroy_captured(kv.second);
  graphs_.clear();
  sampled_graphs_.clear();
  if (pinned_state_ != nullptr) (void)hipHostFree(pinned_state_);
  if (exchange_status_host_ != nullptr) (void)hipHostFree(exchange_status_host_);
  if (step_id_host_ != nullptr) (void)hipHostFree(step_id_host_);
  if (stream_ != nullptr) (void)hipStreamDestroy(stream_);
  (void)hipFree(weight_block_);
  (void)hipFree(inv_freq_);
  (void)hipFree(rope_table_);
}

// Layout and checks follow the reference's src/model.cu:112-213: one device
// block in reading order, 256-byte aligned pieces, q/k/v and gate/up
// concatenated by rows, tied output head = embedding.
void Model::load_weights(const SafetensorsArchive& archive) {
  layers_.assign(static_cast<size_t>(config_.num_layers), LayerWeights{});
  struct Block {
    const elem_t** destination;
    std::vector<const TensorView*> pieces;
    size_t bytes = 0;
  };
  std::vector<Block> blocks;
  auto check = [&](const std::string& name, const std::vector<int64_t>& shape) {
    const TensorView& t = archive.get(name);
    LCR_CHECK(t.dtype == kElemDType,
              "tensor \"" << name << "\" is " << dtype_name(t.dtype) << " but this build computes in "
                          << kElemName << "; rebuild with -DLCR_DTYPE="
                          << (kElemDType == DType::kBF16 ? "fp16" : "bf16"));
    t.expect_shape(shape);
    return &t;
  };
  auto add = [&](const elem_t** dest, std::vector<const TensorView*> pieces) {
    Block b;
    b.destination = dest;
    for (const TensorView* t : pieces) b.bytes += t->nbytes;
    b.pieces = std::move(pieces);
    blocks.push_back(std::move(b));
  };
  const int64_t hidden = config_.hidden_size;
  const int64_t ffn = config_.intermediate_size;
  const int64_t q_dim = config_.q_dim();
  const int64_t kv_dim = config_.kv_dim();

  add(&embedding_, {check("model.embed_tokens.weight", {config_.vocab_size, hidden})});
  for (int i = 0; i < config_.num_layers; ++i) {
    LayerWeights& w = layers_[static_cast<size_t>(i)];
    const std::string p = "model.layers." + std::to_string(i) + ".";
    add(&w.input_norm, {check(p + "input_layernorm.weight", {hidden})});
    add(&w.qkv_proj, {check(p + "self_attn.q_proj.weight", {q_dim, hidden}),
                      check(p + "self_attn.k_proj.weight", {kv_dim, hidden}),
                      check(p + "self_attn.v_proj.weight", {kv_dim, hidden})});
    add(&w.o_proj, {check(p + "self_attn.o_proj.weight", {hidden, q_dim})});
    add(&w.post_attention_norm, {check(p + "post_attention_layernorm.weight", {hidden})});
    add(&w.gate_up_proj, {check(p + "mlp.gate_proj.weight", {ffn, hidden}),
                          check(p + "mlp.up_proj.weight", {ffn, hidden})});
    add(&w.down_proj, {check(p + "mlp.down_proj.weight", {hidden, ffn})});
  }
  add(&final_norm_, {check("model.norm.weight", {hidden})});
  const bool has_lm_head = archive.has("lm_head.weight");
  if (has_lm_head) {
    add(&lm_head_, {check("lm_head.weight", {config_.vocab_size, hidden})});
  } else {
    LCR_CHECK(config_.tie_word_embeddings,
              "the checkpoint has no lm_head.weight and config.json does not say the "
              "embeddings are tied");
  }

  size_t total = 0;
  for (const Block& b : blocks) total = align_up(total, 256) + b.bytes;
  HIP_CHECK(hipMalloc(&weight_block_, total));
  weight_bytes_ = total;
  size_t offset = 0;
  for (const Block& b : blocks) {
    offset = align_up(offset, 256);
    char* base = reinterpret_cast<char*>(weight_block_) + offset;
    size_t piece_offset = 0;
    for (const TensorView* t : b.pieces) {
      HIP_CHECK(hipMemcpy(base + piece_offset, t->data, t->nbytes, hipMemcpyHostToDevice));
      piece_offset += t->nbytes;
    }
    *b.destination = reinterpret_cast<const elem_t*>(base);
    offset += b.bytes;
  }
  if (!has_lm_head) lm_head_ = embedding_;
}

// The split-K workspace the prefill projections use: the largest the GEMM
// plans ask for over the four projection shapes at every chunk length up to
// the maximum chunk, so each chunk gets its preferred plan (a few thousand
// plan evaluations of a few dozen operations each, once per model).
size_t Model::gemm_workspace_bytes() const {
  const int hidden = config_.hidden_size;
  const int ffn = config_.intermediate_size;
  const int shapes[4][2] = {{config_.q_dim() + 2 * config_.kv_dim(), hidden},
                            {hidden, config_.q_dim()},
                            {2 * ffn, hidden},
                            {hidden, ffn}};
  size_t bytes = 0;
  for (int T = 2; T <= max_tokens_; ++T) {
    for (const auto& s : shapes) bytes = std::max(bytes, lcr_gemm_workspace_bytes(T, s[0], s[1]));
  }
  return align_up(bytes, 256);
}

void Model::allocate_arena() {
  const size_t H = static_cast<size_t>(config_.hidden_size);
  const size_t F = static_cast<size_t>(config_.intermediate_size);
  const size_t T = static_cast<size_t>(max_tokens_);
  const size_t e = sizeof(elem_t);
  const size_t qkv_w = static_cast<size_t>(config_.q_dim() + 2 * config_.kv_dim());
  const size_t qd = static_cast<size_t>(config_.q_dim());
  const size_t attn_floats = std::max<size_t>(
      decode_attention_scratch_floats(config_.num_heads, config_.head_dim, kMaxAttentionSplits),
      sample_scratch_floats(config_.vocab_size, 0));
  const size_t sizes[] = {
      T * H * e,                                 // x_
      T * H * e,                                 // normed_
      T * qkv_w * e,                             // qkv_
      T * qd * e,                                // q_heads_
      T * qd * e,                                // attn_out_
      T * H * e,                                 // proj_out_
      T * 2 * F * e,                             // gate_up_
      T * F * e,                                 // act_
      static_cast<size_t>(config_.vocab_size) * sizeof(float),  // logits_
      attn_floats * sizeof(float),               // attention_scratch_
      T * sizeof(int32_t),                       // token_ids_
      sizeof(int32_t),                           // sampled_id_
      H * sizeof(float),                         // resid_
      3 * sizeof(int32_t),                       // step_state_
      kMaxLmHeadBlocks * sizeof(unsigned long long),                  // argmax_partials_
      (static_cast<size_t>(options_.max_seq) + 1) * sizeof(int32_t),  // history_
      gemm_workspace_bytes(),                                         // gemm_workspace_
      static_cast<size_t>(options_.max_seq) * sizeof(float),          // uniforms_
      sizeof(int32_t),                                                // draw_counter_
      decode_exchange_words(config_.num_heads, config_.head_dim) * sizeof(unsigned long long),  // exchange_words_
      sizeof(uint32_t),                                               // epoch_
  };
  size_t total = 0;
  for (size_t s : sizes) total = align_up(total, 256) + s;
  arena_.reserve(total + 4096);
  x_ = arena_.alloc<elem_t>(T * H);
  normed_ = arena_.alloc<elem_t>(T * H);
  qkv_ = arena_.alloc<elem_t>(T * qkv_w);
  q_heads_ = arena_.alloc<elem_t>(T * qd);
  attn_out_ = arena_.alloc<elem_t>(T * qd);
  proj_out_ = arena_.alloc<elem_t>(T * H);
  gate_up_ = arena_.alloc<elem_t>(T * 2 * F);
  act_ = arena_.alloc<elem_t>(T * F);
  logits_ = arena_.alloc<float>(static_cast<size_t>(config_.vocab_size));
  attention_scratch_ = arena_.alloc<float>(attn_floats);
  token_ids_ = arena_.alloc<int32_t>(T);
  sampled_id_ = arena_.alloc<int32_t>(1);
  resid_ = arena_.alloc<float>(H);
  step_state_ = arena_.alloc<int32_t>(3);
  position_dev_ = step_state_ + 1;
  argmax_partials_ = arena_.alloc<unsigned long long>(kMaxLmHeadBlocks);
  history_ = arena_.alloc<int32_t>(static_cast<size_t>(options_.max_seq) + 1);
  gemm_workspace_size_ = gemm_workspace_bytes();
  gemm_workspace_ = gemm_workspace_size_ > 0 ? arena_.alloc<float>(gemm_workspace_size_ / sizeof(float)) : nullptr;
  uniforms_ = arena_.alloc<float>(static_cast<size_t>(options_.max_seq));
  draw_counter_ = arena_.alloc<int32_t>(1);
  exchange_words_ = arena_.alloc<unsigned long long>(decode_exchange_words(config_.num_heads, config_.head_dim));
  epoch_ = arena_.alloc<uint32_t>(1);
  HIP_CHECK(hipMemset(epoch_, 0, sizeof(uint32_t)));
  clear_exchange();
  HIP_CHECK(hipMemset(token_ids_, 0, T * sizeof(int32_t)));
  HIP_CHECK(hipMemset(step_state_, 0, 3 * sizeof(int32_t)));
}

void Model::reset() {
  position_ = 0;
  step_argmax_ready_ = false;
  step_state_current_ = false;
  taps_.clear();
}

// The split count of the decode step. The reference sizes it for one block
// per (kv head, split), two per multiprocessor (src/kernels/attention.cu:
// 419-431). Here, as measured on MI355X:
//  - below 4096 positions, a single split: one 8-wave block per query head,
//    up to 8 tiles per wave, no merge pass;
//  - below 16384, ceil(CUs / num_heads) splits of per-query-head blocks
//    (about one block per compute unit);
//  - from 16384 on the step is bound by the cache bytes: ceil(CUs /
//    num_kv_heads) splits, which the kernel runs as one block per (kv head,
//    split) loading each key and value once for the whole group.
// Always at least 512 positions (one 64-position tile per wave) per split and
// at most 64 splits.
static int decode_attention_splits(int num_heads, int num_kv_heads, int seq_len, int compute_units) {
  if (seq_len < 4096) return 1;
  const int per = seq_len < 16384 ? std::max(1, num_heads) : std::max(1, num_kv_heads);
  const int want = std::max(1, (compute_units + per - 1) / per);
  const int useful = std::max(1, seq_len / 512);
  return std::max(1, std::min(std::min(want, useful), kMaxAttentionSplits));
}

int Model::decode_splits(int seq_len) const {
  const int s = options_.attention_splits > 0
                    ? std::min(options_.attention_splits, kMaxAttentionSplits)
                    : decode_attention_splits(config_.num_heads, config_.num_kv_heads, seq_len,
                                              multiprocessors_);
  return std::max(1, std::min(s, seq_len));
}

const float* Model::prefill(const std::vector<int>& tokens) {
  LCR_CHECK(!tokens.empty(), "prefill needs at least one token");
  LCR_CHECK(position_ + static_cast<int>(tokens.size()) <= options_.max_seq,
            "prompt of " << tokens.size() << " tokens at position " << position_
                         << " exceeds the cache built for " << options_.max_seq);
  for (int t : tokens) {
    LCR_CHECK(t >= 0 && t < config_.vocab_size,
              "token id " << t << " is outside the vocabulary of " << config_.vocab_size);
  }
  step_argmax_ready_ = false;
  step_state_current_ = false;
  if (options_.prefill_via_decode) {
    GpuTimer timer;
    timer.start(stream_);
    const float* out = nullptr;
    for (int t : tokens) out = decode(t);
    timer.stop(stream_);
    stats_.last_prefill_ms = timer.elapsed_ms();
    return out;
  }
  GpuTimer timer;
  timer.start(stream_);
  size_t consumed = 0;
  while (consumed < tokens.size()) {
    const int chunk = static_cast<int>(std::min<size_t>(static_cast<size_t>(max_tokens_),
                                                        tokens.size() - consumed));
    if (chunk < kMinMfmaPrefillTokens) {
      for (int i = 0; i < chunk; ++i) decode(tokens[consumed + static_cast<size_t>(i)]);
      consumed += static_cast<size_t>(chunk);
      continue;
    }
    std::vector<int32_t> ids(tokens.begin() + static_cast<long>(consumed),
                             tokens.begin() + static_cast<long>(consumed) + chunk);
    HIP_CHECK(hipMemcpyAsync(token_ids_, ids.data(), ids.size() * sizeof(int32_t),
                             hipMemcpyHostToDevice, stream_));
    kv_cache_->reserve_length(position_ + chunk);
    launch_embedding_lookup(x_, embedding_, token_ids_, chunk, config_.hidden_size, stream_);
    run_layers(chunk, position_);
    step_argmax_ready_ = false;  // the chunk's logits, without their argmax
    step_state_current_ = false;
    position_ += chunk;
    consumed += static_cast<size_t>(chunk);
    // The ids buffer above is pageable host memory read by the async copy.
    HIP_CHECK(hipStreamSynchronize(stream_));
  }
  timer.stop(stream_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  stats_.last_prefill_ms = timer.elapsed_ms();
  if (profiler_.enabled()) profiler_.collect();
  return logits_;
}

// want_host_id: the step's output head also writes its greedy id to
// host-coherent memory (a call that returns to the host right after the step).
void Model::write_step_state(int token, bool want_host_id) {
  pinned_state_[0] = token;
  pinned_state_[1] = position_;
  pinned_state_[2] = want_host_id ? 1 : 0;
  HIP_CHECK(hipMemcpyAsync(step_state_, pinned_state_, 3 * sizeof(int32_t), hipMemcpyHostToDevice, stream_));
}

DecodeStepArgs Model::step_args(int splits) const {
  DecodeStepArgs a{};
  a.hidden = config_.hidden_size;
  a.ffn = config_.intermediate_size;
  a.num_heads = config_.num_heads;
  a.num_kv_heads = config_.num_kv_heads;
  a.head_dim = config_.head_dim;
  a.vocab = config_.vocab_size;
  a.eps = config_.rms_norm_eps;
  a.embedding = embedding_;
  a.final_norm = final_norm_;
  a.lm_head = lm_head_;
  a.inv_freq = inv_freq_;
  a.rope_table = rope_table_;
  a.token = step_state_;
  a.position = position_dev_;
  a.sampled = sampled_id_;
  a.next_token = step_state_;
  a.history = history_;
  a.history_len = options_.max_seq + 1;
  a.resid = resid_;
  a.q = q_heads_;
  a.attn = attn_out_;
  a.act = act_;
  a.logits = logits_;
  a.partials = attention_scratch_;
  a.argmax_partials = argmax_partials_;
  a.paged = options_.kv_layout == KvLayout::kPaged;
  a.splits = splits;
  a.compute_units = multiprocessors_;
  a.exchange = exchange_in_use() ? exchange_words_ : nullptr;
  a.exchange_single = exchange_enabled_;
  a.exchange_head = exchange_enabled_ && options_.exchange_head;
  a.layer_grid = layer_grid_enabled_;
  a.exchange_oproj = exchange_oproj_;
  a.exchange_split = exchange_split_slots_ > 0;
  a.exchange_slots = exchange_split_slots_;
  a.exchange_status = exchange_status_;
  a.exchange_spins = std::max(1, options_.exchange_spins);
  a.exchange_read_offset = options_.exchange_test_unwritten
                               ? static_cast<int>(decode_exchange_words(config_.num_heads, config_.head_dim) / 2)
                               : 0;
  a.epoch = epoch_;
  a.sampled_host = step_id_;
  a.want_host_id = step_state_ + 2;
  return a;
}

int Model::exchange_status() const {
  HIP_CHECK(hipStreamSynchronize(stream_));
  return __atomic_load_n(exchange_status_host_, __ATOMIC_ACQUIRE);
}

void Model::check_exchange() {
  if (!exchange_in_use() || __atomic_load_n(exchange_status_host_, __ATOMIC_ACQUIRE) == 0) return;
  clear_exchange();
  LCR_FAIL("a decode step's in-grid exchange wait gave up; its results are not valid");
}

void Model::advance_epoch() {
  uint32_t epoch = 0;
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipMemcpy(&epoch, epoch_, sizeof(uint32_t), hipMemcpyDeviceToHost));
  epoch += 1;
  HIP_CHECK(hipMemcpy(epoch_, &epoch, sizeof(uint32_t), hipMemcpyHostToDevice));
}

void Model::clear_exchange() {
  HIP_CHECK(hipStreamSynchronize(stream_));
  HIP_CHECK(hipMemset(exchange_words_, 0,
                      decode_exchange_words(config_.num_heads, config_.head_dim) * sizeof(unsigned long long)));
  HIP_CHECK(hipDeviceSynchronize());
  __atomic_store_n(exchange_status_host_, 0, __ATOMIC_RELEASE);
}

void Model::destroy_captured(CapturedStep& c) {
  if (c.exec != nullptr) (void)hipGraphExecDestroy(c.exec);
  if (c.graph != nullptr) (void)hipGraphDestroy(c.graph);
  c.exec = nullptr;
  c.graph = nullptr;
}

template <typename Enqueue>
Model::CapturedStep Model::capture_step(Enqueue enqueue) {
  CapturedStep c;
  HIP_CHECK(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
  try {
    enqueue();
  } catch (...) {
    hipGraph_t discard = nullptr;
    (void)hipStreamEndCapture(stream_, &discard);
    if (discard != nullptr) (void)hipGraphDestroy(discard);
    throw;
  }
  HIP_CHECK(hipStreamEndCapture(stream_, &c.graph));
  const hipError_t status = hipGraphInstantiate(&c.exec, c.graph, nullptr, nullptr, 0);
  if (status != hipSuccess) {
    destroy_captured(c);
    HIP_CHECK(status);
  }
  return c;
}

void Model::launch_fused_step(int seq_len) {
  const int splits = decode_splits(seq_len);
  const DecodeStepArgs args = step_args(splits);
  auto enqueue = [&]() {
    for (int layer = 0; layer < config_.num_layers; ++layer) {
      const LayerWeights& lw = layers_[static_cast<size_t>(layer)];
      LayerDevicePtrs w{lw.input_norm, lw.qkv_proj, lw.o_proj, lw.post_attention_norm,
                        lw.gate_up_proj, lw.down_proj};
      enqueue_decode_layer(args, w, kv_cache_->view(layer), layer, stream_);
    }
    enqueue_decode_head(args, stream_);
  };
  if (!options_.use_graph || synchronous_launches()) {
    enqueue();
    return;
  }
  auto it = graphs_.find(splits);
  if (it == graphs_.end()) it = graphs_.emplace(splits, capture_step(enqueue)).first;
  HIP_CHECK(hipGraphLaunch(it->second.exec, stream_));
}

const float* Model::decode(int token) {
  LCR_CHECK(position_ < options_.max_seq,
            "sequence reached " << position_ << " positions, the cache limit");
  LCR_CHECK(token >= 0 && token < config_.vocab_size,
            "token id " << token << " is outside the vocabulary of " << config_.vocab_size);
  step_argmax_ready_ = false;
  const bool fused_step = fused_ && !capture_activations_;
  // The previous fused step left this token, this position and the host-id
  // flag in the step state (the reference's greedy loop feeds the argmax
  // back): no copy.
  const bool state_current = fused_step && step_state_current_ && token == device_token_;
  step_state_current_ = false;
  GpuTimer& timer = *decode_timer_;
  timer.start(stream_);
  kv_cache_->reserve_length(position_ + 1);
  if (fused_step) {
    if (!state_current) write_step_state(token, true);
    launch_fused_step(position_ + 1);
  } else {
    pinned_state_[0] = token;
    HIP_CHECK(hipMemcpyAsync(token_ids_, &pinned_state_[0], sizeof(int32_t),
                             hipMemcpyHostToDevice, stream_));
    launch_embedding_lookup(x_, embedding_, token_ids_, 1, config_.hidden_size, stream_);
    run_layers(1, position_);
  }
  position_ += 1;
  timer.stop(stream_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  stats_.last_decode_ms = timer.elapsed_ms();
  check_exchange();
  step_argmax_ready_ = fused_step;
  if (fused_step) {
    device_token_ = __atomic_load_n(step_id_host_, __ATOMIC_ACQUIRE);
    step_state_current_ = true;
  }
  if (profiler_.enabled()) profiler_.collect();
  return logits_;
}

void Model::clear_sampled_graphs() {
  for (auto& kv : sampled_graphs_) destroy_captured(kv.second);
  sampled_graphs_.clear();
}

// One sampled step: the layers as in launch_fused_step, then the head with
// the sampler instead of the argmax.
void Model::launch_sampled_step(int seq_len) {
  const int splits = decode_splits(seq_len);
  const DecodeStepArgs args = step_args(splits);
  const SampledHead head{sampled_params_.temperature, sampled_params_.top_k, sampled_params_.top_p, uniforms_,
                         draw_counter_, options_.max_seq};
  auto enqueue = [&]() {
    for (int layer = 0; layer < config_.num_layers; ++layer) {
      const LayerWeights& lw = layers_[static_cast<size_t>(layer)];
      LayerDevicePtrs w{lw.input_norm, lw.qkv_proj, lw.o_proj, lw.post_attention_norm,
                        lw.gate_up_proj, lw.down_proj};
      enqueue_decode_layer(args, w, kv_cache_->view(layer), layer, stream_);
    }
    enqueue_decode_head_sampled(args, head, stream_);
  };
  if (!options_.use_graph || synchronous_launches()) {
    enqueue();
    return;
  }
  auto it = sampled_graphs_.find(splits);
  if (it == sampled_graphs_.end()) it = sampled_graphs_.emplace(splits, capture_step(enqueue)).first;
  HIP_CHECK(hipGraphLaunch(it->second.exec, stream_));
}

std::vector<int> Model::generate_sampled(int first_token, int steps, float temperature, int top_k,
                                         float top_p, const float* uniforms, double* elapsed_ms) {
  LCR_CHECK(fused_, "device-side sampled generation needs the fused decode path");
  step_argmax_ready_ = false;
  step_state_current_ = false;
  LCR_CHECK(steps >= 0, "steps must be non-negative");
  LCR_CHECK(temperature > 0.0f, "sampled generation needs a positive temperature (greedy: generate_greedy)");
  LCR_CHECK(top_p > 0.0f && top_p <= 1.0f, "top_p must be in (0, 1], got " << top_p);
  LCR_CHECK(steps == 0 || uniforms != nullptr, "sampled generation needs one draw per step");
  LCR_CHECK(first_token >= 0 && first_token < config_.vocab_size,
            "token id " << first_token << " is outside the vocabulary of " << config_.vocab_size);
  LCR_CHECK(position_ + steps <= options_.max_seq,
            "generating " << steps << " tokens at position " << position_
                          << " exceeds the cache built for " << options_.max_seq);
  std::vector<int> out(static_cast<size_t>(steps));
  if (steps == 0) {
    if (elapsed_ms) *elapsed_ms = 0.0;
    return out;
  }
  const SampledParams params{temperature, top_k, top_p};
  if (!(params == sampled_params_)) {
    clear_sampled_graphs();
    sampled_params_ = params;
  }
  const int start = position_;
  kv_cache_->reserve_length(position_ + steps);
  HIP_CHECK(hipMemcpy(uniforms_, uniforms, static_cast<size_t>(steps) * sizeof(float), hipMemcpyHostToDevice));
  // Capture every graph this run needs before timing it (a capture runs its
  // graph once, which moves the position and the counter: both are reset).
  HIP_CHECK(hipMemsetAsync(draw_counter_, 0, sizeof(int32_t), stream_));
  for (int s = 0; s < steps; ++s) {
    const int splits = decode_splits(start + s + 1);
    if (options_.use_graph && sampled_graphs_.find(splits) == sampled_graphs_.end()) {
      write_step_state(first_token, false);
      launch_sampled_step(start + s + 1);
      HIP_CHECK(hipStreamSynchronize(stream_));
    }
  }
  write_step_state(first_token, false);
  HIP_CHECK(hipMemsetAsync(draw_counter_, 0, sizeof(int32_t), stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  GpuTimer timer;
  timer.start(stream_);
  for (int s = 0; s < steps; ++s) launch_sampled_step(start + s + 1);
  timer.stop(stream_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  const double ms = timer.elapsed_ms();
  if (elapsed_ms) *elapsed_ms = ms;
  stats_.last_decode_ms = ms / steps;
  position_ = start + steps;
  std::vector<int32_t> ids(static_cast<size_t>(steps));
  HIP_CHECK(hipMemcpy(ids.data(), history_ + start + 1, ids.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
  check_exchange();
  for (int s = 0; s < steps; ++s) {
    LCR_CHECK(ids[static_cast<size_t>(s)] >= 0 && ids[static_cast<size_t>(s)] < config_.vocab_size,
              "sampling produced token id " << ids[static_cast<size_t>(s)] << ", outside the vocabulary");
    out[static_cast<size_t>(s)] = ids[static_cast<size_t>(s)];
  }
  return out;
}

std::vector<int> Model::generate_greedy(int first_token, int steps, double* elapsed_ms) {
  LCR_CHECK(fused_, "device-side greedy generation needs the fused decode path");
  step_argmax_ready_ = false;
  step_state_current_ = false;
  LCR_CHECK(steps >= 0, "steps must be non-negative");
  LCR_CHECK(first_token >= 0 && first_token < config_.vocab_size,
            "token id " << first_token << " is outside the vocabulary of " << config_.vocab_size);
  LCR_CHECK(position_ + steps <= options_.max_seq,
            "generating " << steps << " tokens at position " << position_
                          << " exceeds the cache built for " << options_.max_seq);
  std::vector<int> out(static_cast<size_t>(steps));
  if (steps == 0) {
    if (elapsed_ms) *elapsed_ms = 0.0;
    return out;
  }
  const int start = position_;
  kv_cache_->reserve_length(position_ + steps);
  // Capture every graph this run needs before timing it.
  for (int s = 0; s < steps; ++s) {
    const int splits = decode_splits(start + s + 1);
    if (options_.use_graph && graphs_.find(splits) == graphs_.end()) {
      write_step_state(first_token, false);
      launch_fused_step(start + s + 1);  // captures, then runs once at `start`
      HIP_CHECK(hipStreamSynchronize(stream_));
    }
  }
  write_step_state(first_token, false);
  GpuTimer timer;
  timer.start(stream_);
  for (int s = 0; s < steps; ++s) launch_fused_step(start + s + 1);
  timer.stop(stream_);
  HIP_CHECK(hipStreamSynchronize(stream_));
  const double ms = timer.elapsed_ms();
  if (elapsed_ms) *elapsed_ms = ms;
  stats_.last_decode_ms = ms / steps;
  position_ = start + steps;
  std::vector<int32_t> ids(static_cast<size_t>(steps));
  HIP_CHECK(hipMemcpy(ids.data(), history_ + start + 1, static_cast<size_t>(steps) * sizeof(int32_t),
                      hipMemcpyDeviceToHost));
  check_exchange();
  for (int s = 0; s < steps; ++s) out[static_cast<size_t>(s)] = ids[static_cast<size_t>(s)];
  return out;
}

double Model::time_decode_kernel(const std::string& kernel, int launches,
                                 double* bytes_per_launch) {
  LCR_CHECK(fused_, "kernel timing needs the fused decode path");
  step_argmax_ready_ = false;
  step_state_current_ = false;
  LCR_CHECK(launches > 0, "launches must be positive");
  LCR_CHECK(position_ > 0, "time kernels after a prefill, so the step state is valid");
  const double H = config_.hidden_size, F = config_.intermediate_size, V = config_.vocab_size;
  const double qd = config_.q_dim(), kvd = config_.kv_dim();
  const double e = sizeof(elem_t);
  const int seq_len = position_;  // attention reads the positions present
  unsigned mask = 0;
  bool argmax_only = false;
  bool head_with_argmax = false;
  double bytes = 0.0;
  if (kernel == "qkv") {
    mask = kDecodeQkv;
    bytes = (qd + 2 * kvd) * H * e + H * e + H * 4 + (qd + 2 * kvd) * e;
  } else if (kernel == "qkv_attention") {
    // The exchange grid of q/k/v and attention when the step uses it, else
    // the two kernels.
    mask = kDecodeQkv | kDecodeAttention;
    bytes = (qd + 2 * kvd) * H * e + H * e + H * 4 + (qd + 2 * kvd) * e + 2.0 * kvd * seq_len * e + qd * e;
  } else if (kernel == "qkv_attention_oproj") {
    // The exchange grid of q/k/v, attention and o_proj when the step uses
    // it, else what runs in its place.
    mask = kDecodeQkv | kDecodeAttention | kDecodeOProj;
    bytes = (qd + 2 * kvd) * H * e + H * e + H * 4 + (qd + 2 * kvd) * e + 2.0 * kvd * seq_len * e + qd * e +
            H * qd * e + 2 * H * 4;
  } else if (kernel == "layer") {
    // The whole layer: the layer grid when the step uses it, else the
    // kernels that run in its place.
    mask = kDecodeAll;
    bytes = ((qd + 2 * kvd) * H + H * qd + 2 * F * H + H * F) * e + 2 * H * e + 2.0 * kvd * seq_len * e +
            2 * H * 4;
  } else if (kernel == "attention") {
    mask = kDecodeAttention;
    bytes = 2.0 * kvd * seq_len * e + qd * e + qd * e;
  } else if (kernel == "o_proj") {
    mask = kDecodeOProj;
    bytes = H * qd * e + qd * e + 2 * H * 4;
  } else if (kernel == "gate_up") {
    mask = kDecodeGateUp;
    bytes = 2 * F * H * e + H * e + H * 4 + F * e;
  } else if (kernel == "down") {
    mask = kDecodeDown;
    bytes = H * F * e + F * e + 2 * H * 4;
  } else if (kernel == "lm_head") {
    bytes = V * H * e + H * e + H * 4 + V * 4;
  } else if (kernel == "argmax") {
    argmax_only = true;
    bytes = 8.0 * lm_head_blocks(config_.vocab_size, multiprocessors_) + 3 * 4;
  } else if (kernel == "head") {
    // The output head as the step runs it: lm_head and the argmax (folded
    // into lm_head's grid when the step exchanges words, else the one-block
    // kernel after it).
    head_with_argmax = true;
    bytes = V * H * e + H * e + H * 4 + V * 4 + 8.0 * lm_head_blocks(config_.vocab_size, multiprocessors_) + 3 * 4;
  } else {
    LCR_FAIL("unknown decode kernel \"" << kernel << "\"");
  }
  if (bytes_per_launch) *bytes_per_launch = bytes;
  // Each launch of an exchange grid tags its broadcast words with its own
  // slot of the epoch, so one timing graph holds at most that many.
  const bool exchange_grid = exchange_in_use() && (mask & kDecodeQkv) && (mask & kDecodeAttention);
  LCR_CHECK(!exchange_grid || launches <= kExchangeTagSlots,
            "timing an exchange grid takes at most " << kExchangeTagSlots << " launches, got " << launches);
  pinned_state_[1] = position_ - 1;  // the step that produced the current cache length
  HIP_CHECK(hipMemcpyAsync(position_dev_, &pinned_state_[1], sizeof(int32_t), hipMemcpyHostToDevice,
                           stream_));
  const DecodeStepArgs args = step_args(decode_splits(seq_len));
  // The launches are captured back to back into one graph (cycling through the
  // layers, so each launch streams weights no earlier launch left in a cache)
  // and the graph is timed between two events: the mean launch time then
  // excludes the host's enqueue cost, as a profiler's kernel duration does.
  auto enqueue = [&]() {
    for (int i = 0; i < launches; ++i) {
      const int layer = i % config_.num_layers;
      if (argmax_only) {
        enqueue_decode_argmax(args, stream_);
      } else if (mask == 0) {
        enqueue_decode_head(args, stream_, head_with_argmax);
      } else {
        const LayerWeights& lw = layers_[static_cast<size_t>(layer)];
        LayerDevicePtrs w{lw.input_norm, lw.qkv_proj, lw.o_proj, lw.post_attention_norm,
                          lw.gate_up_proj, lw.down_proj};
        enqueue_decode_layer(args, w, kv_cache_->view(layer), layer, stream_, mask, i);
      }
    }
  };
  CapturedStep timing = capture_step(enqueue);
  hipEvent_t start = nullptr, stop = nullptr;
  float ms = 0.0f;
  try {
    HIP_CHECK(hipEventCreate(&start));
    HIP_CHECK(hipEventCreate(&stop));
    HIP_CHECK(hipGraphLaunch(timing.exec, stream_));  // warm-up replay
    // A new epoch for the timed replay, so no exchange word of the warm-up
    // replay passes for one of its own, and another after it, so none of the
    // timed replay's words passes for one of the next decode step (whose
    // launches use the same slots, one per layer).
    advance_epoch();
    HIP_CHECK(hipEventRecord(start, stream_));
    HIP_CHECK(hipGraphLaunch(timing.exec, stream_));
    HIP_CHECK(hipEventRecord(stop, stream_));
    HIP_CHECK(hipEventSynchronize(stop));
    HIP_CHECK(hipEventElapsedTime(&ms, start, stop));
    advance_epoch();
    check_exchange();
  } catch (...) {
    if (start != nullptr) (void)hipEventDestroy(start);
    if (stop != nullptr) (void)hipEventDestroy(stop);
    destroy_captured(timing);
    throw;
  }
  (void)hipEventDestroy(start);
  (void)hipEventDestroy(stop);
  destroy_captured(timing);
  return static_cast<double>(ms) / launches;
}

void Model::set_position(int position) {
  LCR_CHECK(position >= 0 && position <= options_.max_seq,
            "position " << position << " outside [0, " << options_.max_seq << "]");
  kv_cache_->reserve_length(position);
  position_ = position;
  step_state_current_ = false;
}

void Model::fill_kv_normal(uint64_t seed, float stddev) {
  fill_normal(kv_cache_->key_pool(), kv_cache_->pool_elements(), seed, stddev, stream_);
  fill_normal(kv_cache_->value_pool(), kv_cache_->pool_elements(), seed ^ 0x5bf03635f0a5c3a9ull,
              stddev, stream_);
  HIP_CHECK(hipStreamSynchronize(stream_));
}

// The reference's run_layers (src/model.cu:370-484) on the kernel ABI: the
// unfused path, used for prefill chunks and whenever the fused kernels do not
// cover the model's geometry or activations are being captured.
void Model::run_layers(int tokens, int start_position) {
  const int hidden = config_.hidden_size;
  const int ffn = config_.intermediate_size;
  input_norm_done_ = false;
  if (capture_activations_) {
    taps_.clear();
    capture("embed", x_, tokens, hidden);
  }
  const int qkv_stride = config_.q_dim() + 2 * config_.kv_dim();
  const bool paged = options_.kv_layout == KvLayout::kPaged;
  for (int layer = 0; layer < config_.num_layers; ++layer) {
    const LayerWeights& w = layers_[static_cast<size_t>(layer)];
    if (!input_norm_done_) {
      ProfileScope scope(&profiler_, "rmsnorm", stream_);
      launch_rmsnorm(normed_, x_, w.input_norm, tokens, hidden, config_.rms_norm_eps, stream_);
    }
    input_norm_done_ = false;
    const KvCacheView view = kv_cache_->view(layer);
    if (tokens > 1 && qkv_rope_) {
      ProfileScope scope(&profiler_, "qkv_proj + rope + kv write", stream_);
      launch_gemm_qkv_rope(q_heads_, view, normed_, w.qkv_proj, rope_table_, tokens, config_.num_heads, hidden,
                           start_position, paged, gemm_workspace_, gemm_workspace_size_, stream_);
    } else {
      {
        ProfileScope scope(&profiler_, "qkv_proj", stream_);
        if (tokens == 1) {
          launch_gemv(qkv_, false, w.qkv_proj, normed_, qkv_stride, hidden, stream_);
        } else {
          launch_gemm(qkv_, false, normed_, w.qkv_proj, tokens, qkv_stride, hidden, gemm_workspace_,
                      gemm_workspace_size_, stream_);
        }
      }
      ProfileScope scope(&profiler_, "rope + kv write", stream_);
      launch_rope_q(q_heads_, qkv_, inv_freq_, tokens, start_position, config_.num_heads,
                    config_.head_dim, qkv_stride, stream_);
      launch_rope_write_kv(view, qkv_ + config_.q_dim(), qkv_ + config_.q_dim() + config_.kv_dim(),
                           inv_freq_, tokens, start_position, paged, qkv_stride, stream_);
    }
    {
      ProfileScope scope(&profiler_, "attention", stream_);
      if (tokens == 1) {
        attention_decode(layer, start_position);
      } else {
        attention_prefill(layer, tokens, start_position);
      }
    }
    if (tokens > 1) {
      ProfileScope scope(&profiler_, "o_proj + residual+rmsnorm", stream_);
      launch_gemm_residual_rmsnorm(normed_, x_, proj_out_, attn_out_, w.o_proj, w.post_attention_norm, tokens,
                                   hidden, config_.q_dim(), config_.rms_norm_eps, gemm_workspace_,
                                   gemm_workspace_size_, stream_);
    } else {
      {
        ProfileScope scope(&profiler_, "o_proj", stream_);
        launch_gemv(proj_out_, false, w.o_proj, attn_out_, hidden, config_.q_dim(), stream_);
      }
      ProfileScope scope(&profiler_, "residual+rmsnorm", stream_);
      launch_add_residual_rmsnorm(normed_, x_, proj_out_, w.post_attention_norm, tokens, hidden,
                                  config_.rms_norm_eps, stream_);
    }
    if (tokens > 1 && ffn % 16 == 0) {
      ProfileScope scope(&profiler_, "gate/up+swiglu", stream_);
      launch_gemm_swiglu(act_, normed_, w.gate_up_proj, tokens, ffn, hidden, gemm_workspace_,
                         gemm_workspace_size_, stream_);
    } else {
      {
        ProfileScope scope(&profiler_, "gate/up", stream_);
        if (tokens == 1) {
          launch_gemv(gate_up_, false, w.gate_up_proj, normed_, 2 * ffn, hidden, stream_);
        } else {
          launch_gemm(gate_up_, false, normed_, w.gate_up_proj, tokens, 2 * ffn, hidden,
                      gemm_workspace_, gemm_workspace_size_, stream_);
        }
      }
      {
        ProfileScope scope(&profiler_, "swiglu", stream_);
        launch_swiglu_strided(act_, gate_up_, gate_up_ + ffn, tokens, ffn, 2 * ffn, stream_);
      }
    }
    {
      // The MLP residual join fuses with the norm that comes next: the next
      // layer's input norm, or the final norm after the last layer.
      const elem_t* next = (layer + 1 < config_.num_layers)
                               ? layers_[static_cast<size_t>(layer + 1)].input_norm
                               : final_norm_;
      if (tokens > 1) {
        ProfileScope scope(&profiler_, "down + residual+rmsnorm", stream_);
        launch_gemm_residual_rmsnorm(normed_, x_, proj_out_, act_, w.down_proj, next, tokens, hidden, ffn,
                                     config_.rms_norm_eps, gemm_workspace_, gemm_workspace_size_, stream_);
      } else {
        {
          ProfileScope scope(&profiler_, "down", stream_);
          launch_gemv(proj_out_, false, w.down_proj, act_, hidden, ffn, stream_);
        }
        ProfileScope scope(&profiler_, "residual+rmsnorm", stream_);
        launch_add_residual_rmsnorm(normed_, x_, proj_out_, next, tokens, hidden, config_.rms_norm_eps, stream_);
      }
      input_norm_done_ = true;
    }
    if (capture_activations_) capture("layer_" + std::to_string(layer), x_, tokens, hidden);
  }
  if (!input_norm_done_) {
    ProfileScope scope(&profiler_, "final norm", stream_);
    launch_rmsnorm(normed_, x_, final_norm_, tokens, hidden, config_.rms_norm_eps, stream_);
  }
  input_norm_done_ = false;
  if (capture_activations_) capture("final_norm", normed_, tokens, hidden);
  const elem_t* last = normed_ + static_cast<int64_t>(tokens - 1) * hidden;
  {
    ProfileScope scope(&profiler_, "lm_head", stream_);
    launch_gemv(logits_, true, lm_head_, last, config_.vocab_size, hidden, stream_);
  }
}

void Model::attention_prefill(int layer, int tokens, int start_position) {
  const float scale = 1.0f / std::sqrt(static_cast<float>(config_.head_dim));
  launch_prefill_attention(attn_out_, q_heads_, kv_cache_->view(layer), config_.num_heads,
                           config_.heads_per_kv(), tokens, start_position, scale,
                           options_.kv_layout == KvLayout::kPaged, stream_);
}

void Model::attention_decode(int layer, int position) {
  const int seq_len = position + 1;
  const float scale = 1.0f / std::sqrt(static_cast<float>(config_.head_dim));
  launch_decode_attention(attn_out_, q_heads_, kv_cache_->view(layer), config_.num_heads,
                          config_.heads_per_kv(), seq_len, scale,
                          options_.kv_layout == KvLayout::kPaged, decode_splits(seq_len),
                          attention_scratch_, stream_);
}

void Model::capture(const std::string& name, const elem_t* source, int tokens, int width) {
  const size_t count = static_cast<size_t>(tokens) * width;
  std::vector<elem_t> host(count);
  HIP_CHECK(hipMemcpyAsync(host.data(), source, count * sizeof(elem_t), hipMemcpyDeviceToHost, stream_));
  HIP_CHECK(hipStreamSynchronize(stream_));
  Tap tap;
  tap.name = name;
  tap.tokens = tokens;
  tap.width = width;
  tap.values.resize(count);
  for (size_t i = 0; i < count; ++i) tap.values[i] = elem_to_float(host[i]);
  taps_.push_back(std::move(tap));
}

int Model::sample(const float* device_logits, float temperature, int top_k, float top_p,
                  float uniform) {
  // A greedy pick of the logits the last fused decode step wrote (decode()
  // has synchronised with it) reads the id that step's output head already
  // wrote to host-coherent memory; anything else runs the sampler.
  const bool own_logits = device_logits == logits_;
  int32_t id = 0;
  if (temperature <= 0.0f && own_logits && step_argmax_ready_) {
    id = __atomic_load_n(step_id_host_, __ATOMIC_ACQUIRE);
  } else {
    step_argmax_ready_ = false;
    launch_sample(sampled_id_, device_logits, config_.vocab_size, temperature, top_k, top_p, uniform,
                  attention_scratch_, stream_);
    HIP_CHECK(hipMemcpyAsync(&id, sampled_id_, sizeof(int32_t), hipMemcpyDeviceToHost, stream_));
    HIP_CHECK(hipStreamSynchronize(stream_));
    if (temperature <= 0.0f && own_logits) {
      __atomic_store_n(step_id_host_, id, __ATOMIC_RELEASE);
      step_argmax_ready_ = true;
    }
  }
  LCR_CHECK(id >= 0 && id < config_.vocab_size,
            "sampling produced token id " << id << ", outside the vocabulary");
  return static_cast<int>(id);
}

std::vector<float> Model::logits_to_host(const float* device_logits) const {
  std::vector<float> host(static_cast<size_t>(config_.vocab_size));
  HIP_CHECK(hipMemcpy(host.data(), device_logits, host.size() * sizeof(float), hipMemcpyDeviceToHost));
  return host;
}

}  // namespace lcr
