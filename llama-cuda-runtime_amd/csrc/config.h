// Model geometry from a checkpoint's config.json, and the RoPE frequency table.
//
// Same interface as the reference's src/config.h:15-83 (RopeScaling,
// ModelConfig with load / from_json_string / validate / summary, WeightSpec,
// required_weights, compute_rope_inv_freq), so the Model and the host tests are
// drop-in. Error messages keep the reference's wording because its tests match
// on substrings of them.
#pragma once

#include <cstdint>
#include <string>
#include <vector>

#include "common.h"

namespace lcr {

// Llama 3 frequency rescaling: slow rotary pairs are divided by `factor`, fast
// pairs are kept, and the band between is interpolated. Disabled = plain RoPE.
struct RopeScaling {
  bool enabled = false;
  float factor = 32.0f;
  float low_freq_factor = 1.0f;
  float high_freq_factor = 4.0f;
  int original_max_position_embeddings = 8192;
};

struct ModelConfig {
  int hidden_size = 0;
  int intermediate_size = 0;
  int num_layers = 0;
  int num_heads = 0;
  int num_kv_heads = 0;
  int head_dim = 0;
  int vocab_size = 0;
  int max_position_embeddings = 0;
  float rms_norm_eps = 1e-5f;
  float rope_theta = 500000.0f;
  bool tie_word_embeddings = true;
  RopeScaling rope_scaling;

  int bos_token_id = -1;
  std::vector<int> eos_token_ids;

  int heads_per_kv() const { return num_heads / num_kv_heads; }
  int kv_dim() const { return num_kv_heads * head_dim; }
  int q_dim() const { return num_heads * head_dim; }
  // Cache bytes one position occupies over every layer, keys and values.
  size_t kv_bytes_per_token(size_t elem_size) const {
    return static_cast<size_t>(num_layers) * 2 * static_cast<size_t>(kv_dim()) * elem_size;
  }

  bool is_eos(int token_id) const;

  // config.json, plus generation_config.json (stop tokens) when present.
  static ModelConfig load(const std::string& model_dir);
  static ModelConfig from_json_string(const std::string& text);

  void validate() const;
  std::string summary() const;
};

struct WeightSpec {
  std::string name;
  std::vector<int64_t> shape;
};

// Every tensor the forward pass reads, in reading order (the output head is
// not listed: it is lm_head.weight if present, else the tied embedding).
std::vector<WeightSpec> required_weights(const ModelConfig& config);

// Weight bytes one decoded token streams, the reference's accounting
// (src/model.cu:86-102): every tensor of required_weights() once, except that
// the step reads one row of the embedding table and all of the output head,
// which has the embedding's shape (tied or not). 2,471,628,800 for
// Llama-3.2-1B in bf16.
size_t weight_bytes_per_token(const ModelConfig& config, size_t elem_size);

// head_dim/2 inverse frequencies, computed in double and rounded to float once,
// with the llama3 bands applied when the config enables them.
std::vector<float> compute_rope_inv_freq(const ModelConfig& config);

}  // namespace lcr
