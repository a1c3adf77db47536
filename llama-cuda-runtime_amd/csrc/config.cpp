// config.json is read against a schema: a table row per key this runtime
// understands, naming the ModelConfig member it fills, whether the key must be
// there, and which values are refused. The reader walks the tables once;
// derived defaults (kv heads, head_dim) and the cross-field rules of
// validate() run after. The keys, their meanings and the refusal messages
// follow the reference (src/config.cpp:36-221; its tests match the message
// substrings), the structure is this file's own.
#include "config.h"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <functional>
#include <iterator>
#include <sstream>

#include "json.h"

namespace lcr {
namespace {

using json::Value;

// ---------------------------------------------------------------------------
// Schema tables
// ---------------------------------------------------------------------------

// An integer key. Required keys must be numbers; optional ones are taken when
// they are numbers and otherwise leave the member at its sentinel (0) for the
// derived-default pass.
struct IntKey {
  const char* key;
  int ModelConfig::*member;
  bool required;
};

constexpr IntKey kIntKeys[] = {
    {"hidden_size", &ModelConfig::hidden_size, true},
    {"intermediate_size", &ModelConfig::intermediate_size, true},
    {"num_hidden_layers", &ModelConfig::num_layers, true},
    {"num_attention_heads", &ModelConfig::num_heads, true},
    {"vocab_size", &ModelConfig::vocab_size, true},
    {"max_position_embeddings", &ModelConfig::max_position_embeddings, true},
    {"num_key_value_heads", &ModelConfig::num_kv_heads, false},  // absent: multi-head attention
    {"head_dim", &ModelConfig::head_dim, false},                  // absent: hidden / heads
};

// Optional real and boolean keys over the member's default.
struct RealKey {
  const char* key;
  float ModelConfig::*member;
};
constexpr RealKey kRealKeys[] = {
    {"rms_norm_eps", &ModelConfig::rms_norm_eps},
    {"rope_theta", &ModelConfig::rope_theta},
};

struct FlagKey {
  const char* key;
  bool ModelConfig::*member;
};
constexpr FlagKey kFlagKeys[] = {
    {"tie_word_embeddings", &ModelConfig::tie_word_embeddings},
};

// String keys whose only accepted value is `accepted` (when present). The
// message is completed with the value found and a closing quote.
struct OnlyValue {
  const char* key;
  const char* accepted;
  const char* refusal;
};
constexpr OnlyValue kOnlyValues[] = {
    {"model_type", "llama",
     "this runtime only implements the Llama architecture, config.json says model_type=\""},
    {"hidden_act", "silu", "only the SiLU/SwiGLU MLP is implemented, config.json says \""},
};

// Boolean features this runtime does not implement: refused when true.
struct Unsupported {
  const char* key;
  const char* refusal;
};
constexpr Unsupported kUnsupported[] = {
    {"attention_bias", "attention projections with bias are not implemented"},
    {"mlp_bias", "MLP projections with bias are not implemented"},
};

// The llama3 rope_scaling block's numbers, over RopeScaling's defaults.
struct RopeRealKey {
  const char* key;
  float RopeScaling::*member;
};
constexpr RopeRealKey kRopeRealKeys[] = {
    {"factor", &RopeScaling::factor},
    {"low_freq_factor", &RopeScaling::low_freq_factor},
    {"high_freq_factor", &RopeScaling::high_freq_factor},
};

// ---------------------------------------------------------------------------
// Readers
// ---------------------------------------------------------------------------

const Value* number_at(const Value& obj, const char* key) {
  const Value* v = obj.find(key);
  return (v != nullptr && v->is_number()) ? v : nullptr;
}

// Token ids: one integer (older checkpoints) or a list of them (Llama 3.x
// stops on several). Anything else contributes nothing.
std::vector<int> token_list(const Value* node) {
  std::vector<int> ids;
  if (node == nullptr) return ids;
  if (node->is_integer()) {
    ids.push_back(node->as_int());
  } else if (node->is_array()) {
    for (const Value& item : node->items()) {
      if (item.is_integer()) ids.push_back(item.as_int());
    }
  }
  return ids;
}

// The scaling scheme a rope_scaling block names ("rope_type" in current
// checkpoints, "type" in older ones); "default" when it names none.
std::string rope_scheme(const Value& block) {
  for (const char* key : {"rope_type", "type"}) {
    const Value* v = block.find(key);
    if (v != nullptr && v->is_string()) return v->as_string();
  }
  return "default";
}

void read_rope_scaling(const Value& block, RopeScaling* out) {
  const std::string scheme = rope_scheme(block);
  if (scheme == "default" || scheme == "none") return;
  LCR_CHECK(scheme == "llama3",
            "only llama3 RoPE scaling is implemented, config.json says \"" << scheme << "\"");
  out->enabled = true;
  for (const RopeRealKey& k : kRopeRealKeys) {
    if (const Value* v = number_at(block, k.key)) out->*k.member = v->as_float();
  }
  if (const Value* v = number_at(block, "original_max_position_embeddings")) {
    out->original_max_position_embeddings = v->as_int();
  }
}

std::string file_in(const std::string& dir, const char* name) {
  if (dir.empty()) return name;
  return dir + (dir.back() == '/' ? "" : "/") + name;
}

// The whole file, or false when it cannot be opened.
bool slurp(const std::string& path, std::string* text) {
  std::ifstream in(path, std::ios::binary);
  if (!in) return false;
  text->assign(std::istreambuf_iterator<char>(in), std::istreambuf_iterator<char>());
  return true;
}

// ---------------------------------------------------------------------------
// Cross-field rules, checked in order; the first that fails is reported.
// ---------------------------------------------------------------------------

struct Rule {
  std::function<bool(const ModelConfig&)> holds;
  std::function<std::string(const ModelConfig&)> message;
};

std::string text(const char* s) { return s; }

const std::vector<Rule>& rules() {
  static const std::vector<Rule> table = {
      {[](const ModelConfig& c) { return c.hidden_size > 0 && c.intermediate_size > 0 && c.num_layers > 0; },
       [](const ModelConfig&) { return text("config.json needs positive hidden_size, intermediate_size and "
                                            "num_hidden_layers"); }},
      {[](const ModelConfig& c) { return c.num_heads > 0 && c.num_kv_heads > 0; },
       [](const ModelConfig& c) {
         std::ostringstream m;
         m << "config.json needs positive head counts, got " << c.num_heads << " query and " << c.num_kv_heads
           << " key/value heads";
         return m.str();
       }},
      {[](const ModelConfig& c) { return c.num_heads % c.num_kv_heads == 0; },
       [](const ModelConfig& c) {
         std::ostringstream m;
         m << "num_attention_heads (" << c.num_heads << ") must be a multiple of num_key_value_heads ("
           << c.num_kv_heads << ")";
         return m.str();
       }},
      {[](const ModelConfig& c) { return c.head_dim > 0 && c.head_dim % 2 == 0; },
       [](const ModelConfig& c) {
         return "RoPE rotates pairs, so head_dim must be positive and even; got " + std::to_string(c.head_dim);
       }},
      {[](const ModelConfig& c) { return c.vocab_size > 0; },
       [](const ModelConfig&) { return text("vocab_size must be positive"); }},
      {[](const ModelConfig& c) { return c.rms_norm_eps > 0.0f; },
       [](const ModelConfig&) { return text("rms_norm_eps must be positive"); }},
      {[](const ModelConfig& c) { return c.rope_theta > 1.0f; },
       [](const ModelConfig&) { return text("rope_theta must be greater than 1"); }},
      {[](const ModelConfig& c) { return !c.rope_scaling.enabled || c.rope_scaling.factor > 0.0f; },
       [](const ModelConfig&) { return text("the llama3 RoPE factor must be positive"); }},
      {[](const ModelConfig& c) {
         return !c.rope_scaling.enabled || c.rope_scaling.high_freq_factor > c.rope_scaling.low_freq_factor;
       },
       [](const ModelConfig&) { return text("llama3 RoPE needs high_freq_factor > low_freq_factor"); }},
      {[](const ModelConfig& c) {
         return !c.rope_scaling.enabled || c.rope_scaling.original_max_position_embeddings > 0;
       },
       [](const ModelConfig&) { return text("llama3 RoPE needs a positive original_max_position_embeddings"); }},
  };
  return table;
}

}  // namespace

bool ModelConfig::is_eos(int token_id) const {
  return std::count(eos_token_ids.begin(), eos_token_ids.end(), token_id) > 0;
}

ModelConfig ModelConfig::from_json_string(const std::string& document) {
  Value doc;
  std::string why;
  LCR_CHECK(json::parse(document, &doc, &why), "config.json is not valid JSON (" << why << ")");
  LCR_CHECK(doc.is_object(), "config.json is not a JSON object");

  for (const OnlyValue& k : kOnlyValues) {
    const Value* v = doc.find(k.key);
    if (v != nullptr && v->is_string()) {
      LCR_CHECK(v->as_string() == k.accepted, k.refusal << v->as_string() << "\"");
    }
  }
  for (const Unsupported& k : kUnsupported) {
    const Value* v = doc.find(k.key);
    LCR_CHECK(v == nullptr || !v->is_bool() || !v->as_bool(), k.refusal);
  }

  ModelConfig c;
  for (const IntKey& k : kIntKeys) {
    const Value* v = number_at(doc, k.key);
    LCR_CHECK(v != nullptr || !k.required, "config.json is missing the integer field \"" << k.key << "\"");
    if (v != nullptr) c.*k.member = v->as_int();
  }
  for (const RealKey& k : kRealKeys) {
    if (const Value* v = number_at(doc, k.key)) c.*k.member = v->as_float();
  }
  for (const FlagKey& k : kFlagKeys) {
    const Value* v = doc.find(k.key);
    if (v != nullptr && v->is_bool()) c.*k.member = v->as_bool();
  }
  // Derived defaults for the optional geometry keys.
  if (c.num_kv_heads == 0) c.num_kv_heads = c.num_heads;
  if (c.head_dim == 0 && c.num_heads > 0) c.head_dim = c.hidden_size / c.num_heads;

  if (const Value* block = doc.find("rope_scaling"); block != nullptr && block->is_object()) {
    read_rope_scaling(*block, &c.rope_scaling);
  }
  if (const Value* v = doc.find("bos_token_id"); v != nullptr && v->is_integer()) c.bos_token_id = v->as_int();
  c.eos_token_ids = token_list(doc.find("eos_token_id"));

  c.validate();
  return c;
}

ModelConfig ModelConfig::load(const std::string& model_dir) {
  const std::string path = file_in(model_dir, "config.json");
  std::string document;
  LCR_CHECK(slurp(path, &document), "cannot read " << path);
  ModelConfig c = from_json_string(document);

  // Stop and start tokens: generation_config.json overrides config.json when
  // it has them (the copy in config.json is often stale). A generation config
  // that does not parse is ignored, as it is optional.
  std::string gen_document;
  Value gen;
  if (slurp(file_in(model_dir, "generation_config.json"), &gen_document) &&
      json::parse(gen_document, &gen, nullptr) && gen.is_object()) {
    const std::vector<int> eos = token_list(gen.find("eos_token_id"));
    if (!eos.empty()) c.eos_token_ids = eos;
    if (const Value* v = gen.find("bos_token_id"); v != nullptr && v->is_integer()) c.bos_token_id = v->as_int();
  }
  return c;
}

void ModelConfig::validate() const {
  for (const Rule& r : rules()) {
    if (!r.holds(*this)) throw Error(r.message(*this));
  }
}

std::string ModelConfig::summary() const {
  std::ostringstream s;
  s << num_layers << " layers, hidden " << hidden_size << ", ffn " << intermediate_size << ", " << num_heads
    << " q heads / " << num_kv_heads << " kv heads x " << head_dim << ", vocab " << vocab_size << ", rope theta "
    << rope_theta;
  if (rope_scaling.enabled) s << " (llama3 x" << rope_scaling.factor << ")";
  s << (tie_word_embeddings ? ", tied head" : ", separate head");
  return s.str();
}

// The checkpoint's tensor names and shapes (the format, the reference's
// src/config.cpp:197-221): the embedding, then per layer the nine tensors of
// kLayerTensors in reading order, then the final norm.
namespace {

// A per-layer tensor: its name after "model.layers.<i>.", and its [rows, cols]
// (cols 0: a vector of `rows`) as functions of the geometry.
struct LayerTensor {
  const char* suffix;
  int64_t (*rows)(const ModelConfig&);
  int64_t (*cols)(const ModelConfig&);
};

int64_t hidden_of(const ModelConfig& c) { return c.hidden_size; }
int64_t ffn_of(const ModelConfig& c) { return c.intermediate_size; }
int64_t q_of(const ModelConfig& c) { return c.q_dim(); }
int64_t kv_of(const ModelConfig& c) { return c.kv_dim(); }
int64_t vector_of(const ModelConfig&) { return 0; }

constexpr LayerTensor kLayerTensors[] = {
    {"input_layernorm.weight", hidden_of, vector_of},
    {"self_attn.q_proj.weight", q_of, hidden_of},
    {"self_attn.k_proj.weight", kv_of, hidden_of},
    {"self_attn.v_proj.weight", kv_of, hidden_of},
    {"self_attn.o_proj.weight", hidden_of, q_of},
    {"post_attention_layernorm.weight", hidden_of, vector_of},
    {"mlp.gate_proj.weight", ffn_of, hidden_of},
    {"mlp.up_proj.weight", ffn_of, hidden_of},
    {"mlp.down_proj.weight", hidden_of, ffn_of},
};

}  // namespace

std::vector<WeightSpec> required_weights(const ModelConfig& c) {
  std::vector<WeightSpec> specs;
  specs.reserve(2 + std::size(kLayerTensors) * static_cast<size_t>(std::max(0, c.num_layers)));
  specs.push_back({"model.embed_tokens.weight", {c.vocab_size, c.hidden_size}});
  for (int layer = 0; layer < c.num_layers; ++layer) {
    const std::string prefix = "model.layers." + std::to_string(layer) + ".";
    for (const LayerTensor& t : kLayerTensors) {
      WeightSpec spec{prefix + t.suffix, {t.rows(c)}};
      if (const int64_t cols = t.cols(c); cols > 0) spec.shape.push_back(cols);
      specs.push_back(std::move(spec));
    }
  }
  specs.push_back({"model.norm.weight", {c.hidden_size}});
  return specs;
}

size_t weight_bytes_per_token(const ModelConfig& config, size_t elem_size) {
  size_t elements = 0;
  for (const WeightSpec& w : required_weights(config)) {
    size_t n = 1;
    for (int64_t d : w.shape) n *= static_cast<size_t>(d);
    elements += n;  // the embedding's count stands for the output head's
  }
  return elements * elem_size;
}

// The llama3 band rule (the reference's src/config.cpp:223-259): a pair whose
// wavelength is shorter than original_context/high_freq_factor keeps its
// frequency, one longer than original_context/low_freq_factor is divided by
// the factor, and one in between is a linear blend of the two weighted by
// (original_context/wavelength - low) / (high - low). Everything is in double,
// rounded to float once at the end.
std::vector<float> compute_rope_inv_freq(const ModelConfig& c) {
  const int pairs = c.head_dim / 2;
  std::vector<double> base(static_cast<size_t>(pairs));
  std::vector<float> out(static_cast<size_t>(pairs));
  for (int i = 0; i < pairs; ++i) {
    const double exponent = static_cast<double>(2 * i) / static_cast<double>(c.head_dim);
    // The unscaled table is rounded to float first, as a stored table would be.
    const float f = static_cast<float>(1.0 / std::pow(static_cast<double>(c.rope_theta), exponent));
    out[static_cast<size_t>(i)] = f;
    base[static_cast<size_t>(i)] = f;
  }
  if (!c.rope_scaling.enabled) return out;

  const RopeScaling& rs = c.rope_scaling;
  const double context = rs.original_max_position_embeddings;
  const double short_limit = context / rs.high_freq_factor;
  const double long_limit = context / rs.low_freq_factor;
  const double tau = 2.0 * M_PI;
  for (int i = 0; i < pairs; ++i) {
    const double freq = base[static_cast<size_t>(i)];
    const double wavelength = tau / freq;
    double scaled = freq;
    if (wavelength > long_limit) {
      scaled = freq / rs.factor;
    } else if (wavelength >= short_limit) {
      const double t = (context / wavelength - rs.low_freq_factor) /
                       (rs.high_freq_factor - rs.low_freq_factor);
      scaled = (1.0 - t) * (freq / rs.factor) + t * freq;
    }
    out[static_cast<size_t>(i)] = static_cast<float>(scaled);
  }
  return out;
}

}  // namespace lcr
