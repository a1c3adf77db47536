#include "config.h"

#include <algorithm>
#include <cmath>
#include <fstream>
#include <sstream>

#include "json.h"

namespace lcr {
namespace {

std::string path_join(const std::string& dir, const std::string& name) {
  if (dir.empty()) return name;
  return dir.back() == '/' ? dir + name : dir + "/" + name;
}

// eos_token_id is an integer in older checkpoints and a list in Llama 3.x.
void append_eos(const json::Value& node, std::vector<int>* out) {
  if (node.is_integer()) {
    out->push_back(node.as_int());
    return;
  }
  if (!node.is_array()) return;
  for (const json::Value& item : node.items()) {
    if (item.is_integer()) out->push_back(item.as_int());
  }
}

bool read_file(const std::string& path, std::string* text) {
  std::ifstream in(path, std::ios::binary);
  if (!in.good()) return false;
  std::ostringstream buffer;
  buffer << in.rdbuf();
  *text = buffer.str();
  return true;
}

}  // namespace

bool ModelConfig::is_eos(int token_id) const {
  return std::find(eos_token_ids.begin(), eos_token_ids.end(), token_id) !=
         eos_token_ids.end();
}

// Field semantics follow the reference's src/config.cpp:40-132.
ModelConfig ModelConfig::from_json_string(const std::string& text) {
  json::Value doc;
  std::string parse_error;
  LCR_CHECK(json::parse(text, &doc, &parse_error),
            "config.json is not valid JSON (" << parse_error << ")");
  LCR_CHECK(doc.is_object(), "config.json is not a JSON object");

  if (const json::Value* type = doc.find("model_type"); type && type->is_string()) {
    LCR_CHECK(type->as_string() == "llama",
              "this runtime only implements the Llama architecture, config.json "
              "says model_type=\"" << type->as_string() << "\"");
  }

  auto required = [&doc](const char* key) {
    const json::Value* v = doc.find(key);
    LCR_CHECK(v != nullptr && v->is_number(),
              "config.json is missing the integer field \"" << key << "\"");
    return v->as_int();
  };

  ModelConfig c;
  c.hidden_size = required("hidden_size");
  c.intermediate_size = required("intermediate_size");
  c.num_layers = required("num_hidden_layers");
  c.num_heads = required("num_attention_heads");
  c.vocab_size = required("vocab_size");
  c.max_position_embeddings = required("max_position_embeddings");

  const json::Value* kv = doc.find("num_key_value_heads");
  c.num_kv_heads = (kv != nullptr && kv->is_number()) ? kv->as_int() : c.num_heads;
  const json::Value* hd = doc.find("head_dim");
  c.head_dim = (hd != nullptr && hd->is_number())
                   ? hd->as_int()
                   : (c.num_heads > 0 ? c.hidden_size / c.num_heads : 0);

  if (const json::Value* v = doc.find("rms_norm_eps"); v && v->is_number()) {
    c.rms_norm_eps = v->as_float();
  }
  if (const json::Value* v = doc.find("rope_theta"); v && v->is_number()) {
    c.rope_theta = v->as_float();
  }
  if (const json::Value* v = doc.find("tie_word_embeddings"); v && v->is_bool()) {
    c.tie_word_embeddings = v->as_bool();
  }
  if (const json::Value* v = doc.find("attention_bias"); v && v->is_bool()) {
    LCR_CHECK(!v->as_bool(), "attention projections with bias are not implemented");
  }
  if (const json::Value* v = doc.find("mlp_bias"); v && v->is_bool()) {
    LCR_CHECK(!v->as_bool(), "MLP projections with bias are not implemented");
  }
  if (const json::Value* v = doc.find("hidden_act"); v && v->is_string()) {
    LCR_CHECK(v->as_string() == "silu",
              "only the SiLU/SwiGLU MLP is implemented, config.json says \""
                  << v->as_string() << "\"");
  }

  if (const json::Value* rs = doc.find("rope_scaling"); rs && rs->is_object()) {
    std::string type = "default";
    if (const json::Value* t = rs->find("rope_type"); t && t->is_string()) {
      type = t->as_string();
    } else if (const json::Value* t2 = rs->find("type"); t2 && t2->is_string()) {
      type = t2->as_string();
    }
    if (type != "default" && type != "none") {
      LCR_CHECK(type == "llama3", "only llama3 RoPE scaling is implemented, "
                                  "config.json says \"" << type << "\"");
      c.rope_scaling.enabled = true;
      if (const json::Value* f = rs->find("factor"); f && f->is_number()) {
        c.rope_scaling.factor = f->as_float();
      }
      if (const json::Value* f = rs->find("low_freq_factor"); f && f->is_number()) {
        c.rope_scaling.low_freq_factor = f->as_float();
      }
      if (const json::Value* f = rs->find("high_freq_factor"); f && f->is_number()) {
        c.rope_scaling.high_freq_factor = f->as_float();
      }
      if (const json::Value* f = rs->find("original_max_position_embeddings");
          f && f->is_number()) {
        c.rope_scaling.original_max_position_embeddings = f->as_int();
      }
    }
  }

  if (const json::Value* b = doc.find("bos_token_id"); b && b->is_integer()) {
    c.bos_token_id = b->as_int();
  }
  if (const json::Value* e = doc.find("eos_token_id")) append_eos(*e, &c.eos_token_ids);

  c.validate();
  return c;
}

ModelConfig ModelConfig::load(const std::string& model_dir) {
  const std::string config_path = path_join(model_dir, "config.json");
  std::string text;
  LCR_CHECK(read_file(config_path, &text), "cannot read " << config_path);
  ModelConfig c = from_json_string(text);

  // generation_config.json, when present, is the authority on stop tokens.
  std::string gen_text;
  if (read_file(path_join(model_dir, "generation_config.json"), &gen_text)) {
    json::Value gen;
    if (json::parse(gen_text, &gen, nullptr) && gen.is_object()) {
      std::vector<int> eos;
      if (const json::Value* e = gen.find("eos_token_id")) append_eos(*e, &eos);
      if (!eos.empty()) c.eos_token_ids = eos;
      if (const json::Value* b = gen.find("bos_token_id"); b && b->is_integer()) {
        c.bos_token_id = b->as_int();
      }
    }
  }
  return c;
}

void ModelConfig::validate() const {
  LCR_CHECK(hidden_size > 0 && intermediate_size > 0 && num_layers > 0,
            "config.json has a non-positive hidden_size, intermediate_size, or "
            "num_hidden_layers");
  LCR_CHECK(num_heads > 0 && num_kv_heads > 0,
            "config.json has a non-positive head count");
  LCR_CHECK(num_heads % num_kv_heads == 0,
            "num_attention_heads (" << num_heads << ") must be a multiple of "
            "num_key_value_heads (" << num_kv_heads << ")");
  LCR_CHECK(head_dim > 0 && head_dim % 2 == 0,
            "head_dim must be positive and even for RoPE, got " << head_dim);
  LCR_CHECK(vocab_size > 0, "vocab_size must be positive");
  LCR_CHECK(rms_norm_eps > 0.0f, "rms_norm_eps must be positive");
  LCR_CHECK(rope_theta > 1.0f, "rope_theta must be greater than one");
  if (rope_scaling.enabled) {
    LCR_CHECK(rope_scaling.factor > 0.0f, "RoPE scaling factor must be positive");
    LCR_CHECK(rope_scaling.high_freq_factor > rope_scaling.low_freq_factor,
              "RoPE high_freq_factor must exceed low_freq_factor");
    LCR_CHECK(rope_scaling.original_max_position_embeddings > 0,
              "RoPE original_max_position_embeddings must be positive");
  }
}

std::string ModelConfig::summary() const {
  std::ostringstream oss;
  oss << "layers=" << num_layers << " hidden=" << hidden_size
      << " ffn=" << intermediate_size << " heads=" << num_heads << "/" << num_kv_heads
      << " head_dim=" << head_dim << " vocab=" << vocab_size
      << " rope_theta=" << rope_theta
      << (rope_scaling.enabled ? " rope_scaling=llama3" : "")
      << (tie_word_embeddings ? " tied_embeddings" : "");
  return oss.str();
}

// Tensor names and order: the reference's src/config.cpp:197-221.
std::vector<WeightSpec> required_weights(const ModelConfig& c) {
  const int64_t hidden = c.hidden_size;
  const int64_t ffn = c.intermediate_size;
  const int64_t q = c.q_dim();
  const int64_t kv = c.kv_dim();
  std::vector<WeightSpec> out;
  out.push_back({"model.embed_tokens.weight", {c.vocab_size, hidden}});
  for (int layer = 0; layer < c.num_layers; ++layer) {
    const std::string p = "model.layers." + std::to_string(layer) + ".";
    out.push_back({p + "input_layernorm.weight", {hidden}});
    out.push_back({p + "self_attn.q_proj.weight", {q, hidden}});
    out.push_back({p + "self_attn.k_proj.weight", {kv, hidden}});
    out.push_back({p + "self_attn.v_proj.weight", {kv, hidden}});
    out.push_back({p + "self_attn.o_proj.weight", {hidden, q}});
    out.push_back({p + "post_attention_layernorm.weight", {hidden}});
    out.push_back({p + "mlp.gate_proj.weight", {ffn, hidden}});
    out.push_back({p + "mlp.up_proj.weight", {ffn, hidden}});
    out.push_back({p + "mlp.down_proj.weight", {hidden, ffn}});
  }
  out.push_back({"model.norm.weight", {hidden}});
  return out;
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

// The llama3 band rule of the reference's src/config.cpp:223-259: a pair whose
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
