// Host-side C++ tests of the drop-in classes (no GPU needed): ModelConfig and
// the RoPE table (the reference's tests/test_config.cpp cases), the
// safetensors reader and writer (tests/test_safetensors.cpp cases), and the
// JSON parser that replaces nlohmann/json. Built by tests/cpp/Makefile against
// liblcr_amd.so and run by tests/test_host.py.
#include <stdlib.h>
#include <unistd.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

#include "common.h"
#include "config.h"
#include "json.h"
#include "kv_cache.h"
#include "safetensors.h"

namespace {

int g_failures = 0;

void report(bool ok, const char* file, int line, const std::string& what) {
  if (ok) return;
  std::fprintf(stderr, "FAIL %s:%d: %s\n", file, line, what.c_str());
  ++g_failures;
}

#define EXPECT(cond) report((cond), __FILE__, __LINE__, "expected " #cond)
#define EXPECT_EQ(a, b)                                                   \
  do {                                                                    \
    auto lhs_ = (a);                                                      \
    auto rhs_ = (b);                                                      \
    if (!(lhs_ == rhs_)) {                                                \
      std::ostringstream oss_;                                            \
      oss_ << #a " == " #b " (" << lhs_ << " vs " << rhs_ << ")";         \
      report(false, __FILE__, __LINE__, oss_.str());                      \
    }                                                                     \
  } while (0)
#define EXPECT_NEAR(a, b, tol)                                             \
  report(std::fabs(static_cast<double>(a) - static_cast<double>(b)) <= (tol), __FILE__, __LINE__, \
         #a " near " #b)

void expect_throws(const char* file, int line, const std::string& needle,
                   const std::function<void()>& body) {
  try {
    body();
  } catch (const std::exception& e) {
    const std::string what = e.what();
    if (what.find(needle) == std::string::npos) {
      report(false, file, line, "threw without \"" + needle + "\": " + what);
    }
    return;
  }
  report(false, file, line, "did not throw (expected \"" + needle + "\")");
}
#define EXPECT_THROWS(needle, body) expect_throws(__FILE__, __LINE__, needle, [&]() body)

using lcr::ModelConfig;

const char* kLlama32_1B = R"({
  "architectures": ["LlamaForCausalLM"], "attention_bias": false, "bos_token_id": 128000,
  "eos_token_id": [128001, 128008, 128009], "head_dim": 64, "hidden_act": "silu",
  "hidden_size": 2048, "intermediate_size": 8192, "max_position_embeddings": 131072,
  "mlp_bias": false, "model_type": "llama", "num_attention_heads": 32, "num_hidden_layers": 16,
  "num_key_value_heads": 8, "rms_norm_eps": 1e-05,
  "rope_scaling": {"factor": 32.0, "high_freq_factor": 4.0, "low_freq_factor": 1.0,
                   "original_max_position_embeddings": 8192, "rope_type": "llama3"},
  "rope_theta": 500000.0, "tie_word_embeddings": true, "torch_dtype": "bfloat16",
  "vocab_size": 128256
})";

void test_config_parse() {
  const ModelConfig c = ModelConfig::from_json_string(kLlama32_1B);
  EXPECT_EQ(c.hidden_size, 2048);
  EXPECT_EQ(c.intermediate_size, 8192);
  EXPECT_EQ(c.num_layers, 16);
  EXPECT_EQ(c.num_heads, 32);
  EXPECT_EQ(c.num_kv_heads, 8);
  EXPECT_EQ(c.head_dim, 64);
  EXPECT_EQ(c.vocab_size, 128256);
  EXPECT_EQ(c.bos_token_id, 128000);
  EXPECT_EQ(c.eos_token_ids.size(), static_cast<size_t>(3));
  EXPECT(c.is_eos(128009));
  EXPECT(!c.is_eos(42));
  EXPECT(c.tie_word_embeddings);
  EXPECT_NEAR(c.rope_theta, 500000.0, 1e-3);
  EXPECT_NEAR(c.rms_norm_eps, 1e-5, 1e-12);
  EXPECT_EQ(c.heads_per_kv(), 4);
  EXPECT_EQ(c.kv_dim(), 512);
  EXPECT_EQ(c.q_dim(), 2048);
  EXPECT_EQ(c.kv_bytes_per_token(2), static_cast<size_t>(16 * 2 * 512 * 2));
  EXPECT(c.rope_scaling.enabled);
  EXPECT_NEAR(c.rope_scaling.factor, 32.0, 1e-6);
  EXPECT_EQ(c.rope_scaling.original_max_position_embeddings, 8192);
  // reading order of the weights
  const auto specs = lcr::required_weights(c);
  EXPECT_EQ(specs.size(), static_cast<size_t>(1 + 16 * 9 + 1));
  EXPECT_EQ(specs[0].name, std::string("model.embed_tokens.weight"));
  EXPECT_EQ(specs[2].name, std::string("model.layers.0.self_attn.q_proj.weight"));
  EXPECT_EQ(specs.back().name, std::string("model.norm.weight"));
}

void test_config_optional_fields() {
  const ModelConfig c = ModelConfig::from_json_string(R"({
    "hidden_size": 2048, "intermediate_size": 5632, "num_hidden_layers": 22,
    "num_attention_heads": 32, "vocab_size": 32000, "max_position_embeddings": 2048,
    "rope_theta": 10000.0})");
  EXPECT_EQ(c.head_dim, 64);
  EXPECT_EQ(c.num_kv_heads, 32);
  EXPECT_EQ(c.heads_per_kv(), 1);
  EXPECT(!c.rope_scaling.enabled);
}

void test_config_rejections() {
  EXPECT_THROWS("only implements the Llama architecture", {
    ModelConfig::from_json_string(R"({"model_type":"mistral","hidden_size":8,"intermediate_size":8,
      "num_hidden_layers":1,"num_attention_heads":2,"vocab_size":8,"max_position_embeddings":8})");
  });
  EXPECT_THROWS("must be a multiple of", {
    ModelConfig::from_json_string(R"({"hidden_size":64,"intermediate_size":64,"num_hidden_layers":1,
      "num_attention_heads":6,"num_key_value_heads":4,"vocab_size":8,"max_position_embeddings":8})");
  });
  EXPECT_THROWS("only llama3 RoPE scaling", {
    ModelConfig::from_json_string(R"({"hidden_size":64,"intermediate_size":64,"num_hidden_layers":1,
      "num_attention_heads":2,"vocab_size":8,"max_position_embeddings":8,
      "rope_scaling":{"rope_type":"yarn","factor":2.0}})");
  });
  EXPECT_THROWS("missing the integer field \"vocab_size\"", {
    ModelConfig::from_json_string(R"({"hidden_size":64,"intermediate_size":64,"num_hidden_layers":1,
      "num_attention_heads":2,"max_position_embeddings":8})");
  });
  EXPECT_THROWS("only the SiLU/SwiGLU MLP", {
    ModelConfig::from_json_string(R"({"hidden_size":64,"intermediate_size":64,"num_hidden_layers":1,
      "num_attention_heads":2,"vocab_size":8,"max_position_embeddings":8,"hidden_act":"gelu"})");
  });
  EXPECT_THROWS("not valid JSON", { ModelConfig::from_json_string("{\"hidden_size\": 3,"); });
}

void test_rope_frequencies() {
  const ModelConfig plain = ModelConfig::from_json_string(R"({
    "hidden_size": 2048, "intermediate_size": 5632, "num_hidden_layers": 22,
    "num_attention_heads": 32, "vocab_size": 32000, "max_position_embeddings": 2048,
    "rope_theta": 10000.0})");
  const std::vector<float> f = lcr::compute_rope_inv_freq(plain);
  EXPECT_EQ(f.size(), static_cast<size_t>(32));
  for (int i = 0; i < 32; ++i) {
    const double want = std::pow(10000.0, -2.0 * i / 64.0);
    EXPECT_NEAR(f[i], want, want * 1e-6);
  }
  const ModelConfig c = ModelConfig::from_json_string(kLlama32_1B);
  const std::vector<float> g = lcr::compute_rope_inv_freq(c);
  int untouched = 0, stretched = 0, blended = 0;
  for (int i = 0; i < 32; ++i) {
    const double base = std::pow(500000.0, -2.0 * i / 64.0);
    const double wl = 2.0 * M_PI / base;
    double want;
    if (wl < 2048.0) {
      want = base;
      ++untouched;
    } else if (wl > 8192.0) {
      want = base / 32.0;
      ++stretched;
    } else {
      const double s = (8192.0 / wl - 1.0) / 3.0;
      want = (1.0 - s) * (base / 32.0) + s * base;
      ++blended;
    }
    EXPECT_NEAR(g[i], want, std::fabs(want) * 1e-5);
  }
  EXPECT(untouched > 0 && stretched > 0 && blended > 0);
  EXPECT_NEAR(g[0], 1.0, 1e-9);
  for (size_t i = 1; i < g.size(); ++i) EXPECT(g[i] < g[i - 1]);
}

std::string temp_dir() {
  char pattern[] = "/tmp/lcr_host_test_XXXXXX";
  const char* dir = ::mkdtemp(pattern);
  EXPECT(dir != nullptr);
  return dir ? std::string(dir) : std::string("/tmp");
}

void write_raw(const std::string& path, const std::string& header, const std::vector<uint8_t>& payload,
               uint64_t declared = 0) {
  std::ofstream out(path, std::ios::binary);
  const uint64_t len = declared ? declared : header.size();
  for (int i = 0; i < 8; ++i) out.put(static_cast<char>((len >> (8 * i)) & 0xff));
  out.write(header.data(), static_cast<std::streamsize>(header.size()));
  out.write(reinterpret_cast<const char*>(payload.data()), static_cast<std::streamsize>(payload.size()));
}

std::vector<uint8_t> float_bytes(const std::vector<float>& v) {
  std::vector<uint8_t> out(v.size() * 4);
  std::memcpy(out.data(), v.data(), out.size());
  return out;
}

void test_safetensors_well_formed() {
  const std::string dir = temp_dir();
  std::vector<uint8_t> payload = float_bytes({1, 2, 3, 4, 5, 6});
  for (uint8_t b : {1, 2, 3, 4, 5, 6, 7, 8}) payload.push_back(b);
  write_raw(dir + "/model.safetensors",
            R"({"__metadata__":{"format":"pt"},)"
            R"("model.embed_tokens.weight":{"dtype":"F32","shape":[2,3],"data_offsets":[0,24]},)"
            R"("model.norm.weight":{"dtype":"BF16","shape":[4],"data_offsets":[24,32]}})",
            payload);
  lcr::SafetensorsArchive a(dir);
  EXPECT_EQ(a.tensor_count(), static_cast<size_t>(2));
  EXPECT_EQ(a.total_bytes(), static_cast<size_t>(32));
  const lcr::TensorView& e = a.get("model.embed_tokens.weight");
  EXPECT(e.dtype == lcr::DType::kF32);
  EXPECT_EQ(e.dim(1), static_cast<int64_t>(3));
  EXPECT_EQ(e.shape_string(), std::string("[2, 3]"));
  EXPECT_EQ(static_cast<const float*>(e.data)[5], 6.0f);
  EXPECT_EQ(static_cast<const uint8_t*>(a.get("model.norm.weight").data)[0], 1);
  EXPECT(!a.has("__metadata__"));
  const auto names = a.names();
  EXPECT_EQ(names[0], std::string("model.embed_tokens.weight"));
  e.expect_shape({2, 3});
  EXPECT_THROWS("expected [3, 2]", { e.expect_shape({3, 2}); });
  EXPECT_THROWS("no tensor named", { a.get("missing.weight"); });
}

void test_safetensors_sharded() {
  const std::string dir = temp_dir();
  write_raw(dir + "/model-00001-of-00002.safetensors", R"({"a":{"dtype":"F32","shape":[2],"data_offsets":[0,8]}})",
            float_bytes({1, 2}));
  write_raw(dir + "/model-00002-of-00002.safetensors", R"({"b":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}})",
            float_bytes({3}));
  std::ofstream(dir + "/model.safetensors.index.json")
      << R"({"metadata":{"total_size":12},"weight_map":{"a":"model-00001-of-00002.safetensors",)"
      << R"("b":"model-00002-of-00002.safetensors"}})";
  lcr::SafetensorsArchive a(dir);
  EXPECT_EQ(a.tensor_count(), static_cast<size_t>(2));
  EXPECT_EQ(static_cast<const float*>(a.get("a").data)[1], 2.0f);
  EXPECT_EQ(static_cast<const float*>(a.get("b").data)[0], 3.0f);
}

void test_safetensors_rejections() {
  auto one = [](const std::string& header, size_t payload, uint64_t declared = 0) {
    const std::string dir = temp_dir();
    write_raw(dir + "/model.safetensors", header, std::vector<uint8_t>(payload, 0), declared);
    return dir;
  };
  {
    const auto d = one(R"({"a":{"dtype":"F32","shape":[4],"data_offsets":[0,8]}})", 8);
    EXPECT_THROWS("needs 16", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = one(R"({"a":{"dtype":"F32","shape":[8],"data_offsets":[0,32]}})", 8);
    EXPECT_THROWS("data buffer", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = one(R"({"a":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}})", 4, 4096);
    EXPECT_THROWS("exceeds the file size", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = one("not json at all{{{", 4);
    EXPECT_THROWS("malformed JSON header", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = one(R"({"a":{"dtype":"FP8_E4M3","shape":[4],"data_offsets":[0,4]}})", 4);
    EXPECT_THROWS("unknown safetensors dtype", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = one(R"({"a":{"dtype":"F32","shape":[1]}})", 4);
    EXPECT_THROWS("missing dtype, shape, or data_offsets", { lcr::SafetensorsArchive a(d); });
  }
  {
    const auto d = temp_dir();
    EXPECT_THROWS("no model.safetensors", { lcr::SafetensorsArchive a(d); });
  }
}

void test_safetensors_writer_round_trip() {
  const std::string dir = temp_dir();
  std::vector<lcr::TensorSpec> specs = {{"x", lcr::DType::kBF16, {3, 5}}, {"y", lcr::DType::kF32, {7}}};
  lcr::write_safetensors(dir + "/model.safetensors", specs, [](size_t i, void* dst, size_t n) {
    for (size_t b = 0; b < n; ++b) static_cast<uint8_t*>(dst)[b] = static_cast<uint8_t>(i * 31 + b);
  });
  lcr::SafetensorsArchive a(dir);
  EXPECT_EQ(a.get("x").nbytes, static_cast<size_t>(30));
  EXPECT_EQ(a.get("y").nbytes, static_cast<size_t>(28));
  EXPECT_EQ(static_cast<const uint8_t*>(a.get("y").data)[3], static_cast<uint8_t>(31 + 3));
  EXPECT_EQ(reinterpret_cast<uintptr_t>(a.get("x").data) % 8, static_cast<uintptr_t>(0));
}

void test_json() {
  lcr::json::Value v;
  std::string err;
  EXPECT(lcr::json::parse(R"({"a":[1,2.5,-3e2,true,false,null],"s":"q\"\\\/\b\f\n\r\t\u00e9\ud83d\ude00"})", &v, &err));
  EXPECT(v.at("a").items()[0].is_integer());
  EXPECT_NEAR(v.at("a").items()[1].as_double(), 2.5, 0);
  EXPECT_NEAR(v.at("a").items()[2].as_double(), -300.0, 0);
  EXPECT(v.at("a").items()[5].is_null());
  EXPECT_EQ(v.at("s").as_string(), std::string("q\"\\/\b\f\n\r\t\xc3\xa9\xf0\x9f\x98\x80"));
  for (const char* bad : {"", "{", "[1,]", "{\"a\" 1}", "01", "\"\\ud800\"", "[1] x", "tru", "\"a\x01\""}) {
    lcr::json::Value w;
    EXPECT(!lcr::json::parse(bad, &w, &err));
  }
  lcr::json::Value o = lcr::json::Value::object();
  o.set("k", lcr::json::Value::integer(3));
  o.set("s", lcr::json::Value::string("a\"b"));
  EXPECT_EQ(o.dump(), std::string(R"({"k":3,"s":"a\"b"})"));
}

// Element-type table, size formatting and the check macro (common.h).
void test_common() {
  using lcr::DType;
  for (DType t : {DType::kF32, DType::kF16, DType::kBF16, DType::kI64, DType::kI32, DType::kI8, DType::kU8,
                  DType::kBool}) {
    EXPECT(lcr::dtype_from_string(lcr::dtype_name(t)) == t);
  }
  EXPECT_EQ(lcr::dtype_size(DType::kBF16), static_cast<size_t>(2));
  EXPECT_EQ(lcr::dtype_size(DType::kI64), static_cast<size_t>(8));
  EXPECT_EQ(lcr::dtype_size(DType::kBool), static_cast<size_t>(1));
  EXPECT_EQ(std::string(lcr::dtype_name(DType::kBF16)), std::string("BF16"));
  EXPECT_THROWS("F64 tensors are not supported", { lcr::dtype_from_string("F64"); });
  EXPECT_THROWS("unknown safetensors dtype \"F8_E4M3\"", { lcr::dtype_from_string("F8_E4M3"); });
  EXPECT_EQ(lcr::format_bytes(0), std::string("0 B"));
  EXPECT_EQ(lcr::format_bytes(1023), std::string("1023 B"));
  EXPECT_EQ(lcr::format_bytes(1024), std::string("1.00 KiB"));
  EXPECT_EQ(lcr::format_bytes(1536), std::string("1.50 KiB"));
  EXPECT_EQ(lcr::format_bytes(static_cast<size_t>(2471628800)), std::string("2.30 GiB"));
  EXPECT_EQ(lcr::align_up(257, 256), static_cast<size_t>(512));
  EXPECT_EQ(lcr::align_up(256, 256), static_cast<size_t>(256));
  try {
    const int n = -3;
    LCR_CHECK(n > 0, "expected a positive length, got " << n);
    report(false, __FILE__, __LINE__, "LCR_CHECK did not throw");
  } catch (const lcr::Error& e) {
    const std::string what = e.what();
    EXPECT(what.find("expected a positive length, got -3") != std::string::npos);
    EXPECT(what.find("n > 0") != std::string::npos);
    EXPECT(what.find("test_host.cpp") != std::string::npos);
  }
}

// Pool and table sizes of both KV layouts (no device memory is touched).
void test_kv_geometry() {
  const ModelConfig c = ModelConfig::from_json_string(kLlama32_1B);
  const lcr::KvGeometry contiguous = lcr::KvGeometry::plan(c, 2048, lcr::KvLayout::kContiguous, 16);
  EXPECT_EQ(contiguous.page_size, 2048);
  EXPECT_EQ(contiguous.pool_pages, 16);
  EXPECT_EQ(contiguous.table_entries(), static_cast<size_t>(0));
  // [16 layers][8 kv heads][2048][64] per pool, as the reference sizes it.
  EXPECT_EQ(contiguous.pool_elements(), static_cast<size_t>(16) * 8 * 2048 * 64);
  const lcr::KvGeometry paged = lcr::KvGeometry::plan(c, 2050, lcr::KvLayout::kPaged, 16);
  EXPECT_EQ(paged.pages_per_layer, 129);  // ceil(2050 / 16)
  EXPECT_EQ(paged.pool_pages, 129 * 16);
  EXPECT_EQ(paged.page_elements, static_cast<size_t>(8) * 16 * 64);
  EXPECT_EQ(paged.table_entries(), static_cast<size_t>(129) * 16);
  EXPECT_EQ(paged.pool_elements(), static_cast<size_t>(129) * 16 * 8 * 16 * 64);
  // 32,768 bytes of keys and values per position (bf16), the reference's
  // per-position accounting.
  EXPECT_EQ(lcr::KvCache::bytes_for(c, 1), static_cast<size_t>(32768));
  EXPECT_THROWS("positive maximum sequence length", { lcr::KvGeometry::plan(c, 0, lcr::KvLayout::kPaged, 16); });
  // The reference's per-token byte accounting (src/model.cu:86-102), written
  // out for Llama-3.2-1B: per layer two norms, q, k and v, o, gate/up/down;
  // then the final norm and the output head.
  const size_t H = 2048, Q = 2048, KV = 512, F = 8192, V = 128256;
  const size_t per_layer = 2 * H + Q * H + 2 * KV * H + H * Q + 3 * F * H;
  EXPECT_EQ(lcr::weight_bytes_per_token(c, 2), (16 * per_layer + H + V * H) * 2);
  EXPECT_EQ(lcr::weight_bytes_per_token(c, 2), static_cast<size_t>(2471628800));
  EXPECT_EQ(c.kv_bytes_per_token(2), static_cast<size_t>(32768));
  EXPECT_THROWS("positive page size", { lcr::KvGeometry::plan(c, 64, lcr::KvLayout::kPaged, 0); });
}

}  // namespace

int main() {
  test_config_parse();
  test_config_optional_fields();
  test_config_rejections();
  test_rope_frequencies();
  test_safetensors_well_formed();
  test_safetensors_sharded();
  test_safetensors_rejections();
  test_safetensors_writer_round_trip();
  test_json();
  test_common();
  test_kv_geometry();
  if (g_failures == 0) {
    std::printf("test_host: all checks passed\n");
    return 0;
  }
  std::fprintf(stderr, "test_host: %d check(s) failed\n", g_failures);
  return 1;
}
