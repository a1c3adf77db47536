// llama-run: text generation from a checkpoint on one MI355X, with an
// optional speed report.
//
// The command line is the reference's (src/main.cu:52-470: the same flags and
// meanings, the Llama 3 chat template, the --json report fields its
// tools/benchmark.py reads); the program is built differently:
//  - one flag table drives parsing and the help text;
//  - a Session owns the model, tokenizer and draw stream and runs the
//    reference's host loop (sample the current logits, then decode the token)
//    into a sink that writes whole UTF-8 characters only;
//  - the report is one list of rows (label, JSON key, value, unit), printed
//    as aligned text or as one JSON object.
// Sampling draws come from the Philox4x32-10 stream of --seed (philox.h), so
// a run is reproducible across hosts and draw for draw comparable with the
// CPU oracle's sampler.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <utility>
#include <vector>

#include "../hip_utils.h"
#include "../json.h"
#include "../model.h"
#include "../philox.h"
#include "../tokenizer.h"

namespace {

// ---------------------------------------------------------------------------
// Settings and the flag table
// ---------------------------------------------------------------------------

struct Settings {
  std::string model_dir;
  std::string prompt = "The capital of France is";
  std::string system_message;
  bool chat = false;
  int max_new_tokens = 128;
  float temperature = 0.0f;  // 0: greedy
  int top_k = 0;
  float top_p = 0.95f;
  uint64_t seed = 0;
  lcr::Model::Options model;
  int warmup = -1;           // -1: 1 when reporting, else 0
  double peak_gbs = 0.0;     // 0: the device's published peak
  bool report = false;
  bool json = false;
  bool profile = false;
  bool quiet = false;
};

struct Flag {
  const char* name;
  const char* value;  // nullptr: a switch
  const char* help;
  std::function<void(Settings&, const std::string&)> apply;
};

int as_int(const std::string& v) { return std::stoi(v); }

const std::vector<Flag>& flags() {
  static const std::vector<Flag> table = {
      {"--model", "DIR", "checkpoint directory: config.json, tokenizer.json, model.safetensors",
       [](Settings& s, const std::string& v) { s.model_dir = v; }},
      {"--prompt", "TEXT", "prompt text (default: a short completion)",
       [](Settings& s, const std::string& v) { s.prompt = v; }},
      {"--system", "TEXT", "system message (with --chat)",
       [](Settings& s, const std::string& v) { s.system_message = v; }},
      {"--chat", nullptr, "wrap the prompt in the Llama 3 chat template",
       [](Settings& s, const std::string&) { s.chat = true; }},
      {"--max-tokens", "N", "tokens to generate (default 128)",
       [](Settings& s, const std::string& v) { s.max_new_tokens = as_int(v); }},
      {"--temperature", "T", "sampling temperature; 0 (default) is greedy",
       [](Settings& s, const std::string& v) { s.temperature = std::stof(v); }},
      {"--top-k", "K", "keep the K most likely tokens; 0 (default) keeps all",
       [](Settings& s, const std::string& v) { s.top_k = as_int(v); }},
      {"--top-p", "P", "nucleus mass (default 0.95)",
       [](Settings& s, const std::string& v) { s.top_p = std::stof(v); }},
      {"--seed", "S", "seed of the Philox sampling draws (default 0)",
       [](Settings& s, const std::string& v) { s.seed = std::stoull(v); }},
      {"--max-seq", "N", "KV cache capacity in positions (default 4096)",
       [](Settings& s, const std::string& v) { s.model.max_seq = as_int(v); }},
      {"--prefill-chunk", "N", "prompt positions per prefill pass (default 2048)",
       [](Settings& s, const std::string& v) { s.model.prefill_chunk = as_int(v); }},
      {"--paged", nullptr, "paged KV cache",
       [](Settings& s, const std::string&) { s.model.kv_layout = lcr::KvLayout::kPaged; }},
      {"--page-size", "N", "positions per cache page (default 16)",
       [](Settings& s, const std::string& v) { s.model.page_size = as_int(v); }},
      {"--splits", "N", "decode attention splits; 0 (default) chooses",
       [](Settings& s, const std::string& v) { s.model.attention_splits = as_int(v); }},
      {"--device", "N", "HIP device index (default 0)",
       [](Settings& s, const std::string& v) { s.model.device = as_int(v); }},
      {"--peak-bandwidth", "GB", "peak GB/s for the report (default: the device's)",
       [](Settings& s, const std::string& v) { s.peak_gbs = std::stod(v); }},
      {"--bench", nullptr, "report timing and bandwidth after the text",
       [](Settings& s, const std::string&) { s.report = true; }},
      {"--warmup", "N", "untimed passes first (default 1 with a report)",
       [](Settings& s, const std::string& v) { s.warmup = as_int(v); }},
      {"--profile", nullptr, "per-stage timing of the decode step (unfused kernels)",
       [](Settings& s, const std::string&) { s.profile = s.report = true; }},
      {"--json", nullptr, "the report as one JSON object",
       [](Settings& s, const std::string&) { s.json = s.report = true; }},
      {"--quiet", nullptr, "no loading messages",
       [](Settings& s, const std::string&) { s.quiet = true; }},
  };
  return table;
}

[[noreturn]] void print_help_and_exit(int code) {
  std::string text = "usage: llama-run --model DIR [options]\n\n";
  for (const Flag& f : flags()) {
    std::string left = std::string("  ") + f.name + (f.value ? std::string(" ") + f.value : "");
    left.resize(std::max<size_t>(left.size() + 1, 25), ' ');
    text += left + f.help + "\n";
  }
  text += "  -h, --help             this text\n";
  std::fputs(text.c_str(), code == 0 ? stdout : stderr);
  std::exit(code);
}

Settings read_command_line(int argc, char** argv) {
  Settings s;
  s.model.prefill_chunk = 2048;
  s.model.max_seq = 4096;
  const std::vector<std::string> words(argv + 1, argv + argc);
  for (size_t i = 0; i < words.size(); ++i) {
    if (words[i] == "-h" || words[i] == "--help") print_help_and_exit(0);
    const auto flag = std::find_if(flags().begin(), flags().end(),
                                   [&](const Flag& f) { return words[i] == f.name; });
    if (flag == flags().end()) {
      std::fprintf(stderr, "unknown option: %s\n", words[i].c_str());
      print_help_and_exit(2);
    }
    std::string value;
    if (flag->value != nullptr) {
      LCR_CHECK(i + 1 < words.size(), words[i] << " needs a value (" << flag->value << ")");
      value = words[++i];
    }
    flag->apply(s, value);
  }
  if (s.model_dir.empty()) {
    std::fprintf(stderr, "--model is required\n");
    print_help_and_exit(2);
  }
  if (s.warmup < 0) s.warmup = s.report ? 1 : 0;
  // Stage timing needs the unfused kernels, launched one by one.
  if (s.profile) s.model.fused_decode = false;
  return s;
}

// ---------------------------------------------------------------------------
// Prompt and output
// ---------------------------------------------------------------------------

// The Llama 3 chat format: every message is a role header, a blank line and
// the body, closed by <|eot_id|>; an open assistant header ends the prompt so
// the model answers as the assistant. The text carries its own
// <|begin_of_text|>.
std::string llama3_chat(const std::vector<std::pair<std::string, std::string>>& messages) {
  std::string out = "<|begin_of_text|>";
  for (const auto& [role, body] : messages) {
    out += "<|start_header_id|>" + role + "<|end_header_id|>\n\n" + body + "<|eot_id|>";
  }
  return out + "<|start_header_id|>assistant<|end_header_id|>\n\n";
}

// Writes bytes to stdout as they come, but never part of a character: a
// decoded token can end inside a multi-byte UTF-8 sequence. `owed` counts the
// continuation bytes the last lead byte still expects; output stops before
// that lead byte until they arrive.
class WholeCharacterSink {
 public:
  void write(const std::string& bytes) {
    for (const char ch : bytes) {
      const auto b = static_cast<unsigned char>(ch);
      if (owed_ > 0 && (b & 0xC0) == 0x80) {
        --owed_;
      } else {
        owed_ = 0;  // a new character (or a malformed one: pass it through)
        lead_ = pending_.size();
        if (b >= 0xF0) owed_ = 3;
        else if (b >= 0xE0) owed_ = 2;
        else if (b >= 0xC0) owed_ = 1;
      }
      pending_.push_back(ch);
    }
    const size_t ready = owed_ > 0 ? lead_ : pending_.size();
    emit(ready);
  }
  void finish() { emit(pending_.size()); }

 private:
  void emit(size_t n) {
    if (n == 0) return;
    std::fwrite(pending_.data(), 1, n, stdout);
    std::fflush(stdout);
    pending_.erase(0, n);
    lead_ = lead_ >= n ? lead_ - n : 0;
  }
  std::string pending_;
  size_t lead_ = 0;
  int owed_ = 0;
};

// ---------------------------------------------------------------------------
// The generation session
// ---------------------------------------------------------------------------

struct Timings {
  double load_ms = 0.0;
  int prompt_tokens = 0;
  double prefill_ms = 0.0;
  int decode_steps = 0;
  double decode_ms = 0.0;
  int final_length = 0;
};

class Session {
 public:
  explicit Session(const Settings& s) : s_(s) {
    const auto t0 = std::chrono::steady_clock::now();
    tokenizer_ = std::make_unique<lcr::Tokenizer>(lcr::Tokenizer::from_model_dir(s.model_dir));
    model_ = std::make_unique<lcr::Model>(s.model_dir, s.model);
    timings_.load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  }

  lcr::Model& model() { return *model_; }
  const Timings& timings() const { return timings_; }

  // The prompt's text (what is echoed) and its ids. A chat prompt brings its
  // own begin-of-text marker; a plain completion gets one added.
  std::string prompt_text() const {
    if (!s_.chat) return s_.prompt;
    std::vector<std::pair<std::string, std::string>> messages;
    if (!s_.system_message.empty()) messages.emplace_back("system", s_.system_message);
    messages.emplace_back("user", s_.prompt);
    return llama3_chat(messages);
  }
  std::vector<int> prompt_ids() const {
    const std::vector<int> ids = tokenizer_->encode(prompt_text(), /*add_bos=*/!s_.chat, /*parse_special=*/true);
    LCR_CHECK(!ids.empty(), "the prompt encoded to no tokens");
    LCR_CHECK(ids.size() < static_cast<size_t>(s_.model.max_seq),
              "prompt of " << ids.size() << " tokens does not fit in --max-seq " << s_.model.max_seq);
    return ids;
  }

  // Untimed passes (code object loading, graph capture): a prefill and one
  // greedy step each.
  void warm_up(const std::vector<int>& ids, int passes) {
    for (int i = 0; i < passes; ++i) {
      model_->decode(model_->sample(model_->prefill(ids), 0.0f, 0, 1.0f, 0.0f));
      model_->reset();
    }
  }

  // The reference's loop: the prefill's logits give the first token; each
  // later token costs one decode step. Stops at an end-of-sequence id, at
  // --max-tokens, or when the cache is full.
  void generate(const std::vector<int>& ids, const std::function<void(int)>& on_token) {
    lcr::PhiloxUniforms draws(s_.seed);
    const float* logits = model_->prefill(ids);
    timings_.prompt_tokens = static_cast<int>(ids.size());
    timings_.prefill_ms = model_->stats().last_prefill_ms;
    const int room = std::min(s_.max_new_tokens, s_.model.max_seq - static_cast<int>(ids.size()));
    for (int produced = 0; produced < room;) {
      const int token = model_->sample(logits, s_.temperature, s_.top_k, s_.top_p, draws.next());
      if (model_->config().is_eos(token)) break;
      on_token(token);
      if (++produced == room) break;
      logits = model_->decode(token);
      timings_.decode_ms += model_->stats().last_decode_ms;
      timings_.decode_steps += 1;
    }
    timings_.final_length = model_->position();
  }

  std::string text_of(int token) const { return tokenizer_->decode_one(token, /*skip_special=*/true); }

 private:
  const Settings& s_;
  std::unique_ptr<lcr::Tokenizer> tokenizer_;
  std::unique_ptr<lcr::Model> model_;
  Timings timings_;
};

// ---------------------------------------------------------------------------
// The report
// ---------------------------------------------------------------------------

// One figure: shown as "label  value unit" in text and as key: value in JSON
// (text-only rows have no key; JSON-only rows no label).
struct Row {
  const char* label;
  const char* key;
  lcr::json::Value value;
  std::string text;  // the value as printed
};

std::string fixed(double v, int digits) {
  char buf[64];
  std::snprintf(buf, sizeof buf, "%.*f", digits, v);
  return buf;
}

std::vector<Row> report_rows(const Settings& s, lcr::Model& m, const lcr::DeviceInfo& dev, const Timings& t) {
  using lcr::json::Value;
  const auto num = [](double v) { return Value::number(v, false); };
  const auto whole = [](int64_t v) { return Value::integer(v); };
  const auto bytes = [](size_t v) { return lcr::format_bytes(v); };
  const lcr::ForwardStats& st = m.stats();
  const lcr::ModelConfig& c = m.config();

  const int steps = std::max(1, t.decode_steps);
  const double ms_per_token = t.decode_ms / steps;
  // Every weight once per token, plus the cache read at the run's mean length
  // (the reference's accounting, src/model.cu:86-102).
  const double mean_length = t.prompt_tokens + (t.decode_steps + 1) / 2.0;
  const double per_token = static_cast<double>(st.weight_bytes_per_token) +
                           mean_length * static_cast<double>(st.kv_bytes_per_position);
  const double achieved = per_token / (ms_per_token / 1000.0);
  const double peak = s.peak_gbs > 0.0 ? s.peak_gbs * 1e9 : dev.peak_bandwidth_bytes_per_second();
  const int page = s.model.page_size;
  const int paged_positions = (t.final_length + page - 1) / page * page;
  const auto kv_at = [&](int64_t positions) { return lcr::KvCache::bytes_for(c, positions); };
  const bool paged = s.model.kv_layout == lcr::KvLayout::kPaged;

  return {
      {nullptr, "runtime", Value::string("llama-cuda-runtime_amd"), ""},
      {"device", "device", Value::string(dev.name), dev.summary()},
      {nullptr, "device_summary", Value::string(dev.summary()), ""},
      {nullptr, "multiprocessors", whole(dev.multiprocessors), ""},
      {"element type", "dtype", Value::string(lcr::kElemName), lcr::kElemName},
      {"model", "model", Value::string(c.summary()), c.summary()},
      {"load", "load_ms", num(t.load_ms), fixed(t.load_ms, 1) + " ms"},
      {"weights on device", "weight_bytes", whole(static_cast<int64_t>(m.weight_bytes())), bytes(m.weight_bytes())},
      {"activation arena", "arena_peak_bytes", whole(static_cast<int64_t>(m.arena().peak())),
       m.arena().usage_string()},
      {"kv cache", nullptr, Value(), m.kv_cache().usage_string()},
      {"prompt", "prompt_tokens", whole(t.prompt_tokens), std::to_string(t.prompt_tokens) + " tokens"},
      {"prefill", "prefill_ms", num(t.prefill_ms), fixed(t.prefill_ms, 2) + " ms"},
      {"prefill rate", "prefill_tokens_per_second", num(t.prompt_tokens / (t.prefill_ms / 1000.0)),
       fixed(t.prompt_tokens / (t.prefill_ms / 1000.0), 0) + " tokens/s"},
      {"decode steps", "decode_steps", whole(t.decode_steps), std::to_string(t.decode_steps)},
      {"decode", "decode_ms", num(t.decode_ms), fixed(t.decode_ms, 2) + " ms"},
      {"per token", "decode_ms_per_token", num(ms_per_token), fixed(ms_per_token, 3) + " ms"},
      {"decode rate", "decode_tokens_per_second", num(1000.0 / ms_per_token),
       fixed(1000.0 / ms_per_token, 1) + " tokens/s"},
      {"weights per token", "weight_bytes_per_token", whole(static_cast<int64_t>(st.weight_bytes_per_token)),
       bytes(st.weight_bytes_per_token)},
      {"cache per position", "kv_bytes_per_position", whole(static_cast<int64_t>(st.kv_bytes_per_position)),
       bytes(st.kv_bytes_per_position)},
      {"bytes per token", "bytes_per_token", num(per_token), fixed(per_token / 1e9, 4) + " GB"},
      {"achieved", "achieved_bandwidth_bytes_per_second", num(achieved), fixed(achieved / 1e9, 0) + " GB/s"},
      {"peak", "peak_bandwidth_bytes_per_second", num(peak), fixed(peak / 1e9, 0) + " GB/s"},
      {"of peak", "bandwidth_utilization", num(achieved / peak), fixed(100.0 * achieved / peak, 1) + " %"},
      {"kv layout", "kv_layout", Value::string(paged ? "paged" : "contiguous"),
       paged ? "paged, " + std::to_string(page) + " positions a page" : "contiguous"},
      {nullptr, "kv_page_size", whole(page), ""},
      {"sequence length", "sequence_length", whole(t.final_length), std::to_string(t.final_length)},
      {"kv, full context", "kv_bytes_contiguous_full_context",
       whole(static_cast<int64_t>(kv_at(c.max_position_embeddings))), bytes(kv_at(c.max_position_embeddings))},
      {"kv, --max-seq", "kv_bytes_contiguous_max_seq", whole(static_cast<int64_t>(kv_at(s.model.max_seq))),
       bytes(kv_at(s.model.max_seq))},
      {"kv, paged", "kv_bytes_paged", whole(static_cast<int64_t>(kv_at(paged_positions))),
       bytes(kv_at(paged_positions))},
      {"kv, this length", "kv_bytes_ideal", whole(static_cast<int64_t>(kv_at(t.final_length))),
       bytes(kv_at(t.final_length))},
  };
}

void print_rows(const std::vector<Row>& rows, bool as_json) {
  if (as_json) {
    lcr::json::Value doc = lcr::json::Value::object();
    for (const Row& r : rows) {
      if (r.key != nullptr) doc.set(r.key, r.value);
    }
    std::printf("%s\n", doc.dump().c_str());
    return;
  }
  std::printf("\n");
  for (const Row& r : rows) {
    if (r.label != nullptr) std::printf("%-20s %s\n", r.label, r.text.c_str());
  }
}

void print_stage_profile(const lcr::Profiler& p, const Timings& t) {
  const int steps = std::max(1, t.decode_steps);
  const double staged_us = 1000.0 * p.total_ms() / steps;
  std::printf("\ndecode stages (unfused kernels), per token over %d steps\n", steps);
  std::printf("%-32s %10s %8s %6s\n", "stage", "us", "share", "calls");
  for (const lcr::Profiler::Entry& e : p.entries()) {
    const double us = 1000.0 * e.total_ms / steps;
    std::printf("%-32s %10.1f %7.1f%% %6d\n", e.name.c_str(), us, staged_us > 0 ? 100.0 * us / staged_us : 0.0,
                e.launches / steps);
  }
  const double wall_us = 1000.0 * t.decode_ms / steps;
  std::printf("%-32s %10.1f\n%-32s %10.1f\n", "stages total", staged_us, "outside stages", wall_us - staged_us);
}

int run(int argc, char** argv) {
  const Settings s = read_command_line(argc, argv);
  const lcr::DeviceInfo dev = lcr::query_device(s.model.device);
  if (!s.quiet) std::fprintf(stderr, "device: %s\nloading %s\n", dev.summary().c_str(), s.model_dir.c_str());
  Session session(s);
  if (!s.quiet) {
    std::fprintf(stderr, "loaded %s of weights in %.1f s\n", lcr::format_bytes(session.model().weight_bytes()).c_str(),
                 session.timings().load_ms / 1000.0);
  }
  const std::vector<int> ids = session.prompt_ids();
  session.warm_up(ids, s.warmup);
  if (s.profile) {
    session.model().profiler().reset();
    session.model().profiler().set_enabled(true);
  }

  WholeCharacterSink out;
  if (!s.chat) out.write(s.prompt);  // a completion continues the prompt's text
  session.generate(ids, [&](int token) { out.write(session.text_of(token)); });
  out.finish();
  std::printf("\n");

  if (s.report) {
    print_rows(report_rows(s, session.model(), dev, session.timings()), s.json);
    if (s.profile) print_stage_profile(session.model().profiler(), session.timings());
  }
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  try {
    return run(argc, argv);
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
