// llama-run: generate text from a checkpoint on one MI355X, or measure how
// fast it generates. The counterpart of the reference's src/main.cu:52-466:
// the same options and defaults, the Llama 3 chat template, streaming output
// held back to whole UTF-8 characters, and the benchmark report as text or
// as JSON with the reference's field names (what its tools/benchmark.py
// reads).
//
// Decoding is the reference's host loop: per token, Model::sample on the
// current logits and then Model::decode (the graph-replayed fused step).
// Sampling draws come from the Philox4x32-10 stream of --seed (philox.h)
// rather than std::mt19937_64, so a run is reproducible across hosts and
// comparable draw for draw with the CPU oracle's sampler.
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "../hip_utils.h"
#include "../json.h"
#include "../model.h"
#include "../philox.h"
#include "../tokenizer.h"

namespace {

using lcr::Model;

struct Args {
  std::string model_dir;
  std::string prompt = "The capital of France is";
  std::string system_prompt;
  bool chat = false;
  bool benchmark = false;
  int max_new_tokens = 128;
  float temperature = 0.0f;
  int top_k = 0;
  float top_p = 0.95f;
  uint64_t seed = 0;
  int max_seq = 4096;
  int prefill_chunk = 2048;
  int page_size = 16;
  bool paged = false;
  int attention_splits = 0;
  int device = 0;
  double peak_bandwidth_gb = 0.0;  // 0: the device's published peak
  int warmup = 0;
  bool profile = false;
  bool quiet = false;
  bool json_output = false;
};

[[noreturn]] void usage(int code) {
  std::fprintf(stderr,
               "usage: llama-run --model DIR [options]\n"
               "\n"
               "  --model DIR            checkpoint directory (config.json, tokenizer.json,\n"
               "                         model.safetensors)\n"
               "  --prompt TEXT          prompt text (default: a short completion)\n"
               "  --system TEXT          system message, chat mode only\n"
               "  --chat                 wrap the prompt in the Llama 3 chat template\n"
               "  --max-tokens N         tokens to generate (default 128)\n"
               "  --temperature T        0 means greedy, which is the default\n"
               "  --top-k K              0 disables the top-k cut (default)\n"
               "  --top-p P              nucleus threshold (default 0.95)\n"
               "  --seed S               seed of the Philox sampling draws\n"
               "  --max-seq N            KV cache capacity in positions (default 4096)\n"
               "  --prefill-chunk N      prompt positions per prefill pass (default 2048)\n"
               "  --paged                use the paged KV cache\n"
               "  --page-size N          positions per page (default 16)\n"
               "  --splits N             decode attention splits, 0 to choose\n"
               "  --device N             HIP device index\n"
               "  --peak-bandwidth GB    peak GB/s used in the report (default: the device's)\n"
               "  --bench                print timing and bandwidth after the text\n"
               "  --warmup N             discard N passes before timing (default 1 with --bench)\n"
               "  --profile              per-stage timing of the decode step (unfused kernels)\n"
               "  --json                 emit the benchmark report as JSON\n"
               "  --quiet                suppress the loading banner\n");
  std::exit(code);
}

std::string need(int argc, char** argv, int* i) {
  LCR_CHECK(*i + 1 < argc, argv[*i] << " needs a value");
  return argv[++(*i)];
}

Args parse_args(int argc, char** argv) {
  Args a;
  bool warmup_set = false;
  for (int i = 1; i < argc; ++i) {
    const std::string f = argv[i];
    if (f == "--model") a.model_dir = need(argc, argv, &i);
    else if (f == "--prompt") a.prompt = need(argc, argv, &i);
    else if (f == "--system") a.system_prompt = need(argc, argv, &i);
    else if (f == "--chat") a.chat = true;
    else if (f == "--bench") a.benchmark = true;
    else if (f == "--json") a.benchmark = a.json_output = true;
    else if (f == "--profile") a.profile = a.benchmark = true;
    else if (f == "--warmup") { a.warmup = std::stoi(need(argc, argv, &i)); warmup_set = true; }
    else if (f == "--quiet") a.quiet = true;
    else if (f == "--paged") a.paged = true;
    else if (f == "--max-tokens") a.max_new_tokens = std::stoi(need(argc, argv, &i));
    else if (f == "--temperature") a.temperature = std::stof(need(argc, argv, &i));
    else if (f == "--top-k") a.top_k = std::stoi(need(argc, argv, &i));
    else if (f == "--top-p") a.top_p = std::stof(need(argc, argv, &i));
    else if (f == "--seed") a.seed = std::stoull(need(argc, argv, &i));
    else if (f == "--max-seq") a.max_seq = std::stoi(need(argc, argv, &i));
    else if (f == "--prefill-chunk") a.prefill_chunk = std::stoi(need(argc, argv, &i));
    else if (f == "--page-size") a.page_size = std::stoi(need(argc, argv, &i));
    else if (f == "--splits") a.attention_splits = std::stoi(need(argc, argv, &i));
    else if (f == "--device") a.device = std::stoi(need(argc, argv, &i));
    else if (f == "--peak-bandwidth") a.peak_bandwidth_gb = std::stod(need(argc, argv, &i));
    else if (f == "-h" || f == "--help") usage(0);
    else {
      std::fprintf(stderr, "unknown option: %s\n", f.c_str());
      usage(2);
    }
  }
  if (a.model_dir.empty()) {
    std::fprintf(stderr, "--model is required\n");
    usage(2);
  }
  if (!warmup_set && a.benchmark) a.warmup = 1;
  return a;
}

// The Llama 3 chat format: a header, a blank line and the body per message,
// each closed by <|eot_id|>; an open assistant header last, so the model
// answers as the assistant.
std::string chat_prompt(const std::string& system, const std::string& user) {
  std::string out = "<|begin_of_text|>";
  auto message = [&](const char* role, const std::string& body) {
    out += "<|start_header_id|>";
    out += role;
    out += "<|end_header_id|>\n\n";
    out += body;
    out += "<|eot_id|>";
  };
  if (!system.empty()) message("system", system);
  message("user", user);
  out += "<|start_header_id|>assistant<|end_header_id|>\n\n";
  return out;
}

// Writes text as it is generated, holding back the bytes of a character that
// is not yet complete (a token can end inside a UTF-8 sequence).
class Utf8Writer {
 public:
  void feed(const std::string& bytes) {
    held_ += bytes;
    const size_t n = whole_characters(held_);
    if (n == 0) return;
    std::fwrite(held_.data(), 1, n, stdout);
    std::fflush(stdout);
    held_.erase(0, n);
  }
  void flush() {
    std::fwrite(held_.data(), 1, held_.size(), stdout);
    std::fflush(stdout);
    held_.clear();
  }

 private:
  // Bytes up to the start of a trailing incomplete sequence.
  static size_t whole_characters(const std::string& s) {
    size_t i = 0;
    while (i < s.size()) {
      const unsigned char c = static_cast<unsigned char>(s[i]);
      const size_t width = c < 0x80 ? 1 : (c >> 5) == 0x6 ? 2 : (c >> 4) == 0xE ? 3 : (c >> 3) == 0x1E ? 4 : 1;
      if (i + width > s.size()) break;
      i += width;
    }
    return i;
  }
  std::string held_;
};

struct Run {
  double load_ms = 0.0;
  int prompt_tokens = 0;
  double prefill_ms = 0.0;
  int decode_steps = 0;
  double decode_ms = 0.0;
  int final_length = 0;
};

struct Bandwidth {
  double bytes_per_token = 0.0;
  double achieved = 0.0;  // bytes per second
  double peak = 0.0;
};

Bandwidth bandwidth(const Args& a, const Model& m, const lcr::DeviceInfo& dev, const Run& r) {
  Bandwidth b;
  b.peak = a.peak_bandwidth_gb > 0.0 ? a.peak_bandwidth_gb * 1e9 : dev.peak_bandwidth_bytes_per_second();
  // Every weight once per token, plus the cache read at the run's mean length.
  const double mean_len = r.prompt_tokens + (r.decode_steps + 1) / 2.0;
  b.bytes_per_token = static_cast<double>(m.stats().weight_bytes_per_token) +
                      mean_len * static_cast<double>(m.stats().kv_bytes_per_position);
  const double s_per_token = r.decode_ms / 1000.0 / std::max(1, r.decode_steps);
  b.achieved = b.bytes_per_token / s_per_token;
  return b;
}

size_t kv_bytes(const Model& m, int positions) { return lcr::KvCache::bytes_for(m.config(), positions); }

void print_report(const Args& a, const Model& m, const lcr::DeviceInfo& dev, const Run& r) {
  const Bandwidth b = bandwidth(a, m, dev, r);
  std::printf("\ndevice            %s\n", dev.summary().c_str());
  std::printf("model             %s\n", m.config().summary().c_str());
  std::printf("weights resident  %s\n", lcr::format_bytes(m.weight_bytes()).c_str());
  std::printf("activation arena  %s\n", m.arena().usage_string().c_str());
  std::printf("kv cache          %s\n\n", m.kv_cache().usage_string().c_str());
  std::printf("prefill           %d tokens in %.2f ms (%.0f tokens/s)\n", r.prompt_tokens, r.prefill_ms,
              r.prompt_tokens / (r.prefill_ms / 1000.0));
  std::printf("decode            %d steps in %.2f ms (%.3f ms/token, %.1f tokens/s)\n\n", r.decode_steps,
              r.decode_ms, r.decode_ms / std::max(1, r.decode_steps), r.decode_steps / (r.decode_ms / 1000.0));
  std::printf("bytes per token   %s weights + %s cache at length %d\n",
              lcr::format_bytes(m.stats().weight_bytes_per_token).c_str(),
              lcr::format_bytes(m.stats().kv_bytes_at(r.final_length)).c_str(), r.final_length);
  std::printf("achieved          %.0f GB/s\n", b.achieved / 1e9);
  std::printf("peak              %.0f GB/s\n", b.peak / 1e9);
  std::printf("utilization       %.1f%% of peak\n\n", 100.0 * b.achieved / b.peak);
  const int paged_len = ((r.final_length + a.page_size - 1) / a.page_size) * a.page_size;
  std::printf("kv cache at this length:\n");
  std::printf("  contiguous, full %d-position context   %s\n", m.config().max_position_embeddings,
              lcr::format_bytes(kv_bytes(m, m.config().max_position_embeddings)).c_str());
  std::printf("  contiguous, --max-seq %d              %s\n", a.max_seq,
              lcr::format_bytes(kv_bytes(m, a.max_seq)).c_str());
  std::printf("  paged, page size %d                    %s\n", a.page_size,
              lcr::format_bytes(kv_bytes(m, paged_len)).c_str());
  std::printf("  strictly needed                        %s\n",
              lcr::format_bytes(kv_bytes(m, r.final_length)).c_str());
}

void print_json(const Args& a, const Model& m, const lcr::DeviceInfo& dev, const Run& r) {
  using lcr::json::Value;
  const Bandwidth b = bandwidth(a, m, dev, r);
  const auto num = [](double v) { return Value::number(v, false); };
  const auto integer = [](int64_t v) { return Value::integer(v); };
  const int paged_len = ((r.final_length + a.page_size - 1) / a.page_size) * a.page_size;
  Value d = Value::object();
  d.set("runtime", Value::string("llama-cuda-runtime_amd"));
  d.set("device", Value::string(dev.name));
  d.set("device_summary", Value::string(dev.summary()));
  d.set("multiprocessors", integer(dev.multiprocessors));
  d.set("dtype", Value::string(lcr::kElemName));
  d.set("model", Value::string(m.config().summary()));
  d.set("load_ms", num(r.load_ms));
  d.set("weight_bytes", integer(static_cast<int64_t>(m.weight_bytes())));
  d.set("arena_peak_bytes", integer(static_cast<int64_t>(m.arena().peak())));
  d.set("prompt_tokens", integer(r.prompt_tokens));
  d.set("prefill_ms", num(r.prefill_ms));
  d.set("prefill_tokens_per_second", num(r.prompt_tokens / (r.prefill_ms / 1000.0)));
  d.set("decode_steps", integer(r.decode_steps));
  d.set("decode_ms", num(r.decode_ms));
  d.set("decode_ms_per_token", num(r.decode_ms / std::max(1, r.decode_steps)));
  d.set("decode_tokens_per_second", num(r.decode_steps / (r.decode_ms / 1000.0)));
  d.set("weight_bytes_per_token", integer(static_cast<int64_t>(m.stats().weight_bytes_per_token)));
  d.set("kv_bytes_per_position", integer(static_cast<int64_t>(m.stats().kv_bytes_per_position)));
  d.set("bytes_per_token", num(b.bytes_per_token));
  d.set("achieved_bandwidth_bytes_per_second", num(b.achieved));
  d.set("peak_bandwidth_bytes_per_second", num(b.peak));
  d.set("bandwidth_utilization", num(b.achieved / b.peak));
  d.set("kv_layout", Value::string(a.paged ? "paged" : "contiguous"));
  d.set("kv_page_size", integer(a.page_size));
  d.set("sequence_length", integer(r.final_length));
  d.set("kv_bytes_contiguous_full_context",
        integer(static_cast<int64_t>(kv_bytes(m, m.config().max_position_embeddings))));
  d.set("kv_bytes_contiguous_max_seq", integer(static_cast<int64_t>(kv_bytes(m, a.max_seq))));
  d.set("kv_bytes_paged", integer(static_cast<int64_t>(kv_bytes(m, paged_len))));
  d.set("kv_bytes_ideal", integer(static_cast<int64_t>(kv_bytes(m, r.final_length))));
  std::printf("%s\n", d.dump().c_str());
}

void print_profile(const Model& m, int steps, double decode_ms) {
  const lcr::Profiler& p = m.profiler();
  const double measured = p.total_ms();
  steps = std::max(1, steps);
  std::printf("\nper-stage decode profile (unfused kernels), averaged over %d steps\n\n", steps);
  std::printf("%-30s %10s %11s %7s\n", "stage", "us/token", "% of stages", "calls");
  for (const lcr::Profiler::Entry& e : p.entries()) {
    std::printf("%-30s %10.1f %10.1f%% %7d\n", e.name.c_str(), 1000.0 * e.total_ms / steps,
                measured > 0 ? 100.0 * e.total_ms / measured : 0.0, e.launches / steps);
  }
  const double wall_us = 1000.0 * decode_ms / steps;
  std::printf("\nwall clock per token, profiled   %.1f us\n", wall_us);
  std::printf("sum of stage timings             %.1f us\n", 1000.0 * measured / steps);
  std::printf("between stages (launch, events)  %.1f us\n", wall_us - 1000.0 * measured / steps);
}

int run(int argc, char** argv) {
  const Args a = parse_args(argc, argv);
  const lcr::DeviceInfo dev = lcr::query_device(a.device);
  if (!a.quiet) std::fprintf(stderr, "device: %s\nloading %s\n", dev.summary().c_str(), a.model_dir.c_str());

  Run r;
  const auto t0 = std::chrono::steady_clock::now();
  const lcr::Tokenizer tokenizer = lcr::Tokenizer::from_model_dir(a.model_dir);
  Model::Options o;
  o.device = a.device;
  o.max_seq = a.max_seq;
  o.prefill_chunk = a.prefill_chunk;
  o.page_size = a.page_size;
  o.attention_splits = a.attention_splits;
  o.kv_layout = a.paged ? lcr::KvLayout::kPaged : lcr::KvLayout::kContiguous;
  // Stage timing needs the eagerly launched, unfused kernels.
  if (a.profile) o.fused_decode = false;
  Model model(a.model_dir, o);
  r.load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  if (!a.quiet) {
    std::fprintf(stderr, "loaded %s of weights in %.1f s\n", lcr::format_bytes(model.weight_bytes()).c_str(),
                 r.load_ms / 1000.0);
  }

  const std::string text = a.chat ? chat_prompt(a.system_prompt, a.prompt) : a.prompt;
  // A chat prompt carries its own <|begin_of_text|>; a raw completion gets one.
  const std::vector<int> prompt = tokenizer.encode(text, /*add_bos=*/!a.chat, /*parse_special=*/true);
  LCR_CHECK(!prompt.empty(), "the prompt encoded to no tokens");
  LCR_CHECK(prompt.size() < static_cast<size_t>(a.max_seq),
            "prompt of " << prompt.size() << " tokens does not fit in --max-seq " << a.max_seq);

  // Discarded passes: first launches load code objects and capture graphs.
  for (int i = 0; i < a.warmup; ++i) {
    const float* warm = model.prefill(prompt);
    model.decode(model.sample(warm, 0.0f, 0, 1.0f, 0.0f));
    model.reset();
  }
  if (a.profile) {
    model.profiler().reset();
    model.profiler().set_enabled(true);
  }

  Utf8Writer out;
  if (!a.chat) out.feed(text);
  const float* logits = model.prefill(prompt);
  r.prompt_tokens = static_cast<int>(prompt.size());
  r.prefill_ms = model.stats().last_prefill_ms;

  lcr::PhiloxUniforms draws(a.seed);
  const int budget = std::min(a.max_new_tokens, a.max_seq - static_cast<int>(prompt.size()));
  int generated = 0;
  // The prefill's logits give the first token; every later token needs one
  // decode step, so there is one step fewer than tokens.
  for (int step = 0; step < budget; ++step) {
    const int token = model.sample(logits, a.temperature, a.top_k, a.top_p, draws.next());
    if (model.config().is_eos(token)) break;
    out.feed(tokenizer.decode_one(token, /*skip_special=*/true));
    if (++generated >= budget) break;
    logits = model.decode(token);
    r.decode_ms += model.stats().last_decode_ms;
    ++r.decode_steps;
  }
  out.flush();
  std::printf("\n");
  r.final_length = model.position();

  if (a.benchmark) {
    if (a.json_output) {
      print_json(a, model, dev, r);
    } else {
      print_report(a, model, dev, r);
    }
    if (a.profile) print_profile(model, r.decode_steps, r.decode_ms);
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
