// lcr-inspect: what a checkpoint holds and what decoding it costs, without a
// GPU. The counterpart of the reference's tools/inspect_main.cpp:63-136: the
// config, whether every tensor the token loop reads is present with the
// expected shape and one element type, and the byte accounting that bounds
// decode (src/model.cu:86-102: weight bytes streamed per token, KV-cache
// bytes per position), here turned into the HBM-roofline token rate of the
// device (MI355X: 8.0 TB/s by default) at the contexts the benchmark runs.
//
//   lcr-inspect --model DIR [--tensors] [--max-seq N] [--page-size N]
//               [--peak-gbs X] [--json]
//
// Exit status: 0 when the checkpoint is complete, 1 when a tensor is missing
// or misshapen (each problem is listed), 2 on a usage error.
#include <cstdio>
#include <fstream>
#include <string>
#include <vector>

#include "../common.h"
#include "../config.h"
#include "../json.h"
#include "../safetensors.h"
#include "../tokenizer.h"

namespace {

struct Options {
  std::string model_dir;
  bool list_tensors = false;
  bool json = false;
  int max_seq = 4096;
  int page_size = 16;
  double peak_gbs = 8000.0;  // MI355X HBM3E
};

int usage() {
  std::fprintf(stderr,
               "usage: lcr-inspect --model DIR [--tensors] [--max-seq N] [--page-size N] "
               "[--peak-gbs X] [--json]\n");
  return 2;
}

bool parse(int argc, char** argv, Options* o) {
  for (int i = 1; i < argc; ++i) {
    const std::string flag = argv[i];
    auto value = [&]() -> std::string {
      LCR_CHECK(i + 1 < argc, flag << " needs a value");
      return argv[++i];
    };
    if (flag == "--model") o->model_dir = value();
    else if (flag == "--tensors") o->list_tensors = true;
    else if (flag == "--json") o->json = true;
    else if (flag == "--max-seq") o->max_seq = std::stoi(value());
    else if (flag == "--page-size") o->page_size = std::stoi(value());
    else if (flag == "--peak-gbs") o->peak_gbs = std::stod(value());
    else return false;
  }
  return !o->model_dir.empty() && o->max_seq > 0 && o->page_size > 0 && o->peak_gbs > 0;
}

struct Report {
  lcr::ModelConfig config;
  size_t tensors_in_file = 0;
  size_t tensors_required = 0;
  size_t bytes_on_disk = 0;
  bool tied_head = true;
  std::string element_type = "unknown";
  size_t element_size = 2;
  std::vector<std::string> problems;
  size_t weight_bytes_per_token = 0;
  size_t kv_bytes_per_position = 0;
  int tokenizer_entries = -1;  // -1: no tokenizer.json
  int tokenizer_bos = -1;
};

Report inspect(const Options& o, const lcr::SafetensorsArchive& archive) {
  Report r;
  r.config = lcr::ModelConfig::load(o.model_dir);
  const std::vector<lcr::WeightSpec> specs = lcr::required_weights(r.config);
  r.tensors_in_file = archive.tensor_count();
  r.tensors_required = specs.size();
  r.bytes_on_disk = archive.total_bytes();
  r.tied_head = !archive.has("lm_head.weight");
  bool first = true;
  for (const lcr::WeightSpec& spec : specs) {
    const lcr::TensorView* t = archive.find(spec.name);
    if (t == nullptr) {
      r.problems.push_back("missing " + spec.name);
      continue;
    }
    try {
      t->expect_shape(spec.shape);
    } catch (const std::exception& e) {
      r.problems.push_back(e.what());
      continue;
    }
    if (first) {
      r.element_type = lcr::dtype_name(t->dtype);
      r.element_size = lcr::dtype_size(t->dtype);
      first = false;
    } else if (lcr::dtype_name(t->dtype) != r.element_type) {
      r.problems.push_back(spec.name + " is " + lcr::dtype_name(t->dtype) + ", the others " + r.element_type);
    }
  }
  if (!r.tied_head) {
    const lcr::TensorView& head = archive.get("lm_head.weight");
    try {
      head.expect_shape({r.config.vocab_size, r.config.hidden_size});
    } catch (const std::exception& e) {
      r.problems.push_back(e.what());
    }
  }
  r.weight_bytes_per_token = lcr::weight_bytes_per_token(r.config, r.element_size);
  r.kv_bytes_per_position = r.config.kv_bytes_per_token(r.element_size);
  const std::string tok_path = o.model_dir + "/tokenizer.json";
  if (std::ifstream(tok_path).good()) {
    const lcr::Tokenizer tok = lcr::Tokenizer::from_file(tok_path);
    r.tokenizer_entries = tok.vocab_size();
    r.tokenizer_bos = tok.bos_id();
    if (r.tokenizer_entries != r.config.vocab_size) {
      r.problems.push_back("tokenizer has " + std::to_string(r.tokenizer_entries) +
                           " entries but config.json says " + std::to_string(r.config.vocab_size));
    }
  }
  return r;
}

// Contexts the benchmark configurations decode at.
const int kContexts[] = {128, 256, 2048, 8192, 32768};

void print_text(const Options& o, const Report& r, const lcr::SafetensorsArchive& archive) {
  const lcr::ModelConfig& c = r.config;
  std::printf("config\n  %s\n", c.summary().c_str());
  std::printf("  context window       %d positions\n", c.max_position_embeddings);
  std::printf("  grouped-query        %d query heads per key/value head\n", c.heads_per_kv());
  std::printf("  stop tokens          ");
  for (size_t i = 0; i < c.eos_token_ids.size(); ++i) std::printf("%s%d", i ? ", " : "", c.eos_token_ids[i]);
  std::printf("\n\ncheckpoint\n");
  std::printf("  tensors in file      %zu\n", r.tensors_in_file);
  std::printf("  tensors required     %zu%s\n", r.tensors_required,
              r.tied_head ? " (output head tied to the embedding)" : " plus lm_head.weight");
  std::printf("  bytes on disk        %s\n", lcr::format_bytes(r.bytes_on_disk).c_str());
  std::printf("  element type         %s\n", r.element_type.c_str());
  if (r.problems.empty()) {
    std::printf("  every required tensor is present with the expected shape\n");
  } else {
    std::printf("  %zu problem(s):\n", r.problems.size());
    for (const std::string& p : r.problems) std::printf("    %s\n", p.c_str());
  }
  std::printf("\ndecode cost per token (bytes every step moves from HBM)\n");
  std::printf("  weights streamed     %zu B (%s)\n", r.weight_bytes_per_token,
              lcr::format_bytes(r.weight_bytes_per_token).c_str());
  std::printf("  KV per position      %zu B\n", r.kv_bytes_per_position);
  std::printf("  at %.0f GB/s peak:\n", o.peak_gbs);
  for (int ctx : kContexts) {
    const double bytes = static_cast<double>(r.weight_bytes_per_token) +
                         static_cast<double>(ctx) * static_cast<double>(r.kv_bytes_per_position);
    std::printf("    context %6d      %s per token, roofline %.0f tok/s\n", ctx,
                lcr::format_bytes(static_cast<size_t>(bytes)).c_str(), o.peak_gbs * 1e9 / bytes);
  }
  std::printf("\nkv cache\n");
  std::printf("  contiguous, --max-seq %d      %s\n", o.max_seq,
              lcr::format_bytes(static_cast<size_t>(o.max_seq) * r.kv_bytes_per_position).c_str());
  std::printf("  contiguous, full context %d  %s\n", c.max_position_embeddings,
              lcr::format_bytes(static_cast<size_t>(c.max_position_embeddings) * r.kv_bytes_per_position).c_str());
  std::printf("  paged, one %d-position page over all layers  %s\n", o.page_size,
              lcr::format_bytes(static_cast<size_t>(o.page_size) * r.kv_bytes_per_position).c_str());
  if (r.tokenizer_entries >= 0) {
    std::printf("\ntokenizer\n  %d entries, begin-of-text id %d\n", r.tokenizer_entries, r.tokenizer_bos);
  }
  if (o.list_tensors) {
    std::printf("\ntensors\n");
    for (const std::string& name : archive.names()) {
      const lcr::TensorView& t = archive.get(name);
      std::printf("  %-52s %-5s %-16s %s\n", name.c_str(), lcr::dtype_name(t.dtype), t.shape_string().c_str(),
                  lcr::format_bytes(t.nbytes).c_str());
    }
  }
}

void print_json(const Options& o, const Report& r) {
  using lcr::json::Value;
  const lcr::ModelConfig& c = r.config;
  Value root = Value::object();
  Value cfg = Value::object();
  cfg.set("hidden_size", Value::integer(c.hidden_size));
  cfg.set("intermediate_size", Value::integer(c.intermediate_size));
  cfg.set("num_layers", Value::integer(c.num_layers));
  cfg.set("num_heads", Value::integer(c.num_heads));
  cfg.set("num_kv_heads", Value::integer(c.num_kv_heads));
  cfg.set("head_dim", Value::integer(c.head_dim));
  cfg.set("vocab_size", Value::integer(c.vocab_size));
  cfg.set("max_position_embeddings", Value::integer(c.max_position_embeddings));
  root.set("config", cfg);
  Value ck = Value::object();
  ck.set("tensors_in_file", Value::integer(static_cast<int64_t>(r.tensors_in_file)));
  ck.set("tensors_required", Value::integer(static_cast<int64_t>(r.tensors_required)));
  ck.set("bytes_on_disk", Value::integer(static_cast<int64_t>(r.bytes_on_disk)));
  ck.set("tied_head", Value::boolean(r.tied_head));
  ck.set("element_type", Value::string(r.element_type));
  Value problems = Value::array();
  for (const std::string& p : r.problems) problems.push_back(Value::string(p));
  ck.set("problems", problems);
  root.set("checkpoint", ck);
  root.set("weight_bytes_per_token", Value::integer(static_cast<int64_t>(r.weight_bytes_per_token)));
  root.set("kv_bytes_per_position", Value::integer(static_cast<int64_t>(r.kv_bytes_per_position)));
  root.set("peak_gbs", Value::number(o.peak_gbs, false));
  Value roof = Value::array();
  for (int ctx : kContexts) {
    const double bytes = static_cast<double>(r.weight_bytes_per_token) +
                         static_cast<double>(ctx) * static_cast<double>(r.kv_bytes_per_position);
    Value row = Value::object();
    row.set("context", Value::integer(ctx));
    row.set("bytes_per_token", Value::number(bytes, false));
    row.set("roofline_tok_s", Value::number(o.peak_gbs * 1e9 / bytes, false));
    roof.push_back(row);
  }
  root.set("roofline", roof);
  Value kv = Value::object();
  kv.set("contiguous_max_seq_bytes",
         Value::integer(static_cast<int64_t>(o.max_seq) * static_cast<int64_t>(r.kv_bytes_per_position)));
  kv.set("page_bytes", Value::integer(static_cast<int64_t>(o.page_size) * static_cast<int64_t>(r.kv_bytes_per_position)));
  root.set("kv_cache", kv);
  if (r.tokenizer_entries >= 0) {
    Value tk = Value::object();
    tk.set("entries", Value::integer(r.tokenizer_entries));
    tk.set("bos_id", Value::integer(r.tokenizer_bos));
    root.set("tokenizer", tk);
  }
  std::printf("%s\n", root.dump().c_str());
}

}  // namespace

int main(int argc, char** argv) {
  Options o;
  try {
    if (!parse(argc, argv, &o)) return usage();
    const lcr::SafetensorsArchive archive(o.model_dir);
    const Report r = inspect(o, archive);
    if (o.json) {
      print_json(o, r);
    } else {
      print_text(o, r, archive);
    }
    return r.problems.empty() ? 0 : 1;
  } catch (const std::exception& e) {
    std::fprintf(stderr, "error: %s\n", e.what());
    return 1;
  }
}
