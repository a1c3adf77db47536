// lcr-validate: layer-by-layer drift of this runtime against a reference
// activation dump. The counterpart of the reference's tools/validate_main.cu:
// the same dump format (a manifest.json naming the prompt's input_ids, the
// float32 [tokens][width] tensors "embed", "layer_<i>", "final_norm" and
// "logits", and optionally a greedy_continuation, as tools/dump_reference.py
// writes them), the same figures per tensor (max-abs, RMS error, RMS error
// over RMS of the reference, smallest per-row cosine), the same pass rule
// (rel-RMS <= --max-relative-rms, default 0.02, and cosine >= --min-cosine,
// default 0.999), the top-5 next tokens and an optional greedy continuation.
//
// The prompt runs as one prefill chunk so every tap covers all of it; the
// prefill takes the MFMA path (or the decode path with --decode-path, for a
// bit-for-bit comparison with a CPU-oracle dump). --json prints the report
// as one JSON object.
//
//   lcr-validate --model DIR --reference DUMP [--generate N] [--json]
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <fstream>
#include <sstream>
#include <string>
#include <vector>

#include "../json.h"
#include "../model.h"

namespace {

struct Tensor {
  std::string name;
  int rows = 0;
  int width = 0;
  std::vector<float> values;
};

struct Dump {
  std::vector<int> input_ids;
  std::vector<Tensor> tensors;
  std::vector<int> greedy;
  std::string dtype;
  const Tensor* find(const std::string& name) const {
    for (const Tensor& t : tensors) {
      if (t.name == name) return &t;
    }
    return nullptr;
  }
};

std::string slurp(const std::string& path) {
  std::ifstream in(path, std::ios::binary);
  LCR_CHECK(in.good(), "cannot read " << path);
  std::ostringstream ss;
  ss << in.rdbuf();
  return ss.str();
}

Dump load_dump(const std::string& dir) {
  using lcr::json::Value;
  Value doc;
  std::string err;
  LCR_CHECK(lcr::json::parse(slurp(dir + "/manifest.json"), &doc, &err), dir << "/manifest.json: " << err);
  Dump d;
  if (const Value* dt = doc.find("dtype")) d.dtype = dt->is_string() ? dt->as_string() : "";
  for (const Value& v : doc.at("input_ids").items()) d.input_ids.push_back(v.as_int());
  if (const Value* g = doc.find("greedy_continuation")) {
    for (const Value& v : g->items()) d.greedy.push_back(v.as_int());
  }
  for (const Value& e : doc.at("tensors").items()) {
    Tensor t;
    t.name = e.at("name").as_string();
    const auto& shape = e.at("shape").items();
    LCR_CHECK(shape.size() == 2, "tensor \"" << t.name << "\" in the dump is not 2-D");
    t.rows = shape[0].as_int();
    t.width = shape[1].as_int();
    const std::string bytes = slurp(dir + "/" + e.at("file").as_string());
    const size_t n = static_cast<size_t>(t.rows) * static_cast<size_t>(t.width);
    LCR_CHECK(bytes.size() == n * sizeof(float),
              e.at("file").as_string() << " holds " << bytes.size() << " bytes, the shape needs " << n * 4);
    t.values.resize(n);
    std::copy(bytes.data(), bytes.data() + bytes.size(), reinterpret_cast<char*>(t.values.data()));
    d.tensors.push_back(std::move(t));
  }
  return d;
}

struct Drift {
  double max_abs = 0.0;
  double rms_error = 0.0;
  double rel_rms = 0.0;
  double min_cosine = 1.0;
};

// Over [rows][width]: error statistics over every element, cosine per row.
Drift drift(const float* ours, const float* theirs, int rows, int width) {
  Drift r;
  double err2 = 0.0, ref2 = 0.0;
  for (int row = 0; row < rows; ++row) {
    double dot = 0.0, na = 0.0, nb = 0.0;
    for (int i = 0; i < width; ++i) {
      const size_t k = static_cast<size_t>(row) * width + i;
      const double a = ours[k], b = theirs[k];
      r.max_abs = std::max(r.max_abs, std::fabs(a - b));
      err2 += (a - b) * (a - b);
      ref2 += b * b;
      dot += a * b;
      na += a * a;
      nb += b * b;
    }
    if (na > 0.0 && nb > 0.0) r.min_cosine = std::min(r.min_cosine, dot / std::sqrt(na * nb));
  }
  const double count = static_cast<double>(rows) * width;
  r.rms_error = std::sqrt(err2 / count);
  const double rms_ref = std::sqrt(ref2 / count);
  r.rel_rms = rms_ref > 0.0 ? r.rms_error / rms_ref : 0.0;
  return r;
}

std::vector<int> top_k(const std::vector<float>& v, int k) {
  std::vector<int> idx(v.size());
  for (size_t i = 0; i < idx.size(); ++i) idx[i] = static_cast<int>(i);
  k = std::min<int>(k, static_cast<int>(idx.size()));
  std::partial_sort(idx.begin(), idx.begin() + k, idx.end(), [&](int a, int b) {
    return v[static_cast<size_t>(a)] > v[static_cast<size_t>(b)] ||
           (v[static_cast<size_t>(a)] == v[static_cast<size_t>(b)] && a < b);
  });
  idx.resize(static_cast<size_t>(k));
  return idx;
}

int run(int argc, char** argv) {
  std::string model_dir, dump_dir;
  double max_rel_rms = 0.02, min_cos = 0.999;
  int device = 0, generate = 0;
  bool json_out = false, decode_path = false;
  for (int i = 1; i < argc; ++i) {
    const std::string f = argv[i];
    auto value = [&]() -> std::string {
      LCR_CHECK(i + 1 < argc, f << " needs a value");
      return argv[++i];
    };
    if (f == "--model") model_dir = value();
    else if (f == "--reference") dump_dir = value();
    else if (f == "--max-relative-rms") max_rel_rms = std::stod(value());
    else if (f == "--min-cosine") min_cos = std::stod(value());
    else if (f == "--device") device = std::stoi(value());
    else if (f == "--generate") generate = std::stoi(value());
    else if (f == "--json") json_out = true;
    else if (f == "--decode-path") decode_path = true;
    else {
      std::fprintf(stderr,
                   "usage: lcr-validate --model DIR --reference DIR [--max-relative-rms X] [--min-cosine X] "
                   "[--generate N] [--decode-path] [--json]\n");
      return 2;
    }
  }
  LCR_CHECK(!model_dir.empty() && !dump_dir.empty(), "--model and --reference are both required");
  const Dump dump = load_dump(dump_dir);
  LCR_CHECK(!dump.input_ids.empty(), "the dump has no input_ids");
  const int T = static_cast<int>(dump.input_ids.size());

  lcr::Model::Options o;
  o.device = device;
  o.prefill_chunk = T;
  o.max_seq = T + std::max(1, generate) + 1;
  o.prefill_via_decode = decode_path;
  lcr::Model model(model_dir, o);
  model.set_capture_activations(!decode_path);
  const float* dev_logits = model.prefill(dump.input_ids);
  const std::vector<float> logits = model.logits_to_host(dev_logits);

  using lcr::json::Value;
  Value report = Value::object();
  Value rows = Value::array();
  bool ok = true;
  if (!json_out) {
    std::printf("reference: %d tokens (%s)\n\n%-14s %10s %12s %12s %10s\n", T, dump.dtype.c_str(), "tensor",
                "max abs", "rms error", "rel rms", "min cos");
  }
  auto add_row = [&](const std::string& name, const Drift& d) {
    const bool pass = d.rel_rms <= max_rel_rms && d.min_cosine >= min_cos;
    ok = ok && pass;
    if (json_out) {
      Value r = Value::object();
      r.set("tensor", Value::string(name));
      r.set("max_abs", Value::number(d.max_abs, false));
      r.set("rms_error", Value::number(d.rms_error, false));
      r.set("rel_rms", Value::number(d.rel_rms, false));
      r.set("min_cosine", Value::number(d.min_cosine, false));
      r.set("pass", Value::boolean(pass));
      rows.push_back(r);
    } else {
      std::printf("%-14s %10.5f %12.6f %12.2e %10.6f %s\n", name.c_str(), d.max_abs, d.rms_error, d.rel_rms,
                  d.min_cosine, pass ? "" : " FAIL");
    }
  };
  for (const lcr::Model::Tap& tap : model.activation_taps()) {
    const Tensor* ref = dump.find(tap.name);
    if (ref == nullptr) continue;
    LCR_CHECK(ref->rows == tap.tokens && ref->width == tap.width,
              "tensor \"" << tap.name << "\" is " << ref->rows << "x" << ref->width << " in the dump, "
                          << tap.tokens << "x" << tap.width << " here");
    add_row(tap.name, drift(tap.values.data(), ref->values.data(), tap.tokens, tap.width));
  }
  std::vector<int> ours_top, theirs_top;
  if (const Tensor* ref = dump.find("logits")) {
    LCR_CHECK(ref->width == static_cast<int>(logits.size()),
              "logits are " << ref->width << " wide in the dump, " << logits.size() << " here");
    // The last row decides the next token; that is the one the runtime keeps.
    const float* last = ref->values.data() + static_cast<size_t>(ref->rows - 1) * ref->width;
    add_row("logits", drift(logits.data(), last, 1, ref->width));
    ours_top = top_k(logits, 5);
    theirs_top = top_k(std::vector<float>(last, last + ref->width), 5);
    if (ours_top[0] != theirs_top[0]) ok = false;
  }
  int matched = -1, compared = 0;
  if (generate > 0 && !dump.greedy.empty()) {
    std::vector<int> produced;
    const float* cur = dev_logits;
    model.set_capture_activations(false);
    const int steps = std::min<int>(generate, static_cast<int>(dump.greedy.size()));
    for (int s = 0; s < steps; ++s) {
      const int tok = model.sample(cur, 0.0f, 0, 1.0f, 0.0f);
      produced.push_back(tok);
      if (model.config().is_eos(tok) || s + 1 == steps) break;
      cur = model.decode(tok);
    }
    compared = static_cast<int>(produced.size());
    matched = 0;
    while (matched < compared && produced[static_cast<size_t>(matched)] == dump.greedy[static_cast<size_t>(matched)]) {
      ++matched;
    }
  }
  if (json_out) {
    report.set("tokens", Value::integer(T));
    report.set("tensors", rows);
    Value a = Value::array(), b = Value::array();
    for (int i : ours_top) a.push_back(Value::integer(i));
    for (int i : theirs_top) b.push_back(Value::integer(i));
    report.set("top5_ours", a);
    report.set("top5_reference", b);
    if (matched >= 0) {
      report.set("greedy_matched", Value::integer(matched));
      report.set("greedy_compared", Value::integer(compared));
    }
    report.set("pass", Value::boolean(ok));
    std::printf("%s\n", report.dump().c_str());
  } else {
    if (!ours_top.empty()) {
      std::printf("\ntop-5 next tokens\n  ours  ");
      for (int i : ours_top) std::printf(" %d", i);
      std::printf("\n  dump  ");
      for (int i : theirs_top) std::printf(" %d", i);
      std::printf("\n");
    }
    if (matched >= 0) std::printf("\ngreedy continuation: %d of %d tokens identical\n", matched, compared);
    std::printf("\n%s\n", ok ? "every tensor is within tolerance" : "one or more tensors are outside tolerance");
  }
  return ok ? 0 : 1;
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
