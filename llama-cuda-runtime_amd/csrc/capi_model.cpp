// extern "C" wrapper of lcr::Model (include/lcr_model.h).
#include <algorithm>
#include <cstring>
#include <vector>

#include "../../include/lcr_model.h"
#include "capi_util.h"
#include "hip_utils.h"
#include "model.h"

struct lcr_model {
  std::unique_ptr<lcr::Model> impl;
};

using namespace lcr;

namespace {

Model& M(lcr_model* m) { return *m->impl; }
const Model& M(const lcr_model* m) { return *m->impl; }

#define CAPI_MODEL(m)                                          \
  do {                                                         \
    capi::clear_error();                                       \
    CAPI_CHECK((m) != nullptr && (m)->impl, "model handle is null"); \
  } while (0)

}  // namespace

extern "C" void lcr_model_default_options(lcr_model_options* o) {
  if (o == nullptr) return;
  o->device = 0;
  o->max_seq = 4096;
  o->paged = 0;
  o->page_size = 16;
  o->prefill_chunk = 2048;
  o->attention_splits = 0;
  o->fused_decode = 1;
  o->use_graph = 1;
  o->prefill_via_decode = 0;
  o->decode_exchange = 1;
  o->exchange_oproj = 1;
  o->exchange_split = 1;
  o->exchange_spins = 1 << 20;
  o->exchange_test_unwritten = 0;
  o->layer_grid = 0;
  o->exchange_head = 1;
}

extern "C" int lcr_model_create(const char* model_dir, const lcr_model_options* options,
                                lcr_model** out) {
  capi::clear_error();
  CAPI_CHECK(model_dir != nullptr && out != nullptr, "model directory and output handle needed");
  return capi::guarded([&]() -> int {
    lcr_model_options o;
    lcr_model_default_options(&o);
    if (options != nullptr) o = *options;
    Model::Options opt;
    opt.device = o.device;
    opt.max_seq = o.max_seq;
    opt.kv_layout = o.paged ? KvLayout::kPaged : KvLayout::kContiguous;
    opt.page_size = o.page_size;
    opt.prefill_chunk = o.prefill_chunk;
    opt.attention_splits = o.attention_splits;
    opt.fused_decode = o.fused_decode != 0;
    opt.use_graph = o.use_graph != 0;
    opt.prefill_via_decode = o.prefill_via_decode != 0;
    opt.decode_exchange = o.decode_exchange != 0;
    opt.exchange_oproj = o.exchange_oproj != 0;
    opt.exchange_split = o.exchange_split != 0;
    opt.exchange_spins = o.exchange_spins > 0 ? o.exchange_spins : (1 << 20);
    opt.exchange_test_unwritten = o.exchange_test_unwritten != 0;
    opt.layer_grid = o.layer_grid != 0;
    opt.exchange_head = o.exchange_head != 0;
    auto handle = std::make_unique<lcr_model>();
    handle->impl = std::make_unique<Model>(model_dir, opt);
    *out = handle.release();
    return LCR_OK;
  });
}

extern "C" void lcr_model_destroy(lcr_model* model) { delete model; }

extern "C" int lcr_model_exchange_status(const lcr_model* m, int* enabled, int* status) {
  CAPI_MODEL(m);
  CAPI_CHECK(enabled != nullptr && status != nullptr, "output pointers needed");
  return capi::guarded([&]() -> int {
    *enabled = m->impl->decode_exchange() ? (m->impl->exchange_oproj() ? 2 : 1) : 0;
    *status = m->impl->exchange_status();
    return LCR_OK;
  });
}

extern "C" int lcr_model_exchange_clear(lcr_model* m) {
  CAPI_MODEL(m);
  return capi::guarded([&]() -> int {
    m->impl->clear_exchange();
    return LCR_OK;
  });
}

extern "C" int lcr_model_prefill(lcr_model* m, const int32_t* tokens, int count,
                                 const float** logits) {
  CAPI_MODEL(m);
  CAPI_CHECK(count >= 0 && (count == 0 || tokens != nullptr), "prefill needs a token array");
  return capi::guarded([&]() -> int {
    std::vector<int> ids(tokens, tokens + count);
    const float* l = M(m).prefill(ids);
    if (logits) *logits = l;
    return LCR_OK;
  });
}

extern "C" int lcr_model_decode(lcr_model* m, int32_t token, const float** logits) {
  CAPI_MODEL(m);
  return capi::guarded([&]() -> int {
    const float* l = M(m).decode(token);
    if (logits) *logits = l;
    return LCR_OK;
  });
}

extern "C" int lcr_model_sample(lcr_model* m, const float* logits, float temperature, int top_k,
                                float top_p, float uniform, int32_t* out_id) {
  CAPI_MODEL(m);
  CAPI_CHECK(out_id != nullptr, "sample needs an output id");
  return capi::guarded([&]() -> int {
    *out_id = M(m).sample(logits, temperature, top_k, top_p, uniform);
    return LCR_OK;
  });
}

extern "C" int lcr_model_logits_to_host(lcr_model* m, const float* logits, float* out) {
  CAPI_MODEL(m);
  CAPI_CHECK(logits != nullptr && out != nullptr, "logits_to_host needs both pointers");
  return capi::guarded([&]() -> int {
    const std::vector<float> host = M(m).logits_to_host(logits);
    std::memcpy(out, host.data(), host.size() * sizeof(float));
    return LCR_OK;
  });
}

extern "C" int lcr_model_reset(lcr_model* m) {
  CAPI_MODEL(m);
  M(m).reset();
  return LCR_OK;
}

extern "C" int lcr_model_position(const lcr_model* m) {
  if (m == nullptr || !m->impl) return -1;
  return M(m).position();
}

extern "C" int lcr_model_stats_get(const lcr_model* m, lcr_model_stats* out) {
  CAPI_MODEL(m);
  CAPI_CHECK(out != nullptr, "stats needs an output struct");
  const Model& model = M(m);
  out->weight_bytes_per_token = model.stats().weight_bytes_per_token;
  out->kv_bytes_per_position = model.stats().kv_bytes_per_position;
  out->last_prefill_ms = model.stats().last_prefill_ms;
  out->last_decode_ms = model.stats().last_decode_ms;
  out->weight_bytes = model.weight_bytes();
  out->arena_peak_bytes = model.arena().peak();
  out->kv_allocated_bytes = model.kv_cache().allocated_bytes();
  out->multiprocessors = model.multiprocessors();
  out->fused = model.fused() ? 1 : 0;
  out->vocab_size = model.config().vocab_size;
  out->hidden_size = model.config().hidden_size;
  out->num_layers = model.config().num_layers;
  out->layer_grid = model.layer_grid() ? 1 : 0;
  return LCR_OK;
}

extern "C" int lcr_model_set_capture_activations(lcr_model* m, int enabled) {
  CAPI_MODEL(m);
  M(m).set_capture_activations(enabled != 0);
  return LCR_OK;
}

extern "C" int lcr_model_tap_count(const lcr_model* m) {
  if (m == nullptr || !m->impl) return -1;
  return static_cast<int>(M(m).activation_taps().size());
}

extern "C" int lcr_model_tap(const lcr_model* m, int index, char* name, size_t name_capacity,
                             int* tokens, int* width, float* values, size_t capacity) {
  CAPI_MODEL(m);
  const auto& taps = M(m).activation_taps();
  CAPI_CHECK(index >= 0 && static_cast<size_t>(index) < taps.size(),
             "tap index " << index << " out of range (" << taps.size() << " taps)");
  const Model::Tap& t = taps[static_cast<size_t>(index)];
  if (name != nullptr && name_capacity > 0) {
    const size_t n = std::min(name_capacity - 1, t.name.size());
    std::memcpy(name, t.name.data(), n);
    name[n] = '\0';
  }
  if (tokens) *tokens = t.tokens;
  if (width) *width = t.width;
  if (values != nullptr) {
    const size_t n = std::min(capacity, t.values.size());
    std::memcpy(values, t.values.data(), n * sizeof(float));
  }
  return LCR_OK;
}

extern "C" int lcr_model_set_profiling(lcr_model* m, int enabled) {
  CAPI_MODEL(m);
  M(m).profiler().set_enabled(enabled != 0);
  return LCR_OK;
}

extern "C" int lcr_model_generate_greedy(lcr_model* m, int32_t first_token, int steps,
                                         int32_t* out_tokens, double* elapsed_ms) {
  CAPI_MODEL(m);
  CAPI_CHECK(steps >= 0 && (steps == 0 || out_tokens != nullptr), "generate needs an output array");
  return capi::guarded([&]() -> int {
    const std::vector<int> ids = M(m).generate_greedy(first_token, steps, elapsed_ms);
    for (int i = 0; i < steps; ++i) out_tokens[i] = ids[static_cast<size_t>(i)];
    return LCR_OK;
  });
}

extern "C" int lcr_model_generate_sampled(lcr_model* m, int32_t first_token, int steps, float temperature,
                                          int top_k, float top_p, const float* uniforms, int32_t* out_tokens,
                                          double* elapsed_ms) {
  CAPI_MODEL(m);
  CAPI_CHECK(steps >= 0 && (steps == 0 || (out_tokens != nullptr && uniforms != nullptr)),
             "sampled generation needs one draw per step and an output array");
  return capi::guarded([&]() -> int {
    const std::vector<int> ids =
        M(m).generate_sampled(first_token, steps, temperature, top_k, top_p, uniforms, elapsed_ms);
    for (int i = 0; i < steps; ++i) out_tokens[i] = ids[static_cast<size_t>(i)];
    return LCR_OK;
  });
}

extern "C" int lcr_model_time_decode_kernel(lcr_model* m, const char* kernel, int launches,
                                            double* avg_ms, double* bytes_per_launch) {
  CAPI_MODEL(m);
  CAPI_CHECK(kernel != nullptr && avg_ms != nullptr, "kernel name and output needed");
  return capi::guarded([&]() -> int {
    *avg_ms = M(m).time_decode_kernel(kernel, launches, bytes_per_launch);
    return LCR_OK;
  });
}

extern "C" int lcr_model_decode_splits(const lcr_model* m, int seq_len) {
  if (m == nullptr || !m->impl) return -1;
  return M(m).decode_splits(seq_len);
}

extern "C" int lcr_model_kv_geometry(const lcr_model* m, int* max_pages, int* pool_pages,
                                     int* page_size, int* length) {
  CAPI_MODEL(m);
  const KvCache& kv = M(m).kv_cache();
  if (max_pages) *max_pages = kv.max_pages();
  if (pool_pages) *pool_pages = kv.pool_pages();
  if (page_size) *page_size = kv.page_size();
  if (length) *length = kv.length();
  return LCR_OK;
}

extern "C" int lcr_model_kv_page_table(const lcr_model* m, int layer, int32_t* out, int capacity) {
  CAPI_MODEL(m);
  const KvCache& kv = M(m).kv_cache();
  CAPI_CHECK(kv.layout() == KvLayout::kPaged, "the cache is contiguous; it has no page table");
  CAPI_CHECK(layer >= 0 && layer < M(m).config().num_layers, "layer " << layer << " out of range");
  CAPI_CHECK(out != nullptr && capacity >= kv.max_pages(), "page table output too small");
  return capi::guarded([&]() -> int {
    const KvCacheView v = kv.view(layer);
    HIP_CHECK(hipMemcpy(out, v.page_table, static_cast<size_t>(kv.max_pages()) * sizeof(int32_t),
                        hipMemcpyDeviceToHost));
    return LCR_OK;
  });
}

extern "C" int lcr_model_set_kv_page_tables(lcr_model* m, const int32_t* tables, size_t count,
                                            int length) {
  CAPI_MODEL(m);
  CAPI_CHECK(tables != nullptr, "page tables needed");
  return capi::guarded([&]() -> int {
    M(m).mutable_kv_cache().set_page_tables(std::vector<int32_t>(tables, tables + count), length);
    return LCR_OK;
  });
}

extern "C" int lcr_model_fill_kv_normal(lcr_model* m, uint64_t seed, float stddev) {
  CAPI_MODEL(m);
  return capi::guarded([&]() -> int {
    M(m).fill_kv_normal(seed, stddev);
    return LCR_OK;
  });
}

extern "C" int lcr_model_set_position(lcr_model* m, int position) {
  CAPI_MODEL(m);
  return capi::guarded([&]() -> int {
    M(m).set_position(position);
    return LCR_OK;
  });
}

extern "C" int lcr_model_kv_read(const lcr_model* m, int layer, int head, int position,
                                 void* key_out, void* value_out) {
  CAPI_MODEL(m);
  const KvCache& kv = M(m).kv_cache();
  const ModelConfig& c = M(m).config();
  CAPI_CHECK(layer >= 0 && layer < c.num_layers, "layer " << layer << " out of range");
  CAPI_CHECK(head >= 0 && head < c.num_kv_heads, "kv head " << head << " out of range");
  CAPI_CHECK(position >= 0 && position < kv.length(),
             "position " << position << " is not in the cache (length " << kv.length() << ")");
  return capi::guarded([&]() -> int {
    const KvCacheView v = kv.view(layer);
    size_t offset;
    if (kv.layout() == KvLayout::kPaged) {
      int32_t page = 0;
      HIP_CHECK(hipMemcpy(&page, v.page_table + position / v.page_size, sizeof(int32_t),
                          hipMemcpyDeviceToHost));
      offset = static_cast<size_t>(page) * v.page_stride + static_cast<size_t>(head) * v.head_stride +
               static_cast<size_t>(position % v.page_size) * v.head_dim;
    } else {
      offset = v.offset<false>(head, position);
    }
    const size_t bytes = static_cast<size_t>(v.head_dim) * sizeof(elem_t);
    if (key_out) HIP_CHECK(hipMemcpy(key_out, v.keys + offset, bytes, hipMemcpyDeviceToHost));
    if (value_out) HIP_CHECK(hipMemcpy(value_out, v.values + offset, bytes, hipMemcpyDeviceToHost));
    return LCR_OK;
  });
}

extern "C" int lcr_model_kv_export(const lcr_model* m, int layer, int positions, void* keys_out,
                                   void* values_out) {
  CAPI_MODEL(m);
  const KvCache& kv = M(m).kv_cache();
  const ModelConfig& c = M(m).config();
  CAPI_CHECK(layer >= 0 && layer < c.num_layers, "layer " << layer << " out of range");
  CAPI_CHECK(positions >= 0 && positions <= kv.length(),
             "positions " << positions << " exceeds the cache length " << kv.length());
  CAPI_CHECK(keys_out != nullptr && values_out != nullptr, "output buffers needed");
  return capi::guarded([&]() -> int {
    const KvCacheView v = kv.view(layer);
    const int heads = c.num_kv_heads;
    const size_t hd = static_cast<size_t>(v.head_dim);
    auto* ko = static_cast<elem_t*>(keys_out);
    auto* vo = static_cast<elem_t*>(values_out);
    if (kv.layout() != KvLayout::kPaged) {
      for (int h = 0; h < heads; ++h) {
        const size_t bytes = static_cast<size_t>(positions) * hd * sizeof(elem_t);
        HIP_CHECK(hipMemcpy(ko + h * positions * hd, v.keys + static_cast<size_t>(h) * v.head_stride, bytes,
                            hipMemcpyDeviceToHost));
        HIP_CHECK(hipMemcpy(vo + h * positions * hd, v.values + static_cast<size_t>(h) * v.head_stride, bytes,
                            hipMemcpyDeviceToHost));
      }
      return LCR_OK;
    }
    std::vector<int32_t> table(static_cast<size_t>(kv.max_pages()));
    HIP_CHECK(hipMemcpy(table.data(), v.page_table, table.size() * sizeof(int32_t), hipMemcpyDeviceToHost));
    std::vector<elem_t> kpage(static_cast<size_t>(v.page_stride)), vpage(static_cast<size_t>(v.page_stride));
    for (int p = 0; p * v.page_size < positions; ++p) {
      const size_t phys = static_cast<size_t>(table[static_cast<size_t>(p)]);
      HIP_CHECK(hipMemcpy(kpage.data(), v.keys + phys * v.page_stride, kpage.size() * sizeof(elem_t),
                          hipMemcpyDeviceToHost));
      HIP_CHECK(hipMemcpy(vpage.data(), v.values + phys * v.page_stride, vpage.size() * sizeof(elem_t),
                          hipMemcpyDeviceToHost));
      const int n = std::min(v.page_size, positions - p * v.page_size);
      for (int h = 0; h < heads; ++h) {
        const size_t dst = (static_cast<size_t>(h) * positions + static_cast<size_t>(p) * v.page_size) * hd;
        const size_t src = static_cast<size_t>(h) * v.head_stride;
        std::memcpy(ko + dst, kpage.data() + src, static_cast<size_t>(n) * hd * sizeof(elem_t));
        std::memcpy(vo + dst, vpage.data() + src, static_cast<size_t>(n) * hd * sizeof(elem_t));
      }
    }
    return LCR_OK;
  });
}

extern "C" int lcr_device_count(void) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return 0;
  return count;
}
