/*
 * lcr_model.h — C-ABI of the model (token loop) of the MI355X build.
 *
 * Wraps lcr::Model, whose C++ interface is the reference's src/model.h:60-127
 * (Model(dir, Options), prefill, decode, sample, logits_to_host, reset,
 * position, stats, activation taps). The C functions exist so hosts without
 * C++ (Python ctypes in this repository's tests and benchmark, or a Go/Java
 * binding) can drive the same object. Return values follow lcr_kernels.h:
 * 0 = ok, LCR_ERR_ARGUMENT with lcr_last_error_message() set otherwise.
 *
 * Additions beyond the reference are marked "extension".
 */
#ifndef LCR_MODEL_H_
#define LCR_MODEL_H_

#include <stddef.h>
#include <stdint.h>

#include "lcr_kernels.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct lcr_model lcr_model;

/* Model::Options (src/model.h:62-76) plus extensions. */
typedef struct lcr_model_options {
  int device;
  int max_seq;
  int paged;            /* KvLayout::kPaged when non-zero */
  int page_size;
  int prefill_chunk;    /* tokens per prefill pass (default 2048; the reference's is 256) */
  int attention_splits; /* 0 = choose from sequence length and CU count */
  int fused_decode;     /* extension: fused decode kernels (default 1) */
  int use_graph;        /* extension: replay the decode step from a hipGraph (default 1) */
  int prefill_via_decode; /* extension: prompts run token by token (default 0) */
  int decode_exchange;  /* extension: q/k/v projection and single-split attention of the
                           decode step in one grid, exchanging the query and the new key
                           and value in-grid (default 1; used when the device holds the grid) */
  int exchange_oproj;   /* extension: the o_proj projection joins that grid too (default 1) */
  int exchange_split;   /* extension: split attention (long contexts) runs as two such grids:
                           q/k/v + attention, and the split merge + o_proj (default 1) */
  int exchange_spins;   /* extension: polls before an exchange wait gives up (default 1 << 20) */
  int exchange_test_unwritten; /* tests only: exchange waits read words no block writes (default 0) */
  int layer_grid;       /* extension: with one attention split, each layer as one grid that
                           streams the o_proj and gate/up weights while the q/k/v -> attention
                           -> o_proj chain runs (default 0: slower than the three kernels it
                           replaces on MI355X; used when asked and the device holds the grid) */
  int exchange_head;    /* extension: the greedy step's argmax runs in the output head's grid,
                           its blocks' maxima exchanged in-grid, instead of in a one-block
                           kernel after it (default 1; used with the one-split exchange grid) */
} lcr_model_options;

/* ForwardStats (src/model.h:46-58) plus sizes. */
typedef struct lcr_model_stats {
  uint64_t weight_bytes_per_token;
  uint64_t kv_bytes_per_position;
  double last_prefill_ms;
  double last_decode_ms;
  uint64_t weight_bytes;
  uint64_t arena_peak_bytes;
  uint64_t kv_allocated_bytes;
  int multiprocessors;
  int fused;
  int vocab_size;
  int hidden_size;
  int num_layers;
  int layer_grid;       /* 1 when single-split decode steps run the layer grid */
} lcr_model_stats;

void lcr_model_default_options(lcr_model_options* options);
int lcr_model_create(const char* model_dir, const lcr_model_options* options, lcr_model** out);
void lcr_model_destroy(lcr_model* model);

/* Model::prefill / decode: device logits [vocab] fp32, valid until the next call. */
int lcr_model_prefill(lcr_model* model, const int32_t* tokens, int count, const float** logits);
int lcr_model_decode(lcr_model* model, int32_t token, const float** logits);
/* Model::sample: temperature <= 0 is argmax; uniform in [0, 1). A greedy
 * sample of the logits the last lcr_model_decode returned reads the id the
 * decode step already computed (same key and ties), with no GPU work. */
int lcr_model_sample(lcr_model* model, const float* logits, float temperature, int top_k,
                     float top_p, float uniform, int32_t* out_id);
int lcr_model_logits_to_host(lcr_model* model, const float* logits, float* out);
int lcr_model_reset(lcr_model* model);
int lcr_model_position(const lcr_model* model);
int lcr_model_stats_get(const lcr_model* model, lcr_model_stats* out);

/* Activation taps (src/model.h:111-127): enable, then run a pass; taps are
 * "embed", "layer_0".."layer_{n-1}", "final_norm". */
int lcr_model_set_capture_activations(lcr_model* model, int enabled);
int lcr_model_tap_count(const lcr_model* model);
/* Copies tap `index`: its name (NUL-terminated, at most name_capacity bytes),
 * tokens, width, and min(capacity, tokens*width) floats into values. */
int lcr_model_tap(const lcr_model* model, int index, char* name, size_t name_capacity,
                  int* tokens, int* width, float* values, size_t capacity);

/* Per-stage profile of eager (unfused) passes (src/profiler.h). */
int lcr_model_set_profiling(lcr_model* model, int enabled);

/* extension: which exchange grid decode steps run (*enabled: 0 none, 1 q/k/v and attention,
 * 2 q/k/v, attention and o_proj), and whether an exchange wait of a past step gave up
 * (*status non-zero: those results are not valid). Synchronizes the model's stream. */
int lcr_model_exchange_status(const lcr_model* model, int* enabled, int* status);
/* extension: clears the exchange words and status (after a wait gave up). */
int lcr_model_exchange_clear(lcr_model* model);

/* extension: greedy generation kept on the device. Decodes first_token, then
 * feeds each argmax to the next step without a host round trip; writes the
 * `steps` generated ids and the elapsed GPU time of the loop. */
int lcr_model_generate_greedy(lcr_model* model, int32_t first_token, int steps,
                              int32_t* out_tokens, double* elapsed_ms);
/* extension: the reference's sampled host loop (src/main.cu:456-466: decode,
 * then Model::sample with the next draw) kept on the device. Decodes
 * first_token, samples with uniforms[0] (temperature > 0, top_k, top_p as
 * lcr_model_sample), feeds the id to the next step, ...: `steps` decodes,
 * the `steps` sampled ids written out, the same ids as decode + sample with
 * the same draws, and the elapsed GPU time of the loop. */
int lcr_model_generate_sampled(lcr_model* model, int32_t first_token, int steps, float temperature,
                               int top_k, float top_p, const float* uniforms, int32_t* out_tokens,
                               double* elapsed_ms);
/* extension: the split count decode uses at a sequence length. */
int lcr_model_decode_splits(const lcr_model* model, int seq_len);
/* extension: times one fused decode kernel in isolation ("qkv", "attention",
 * "o_proj", "gate_up", "down", "lm_head", "argmax": the reduction of the
 * head's per-block keys to the id alone in its own kernel, or "head": the
 * output head with the argmax as the decode step runs them) over `launches`
 * launches on the model's stream, each between its own pair of hipEvents, cycling through the
 * layers; returns the mean duration (ms) and the algorithmic bytes per launch.
 * Call after a prefill or decode. The kernels write their usual outputs (the
 * qkv kernel rewrites the cache at the last position), so the sequence is not
 * meant to be continued afterwards: reset or prefill again. */
int lcr_model_time_decode_kernel(lcr_model* model, const char* kernel, int launches,
                                 double* avg_ms, double* bytes_per_launch);

/* extension, KV cache test hooks (long-context stress, page-index parity). */
int lcr_model_kv_page_table(const lcr_model* model, int layer, int32_t* out, int capacity);
int lcr_model_kv_geometry(const lcr_model* model, int* max_pages, int* pool_pages,
                          int* page_size, int* length);
int lcr_model_set_kv_page_tables(lcr_model* model, const int32_t* tables, size_t count,
                                 int length);
int lcr_model_fill_kv_normal(lcr_model* model, uint64_t seed, float stddev);
int lcr_model_set_position(lcr_model* model, int position);
/* Copies the cached key and value vectors (head_dim elements each) of
 * (layer, kv head, position). */
int lcr_model_kv_read(const lcr_model* model, int layer, int head, int position, void* key_out,
                      void* value_out);
/* Copies positions [0, positions) of every kv head of a layer, in logical
 * order: out[head][position][head_dim] elements, whatever the layout (paged
 * caches are gathered page by page through the page table). */
int lcr_model_kv_export(const lcr_model* model, int layer, int positions, void* keys_out,
                        void* values_out);

/* extension: seeded random-init checkpoint (config.json + model.safetensors)
 * and seeded prompt ids; see llama-cuda-runtime_amd/csrc/synth.cpp. */
int lcr_write_synthetic_checkpoint(const char* dir, const char* config_json, uint64_t seed,
                                   float stddev, int fp16, int threads);
int lcr_synthetic_tokens(uint64_t seed, int count, int vocab, int32_t* out);
/* extension: `count` draws of the Philox4x32-10 uniform stream of `seed` (the
 * sampling draws of llama-run and of the sampling tests); see
 * llama-cuda-runtime_amd/csrc/philox.h. */
int lcr_philox_uniforms(uint64_t seed, int count, float* out);

/* Number of visible HIP devices (0 without a GPU; never an error). */
int lcr_device_count(void);

#ifdef __cplusplus
}
#endif

#endif /* LCR_MODEL_H_ */
