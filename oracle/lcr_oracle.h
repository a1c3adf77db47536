/*
 * lcr_oracle.h — CPU oracle for the token loop. TEST INFRASTRUCTURE ONLY.
 *
 * A plain C++17 restatement, on the CPU, of every function on the reference's
 * decode / prefill / sampling path (mohamadmsalman82/llama-cuda-runtime,
 * src/model.cu:308-597 and the kernels under src/kernels/), used by tests/, by
 * __graft_entry__.smoke() and by bench.py's cpu_baseline leg as the checker.
 * Nothing in the shipped library links, loads or calls it.
 *
 * Element arrays are uint16_t words of the element type named by `kind`
 * (ORC_BF16 or ORC_FP16). Floating-point operations follow the same fixed
 * orders the HIP kernels document (GEMV blocks of 2048 with a 64-lane
 * butterfly, the RMSNorm block-reduction tree, the split-K attention
 * schedule, the sampler's sum tree), so decode-path results are expected to be
 * bit-identical to the GPU's; each function's comment cites the reference
 * file:line whose semantics it restates; lcr_oracle.cpp's header lists them.
 */
#ifndef LCR_ORACLE_H_
#define LCR_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_BF16 0
#define ORC_FP16 1

/* ---- scalar building blocks ------------------------------------------- */
float orc_elem_to_float(uint16_t bits, int kind);
uint16_t orc_float_to_elem(float value, int kind);
float orc_expf(float x);
void orc_sincosf(float angle, float* s, float* c);
void orc_rope_inv_freq(int head_dim, float theta, int llama3, float factor, float low_freq_factor,
                       float high_freq_factor, int original_context, float* out);

/* ---- kernels ------------------------------------------------------------ */
typedef struct orc_kv_view {
  uint16_t* keys;
  uint16_t* values;
  const int32_t* page_table;
  int page_size;
  int page_stride;
  int head_stride;
  int num_kv_heads;
  int head_dim;
} orc_kv_view;

int64_t orc_kv_offset(const orc_kv_view* view, int paged, int head, int position);

void orc_embedding_lookup(uint16_t* out, const uint16_t* table, const int32_t* ids, int tokens,
                          int dim);
void orc_rmsnorm(int kind, uint16_t* out, const uint16_t* x, const uint16_t* w, int tokens,
                 int dim, float eps);
void orc_add_residual_rmsnorm(int kind, uint16_t* out, uint16_t* x, const uint16_t* delta,
                              const uint16_t* w, int tokens, int dim, float eps);
void orc_add_residual(int kind, uint16_t* x, const uint16_t* delta, int64_t count);
void orc_swiglu(int kind, uint16_t* out, const uint16_t* gate, const uint16_t* up, int64_t count);
void orc_swiglu_strided(int kind, uint16_t* out, const uint16_t* gate, const uint16_t* up,
                        int tokens, int width, int src_row_stride);
void orc_merge_heads(uint16_t* out, const uint16_t* heads, int tokens, int num_heads,
                     int head_dim);
void orc_rope_q(int kind, uint16_t* q_heads, const uint16_t* q_proj, const float* inv_freq,
                int tokens, int start_position, int num_heads, int head_dim, int src_row_stride);
void orc_rope_write_kv(int kind, const orc_kv_view* view, const uint16_t* k_proj,
                       const uint16_t* v_proj, const float* inv_freq, int tokens,
                       int start_position, int paged, int src_row_stride);
void orc_gather_kv(uint16_t* out_keys, uint16_t* out_values, const orc_kv_view* view,
                   int positions);
int orc_choose_attention_splits(int num_kv_heads, int seq_len, int multiprocessors);
void orc_decode_attention(int kind, uint16_t* out, const uint16_t* q, const orc_kv_view* view,
                          int num_heads, int heads_per_kv, int seq_len, float scale, int paged,
                          int splits);
void orc_causal_softmax(int kind, uint16_t* probs, const float* scores, int num_heads, int rows,
                        int keys, int start_position);
void orc_prefill_attention(int kind, uint16_t* out, const uint16_t* q_heads,
                           const orc_kv_view* view, int num_heads, int heads_per_kv, int tokens,
                           int start_position, float scale, int paged);
/* y[n] = W[n,:] . x ; y is uint16_t elements (y_fp32 == 0) or float. */
void orc_gemv(int kind, void* y, int y_fp32, const uint16_t* W, const uint16_t* x, int N, int K);
/* Y[t][n] = X[t,:] . W[n,:] with the same per-element order as orc_gemv. */
void orc_gemm(int kind, void* Y, int y_fp32, const uint16_t* X, const uint16_t* W, int T, int N,
              int K);
int32_t orc_argmax(const float* logits, int vocab);
int32_t orc_sample(const float* logits, int vocab, float temperature, int top_k, float top_p,
                   float uniform);

/* ---- whole model -------------------------------------------------------- */
typedef struct orc_config {
  int hidden_size;
  int intermediate_size;
  int num_layers;
  int num_heads;
  int num_kv_heads;
  int head_dim;
  int vocab_size;
  float rms_norm_eps;
  float rope_theta;
  int rope_llama3;
  float rope_factor;
  float rope_low_freq_factor;
  float rope_high_freq_factor;
  int rope_original_context;
} orc_config;

/* Per-layer arrays have num_layers entries. lm_head may equal embed (tied). */
typedef struct orc_weights {
  const uint16_t* embed;
  const uint16_t* final_norm;
  const uint16_t* lm_head;
  const uint16_t* const* input_norm;
  const uint16_t* const* q_proj;
  const uint16_t* const* k_proj;
  const uint16_t* const* v_proj;
  const uint16_t* const* o_proj;
  const uint16_t* const* post_norm;
  const uint16_t* const* gate_proj;
  const uint16_t* const* up_proj;
  const uint16_t* const* down_proj;
} orc_weights;

typedef struct orc_model orc_model;

/* multiprocessors feeds the split heuristic (256 on MI355X); attention_splits
 * > 0 forces a split count, as Model::Options::attention_splits does. */
orc_model* orc_model_create(int kind, const orc_config* config, const orc_weights* weights,
                            int max_seq, int paged, int page_size, int prefill_chunk,
                            int multiprocessors, int attention_splits);
void orc_model_destroy(orc_model* model);
void orc_model_reset(orc_model* model);
int orc_model_position(const orc_model* model);
/* One token at the current position (src/model.cu:347-368); logits [vocab]. */
int orc_model_decode(orc_model* model, int token, float* logits);
/* A prompt at the current position (src/model.cu:308-345). use_decode_path
 * != 0 runs it as single-token decode steps instead of chunked prefill. */
int orc_model_prefill(orc_model* model, const int32_t* tokens, int count, int use_decode_path,
                      float* logits);
/* Residual stream taps of the last pass: "embed", one per layer, "final_norm"
 * (src/model.cu:486-503), each tokens x hidden floats of the last pass.
 * Returns the number of floats copied into out (capacity in floats). */
size_t orc_model_tap(const orc_model* model, int index, float* out, size_t capacity);
const int32_t* orc_model_page_table(const orc_model* model, int layer);
/* Split count of the whole-model decode step (both the HIP model and this
 * oracle use it): 1 below 4096 positions; below 16384 ceil(CUs / num_heads);
 * from 16384 ceil(CUs / num_kv_heads); at least 512 positions per split, at
 * most 64 splits. */
int orc_decode_step_splits(int num_heads, int num_kv_heads, int seq_len, int multiprocessors);
/* Test hooks: writes positions [0, positions) of a layer's cache from logical
 * [kv_head][position][head_dim] arrays; moves the position (the cache keeps
 * its content). */
int orc_model_set_kv(orc_model* model, int layer, int positions, const uint16_t* keys,
                     const uint16_t* values);
int orc_model_set_position(orc_model* model, int position);
const char* orc_last_error(void);
/* OpenMP threads the oracle's parallel loops use from now on (n >= 1), and
 * the current count. */
void orc_set_threads(int n);
int orc_threads(void);

#ifdef __cplusplus
}
#endif

#endif /* LCR_ORACLE_H_ */
