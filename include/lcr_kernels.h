/*
 * lcr_kernels.h — C-ABI kernel layer of the MI355X (gfx950) token loop.
 *
 * Replaces the reference's C++ kernel header src/kernels.cuh:14-134 and the
 * cuBLAS call sites in src/model.cu:38-45 and :537-556. Every launcher of the
 * reference has a counterpart here with the same argument meaning, order and
 * early-return-on-empty behaviour; the reference's C++ names
 * (lcr::launch_*) are kept by the thin C++ wrapper in
 * llama-cuda-runtime_amd/csrc/kernels.h, which turns a non-zero status into
 * lcr::Error with the message below.
 *
 * Conventions
 *  - Element pointers (`void*` / `const void*`) point at 16-bit elements of the
 *    build's type: bf16 in liblcr_amd.so, fp16 in liblcr_amd_fp16.so (the
 *    reference's LCR_DTYPE switch, CMakeLists.txt:79-99). Pointers are device
 *    pointers; nothing here allocates, so every call is graph-capture safe.
 *  - `stream` is a hipStream_t passed as void*; NULL is the default stream.
 *  - Return value: 0 on success; LCR_ERR_ARGUMENT (-1) when an argument check
 *    fails (the same checks, with the same message text, as the reference's
 *    LCR_CHECKs); otherwise the positive hipError_t of a failed HIP call.
 *    lcr_last_error_message() returns the calling thread's last message.
 *  - With LCR_SYNC_KERNELS=1 in the environment every launch is followed by a
 *    device synchronize (src/cuda_utils.cuh:41-49).
 */
#ifndef LCR_KERNELS_H_
#define LCR_KERNELS_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LCR_OK 0
#define LCR_ERR_ARGUMENT (-1)

/* Plain-old-data view of one layer of the KV cache, field for field the
 * reference's KvCacheView (src/kv_cache.cuh:33-46). Element (head, position,
 * d) lives at
 *   page * page_stride + head * head_stride + slot * head_dim + d
 * with page = page_table[position / page_size], slot = position % page_size
 * when paged, and page = 0, slot = position when contiguous
 * (src/kv_cache.cuh:49-56). */
typedef struct lcr_kv_view {
  void* keys;
  void* values;
  const int32_t* page_table;
  int page_size;
  int page_stride;
  int head_stride;
  int num_kv_heads;
  int head_dim;
} lcr_kv_view;

/* Message of the last failed call on this thread ("" if none). */
const char* lcr_last_error_message(void);
/* "bf16" or "fp16": the element type this library was built for. */
const char* lcr_elem_name(void);

/* out[t,:] = table[ids[t],:] — src/kernels.cuh:17-19 */
int lcr_embedding_lookup(void* out, const void* table, const int32_t* ids, int tokens,
                         int dim, void* stream);

/* out[t] = bf16(x[t] * (1/sqrt(mean(x[t]^2) + eps)) * weight) — src/kernels.cuh:24-25 */
int lcr_rmsnorm(void* out, const void* x, const void* weight, int tokens, int dim, float eps,
                void* stream);

/* x += delta elementwise — src/kernels.cuh:28-29 */
int lcr_add_residual(void* x, const void* delta, int64_t count, void* stream);

/* x = bf16(x + delta); out = rmsnorm(x) * weight, the sum of squares taken over
 * the unrounded x + delta — src/kernels.cuh:39-41 */
int lcr_add_residual_rmsnorm(void* out, void* x, const void* delta, const void* weight,
                             int tokens, int dim, float eps, void* stream);

/* out = silu(gate) * up — src/kernels.cuh:44-45 */
int lcr_swiglu(void* out, const void* gate, const void* up, int64_t count, void* stream);

/* Same with gate/up read from rows of stride src_row_stride — src/kernels.cuh:49-51 */
int lcr_swiglu_strided(void* out, const void* gate, const void* up, int tokens, int width,
                       int src_row_stride, void* stream);

/* Half-split RoPE of Q and transpose to [num_heads][tokens][head_dim] —
 * src/kernels.cuh:62-64 */
int lcr_rope_q(void* q_heads, const void* q_proj, const float* inv_freq, int tokens,
               int start_position, int num_heads, int head_dim, int src_row_stride,
               void* stream);

/* RoPE of K, copy of V, both written into the cache at view offsets —
 * src/kernels.cuh:69-72 */
int lcr_rope_write_kv(const lcr_kv_view* view, const void* k_proj, const void* v_proj,
                      const float* inv_freq, int tokens, int start_position, int paged,
                      int src_row_stride, void* stream);

/* fp32 causal softmax of prefill scores into 16-bit probabilities; masked
 * entries are written as exactly 0 — src/kernels.cuh:79-81 */
int lcr_causal_softmax(void* probs, const float* scores, int num_heads, int rows, int keys,
                       int start_position, void* stream);

/* [num_heads][tokens][head_dim] -> [tokens][num_heads*head_dim] — src/kernels.cuh:85-86 */
int lcr_merge_heads(void* out, const void* heads, int tokens, int num_heads, int head_dim,
                    void* stream);

/* Paged cache -> contiguous [num_kv_heads][positions][head_dim] — src/kernels.cuh:92-94 */
int lcr_gather_kv(void* out_keys, void* out_values, const lcr_kv_view* view, int positions,
                  void* stream);

/* Single-query GQA attention over seq_len cached positions, split-K over
 * `splits` blocks per kv head with a merge pass — src/kernels.cuh:106-110.
 * head_dim in {64, 128}, heads_per_kv in {1, 2, 4, 8}. */
int lcr_decode_attention(void* out, const void* q, const lcr_kv_view* view, int num_heads,
                         int heads_per_kv, int seq_len, float scale, int paged, int splits,
                         float* scratch, void* stream);

/* Largest partials buffer lcr_decode_attention_noalloc holds: 2 MiB of floats
 * (32 heads x 64 splits x (2 + 128) = 266,240 floats fit). */
#define LCR_NOALLOC_ATTENTION_SCRATCH_FLOATS (524288)

/* lcr_decode_attention without a scratch argument and without allocating: the
 * split partials go to a fixed device array of the library
 * (LCR_NOALLOC_ATTENTION_SCRATCH_FLOATS floats, one per device, held until the
 * process ends). No counterpart in the reference; it is for callers that cannot
 * allocate (code under graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). Arguments and results are those of lcr_decode_attention;
 * a call whose partials would exceed the array fails with LCR_ERR_ARGUMENT.
 * Every call on a device shares that device's array (nothing in it needs to
 * start at zero: each split writes all of its partials before the merge reads
 * them), so calls that overlap in time on one device race. */
int lcr_decode_attention_noalloc(void* out, const void* q, const lcr_kv_view* view, int num_heads,
                                 int heads_per_kv, int seq_len, float scale, int paged, int splits,
                                 void* stream);

/* Floats of scratch lcr_decode_attention needs (0 when splits <= 1) —
 * src/kernels.cuh:114 */
size_t lcr_decode_attention_scratch_floats(int num_heads, int head_dim, int splits);

/* Split count heuristic — src/kernels.cuh:118, src/kernels/attention.cu:419-431 */
int lcr_choose_attention_splits(int num_kv_heads, int seq_len, int multiprocessors);

/* Next token id: argmax when temperature <= 0, else temperature / top-k /
 * top-p sampling with the host-drawn uniform — src/kernels.cuh:128-130 */
int lcr_sample(int32_t* out_id, const float* logits, int vocab, float temperature, int top_k,
               float top_p, float uniform, float* scratch, void* stream);

/* Floats of scratch lcr_sample needs — src/kernels.cuh:132 */
size_t lcr_sample_scratch_floats(int vocab, int top_k);

/* ---- projections (the reference calls cuBLAS for these) ------------------ */

/* y[n] = sum_k W[n][k] * x[k], W row-major [N][K] 16-bit, fp32 accumulation,
 * y 16-bit (y_fp32 == 0) or fp32 (y_fp32 != 0). K % 8 == 0. Replaces
 * gemm_nt(..., rows = 1, ...) → cublasGemmEx(OP_T, OP_N), src/model.cu:38-45,
 * called at :393, :420, :431, :441 and (fp32 out) :481. */
int lcr_gemv(void* y, int y_fp32, const void* W, const void* x, int N, int K, void* stream);

/* Y[t][n] = sum_k X[t][k] * W[n][k] for t < T (the same gemm_nt at rows = T,
 * src/model.cu:38-45), on MFMA matrix cores, fp32 accumulation, 16-bit or
 * fp32 output. K % 8 == 0. */
int lcr_gemm(void* Y, int y_fp32, const void* X, const void* W, int T, int N, int K,
             void* stream);

/* lcr_gemm with a caller-provided device workspace (16-byte aligned): when the
 * output tiles alone would leave compute units idle, K is split into slices
 * whose fp32 partial products go to the workspace and are summed in slice
 * order by a second kernel. A workspace smaller than the preferred split needs
 * gives a plan that fits (down to no split). No counterpart in the reference,
 * which hands this choice to cuBLAS and its internal workspace
 * (src/model.cu:38-45). */
int lcr_gemm_ws(void* Y, int y_fp32, const void* X, const void* W, int T, int N, int K,
                void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes lcr_gemm_ws uses for its preferred plan at this shape on the
 * current device (0: no split). */
size_t lcr_gemm_workspace_bytes(int T, int N, int K);

/* act[t][f] = rne(silu(g) * u) with g, u the 16-bit-rounded outputs of the
 * fused gate/up projection W_gate_up[2 ffn][K] (gate rows first, as the
 * reference fuses them, src/model.cu:165-172): the gate/up GEMM of
 * src/model.cu:441 and launch_swiglu_strided (src/kernels.cuh:40) in one
 * kernel, bit-identical to the pair. ffn % 16 == 0; workspace as for
 * lcr_gemm_ws with N = 2 ffn. */
int lcr_gemm_swiglu_ws(void* act, const void* X, const void* W_gate_up, int T, int ffn, int K,
                       void* workspace, size_t workspace_bytes, void* stream);

/* A projection followed by the residual join and RMSNorm that always follows
 * it: o_proj (src/model.cu:420-427) or the MLP down projection and the next
 * layer's input norm (src/model.cu:441-458), i.e. lcr_gemm_ws into delta
 * [T][N] and lcr_add_residual_rmsnorm(out, x, delta, weight) (src/kernels.cuh:39),
 * bit-identical to that pair. When the plan splits K, the norm's row pass
 * sums the slices itself and delta is left unwritten; otherwise delta holds
 * the projection. Workspace as for lcr_gemm_ws. */
int lcr_gemm_residual_rmsnorm_ws(void* out, void* x, void* delta, const void* X, const void* W,
                                 const void* weight, int T, int N, int K, float eps, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* table[p * (head_dim / 2) + i] = (cos a, sin a) for a = float(p) * inv_freq[i]
 * and p < positions: the per-position angles lcr_rope_q and lcr_rope_write_kv
 * evaluate (src/kernels/rope.cu:33-87), the same values, tabulated once. The
 * table is positions * head_dim / 2 pairs of floats. */
int lcr_rope_table(float* table, const float* inv_freq, int positions, int head_dim, void* stream);

/* The fused q/k/v projection of src/model.cu:393 followed by launch_rope_q and
 * launch_rope_write_kv (src/model.cu:396-406, src/kernels.cuh:62-72) in one
 * pass, bit-identical to lcr_gemm_ws into a [T][N] buffer and those two
 * kernels reading it: each output is rounded to the element type, queries
 * are rotated into q_heads [num_heads][T][head_dim], keys rotated and values
 * copied into the cache through the view at positions start_position + t.
 * W_qkv holds the num_heads query heads, then the view's num_kv_heads key and
 * value heads, head_dim rows each (N = (num_heads + 2 num_kv_heads) head_dim).
 * rope_table comes from lcr_rope_table and covers positions up to
 * start_position + T. head_dim is 64 or 128; workspace as for lcr_gemm_ws. */
int lcr_gemm_qkv_rope_ws(void* q_heads, const lcr_kv_view* view, const void* X, const void* W_qkv,
                         const float* rope_table, int T, int num_heads, int K, int start_position,
                         int paged, void* workspace, size_t workspace_bytes, void* stream);

/* Causal GQA attention for a prefill chunk: the two strided-batched GEMMs and
 * the softmax of src/model.cu:509-560 (K13 gather + G6 + K10 + G7 + K7) in
 * one flash-style pass reading the cache through the view.
 *   q_heads: [num_heads][tokens][head_dim] (RoPE applied), query row r sits at
 *            position start_position + r and sees keys 0 .. start_position + r.
 *   out:     [tokens][num_heads * head_dim]
 * Probabilities are rounded to the element type before the value product, as
 * the reference's bf16 probs buffer does. */
int lcr_prefill_attention(void* out, const void* q_heads, const lcr_kv_view* view,
                          int num_heads, int heads_per_kv, int tokens, int start_position,
                          float scale, int paged, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LCR_KERNELS_H_ */
