// C++ face of the kernel layer: the reference's src/kernels.cuh:14-134
// signatures, namespace and semantics (hipStream_t in place of cudaStream_t),
// implemented over the C-ABI in include/lcr_kernels.h. A non-zero status
// becomes lcr::Error carrying the C layer's message, so code written against
// the reference (its Model, its kernel tests' CHECK_THROWS) runs unchanged.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/lcr_kernels.h"
#include "dtype.h"
#include "kv_cache.h"

namespace lcr {

inline void check_kernel_status(int status) {
  if (status != LCR_OK) throw Error(lcr_last_error_message());
}

inline void launch_embedding_lookup(elem_t* out, const elem_t* table, const int32_t* ids,
                                    int tokens, int dim, hipStream_t stream) {
  check_kernel_status(lcr_embedding_lookup(out, table, ids, tokens, dim, stream));
}

inline void launch_rmsnorm(elem_t* out, const elem_t* x, const elem_t* weight, int tokens,
                           int dim, float eps, hipStream_t stream) {
  check_kernel_status(lcr_rmsnorm(out, x, weight, tokens, dim, eps, stream));
}

inline void launch_add_residual(elem_t* x, const elem_t* delta, int64_t count, hipStream_t stream) {
  check_kernel_status(lcr_add_residual(x, delta, count, stream));
}

inline void launch_add_residual_rmsnorm(elem_t* out, elem_t* x, const elem_t* delta,
                                        const elem_t* weight, int tokens, int dim, float eps,
                                        hipStream_t stream) {
  check_kernel_status(lcr_add_residual_rmsnorm(out, x, delta, weight, tokens, dim, eps, stream));
}

inline void launch_swiglu(elem_t* out, const elem_t* gate, const elem_t* up, int64_t count,
                          hipStream_t stream) {
  check_kernel_status(lcr_swiglu(out, gate, up, count, stream));
}

inline void launch_swiglu_strided(elem_t* out, const elem_t* gate, const elem_t* up, int tokens,
                                  int width, int src_row_stride, hipStream_t stream) {
  check_kernel_status(lcr_swiglu_strided(out, gate, up, tokens, width, src_row_stride, stream));
}

inline void launch_rope_q(elem_t* q_heads, const elem_t* q_proj, const float* inv_freq,
                          int tokens, int start_position, int num_heads, int head_dim,
                          int src_row_stride, hipStream_t stream) {
  check_kernel_status(lcr_rope_q(q_heads, q_proj, inv_freq, tokens, start_position, num_heads,
                                 head_dim, src_row_stride, stream));
}

inline void launch_rope_write_kv(const KvCacheView& view, const elem_t* k_proj,
                                 const elem_t* v_proj, const float* inv_freq, int tokens,
                                 int start_position, bool paged, int src_row_stride,
                                 hipStream_t stream) {
  const lcr_kv_view v = view.to_c();
  check_kernel_status(lcr_rope_write_kv(&v, k_proj, v_proj, inv_freq, tokens, start_position,
                                        paged ? 1 : 0, src_row_stride, stream));
}

inline void launch_causal_softmax(elem_t* probs, const float* scores, int num_heads, int rows,
                                  int keys, int start_position, hipStream_t stream) {
  check_kernel_status(lcr_causal_softmax(probs, scores, num_heads, rows, keys, start_position, stream));
}

inline void launch_merge_heads(elem_t* out, const elem_t* heads, int tokens, int num_heads,
                               int head_dim, hipStream_t stream) {
  check_kernel_status(lcr_merge_heads(out, heads, tokens, num_heads, head_dim, stream));
}

inline void launch_gather_kv(elem_t* out_keys, elem_t* out_values, const KvCacheView& view,
                             int positions, hipStream_t stream) {
  const lcr_kv_view v = view.to_c();
  check_kernel_status(lcr_gather_kv(out_keys, out_values, &v, positions, stream));
}

inline void launch_decode_attention(elem_t* out, const elem_t* q, const KvCacheView& view,
                                    int num_heads, int heads_per_kv, int seq_len, float scale,
                                    bool paged, int splits, float* scratch, hipStream_t stream) {
  const lcr_kv_view v = view.to_c();
  check_kernel_status(lcr_decode_attention(out, q, &v, num_heads, heads_per_kv, seq_len, scale,
                                           paged ? 1 : 0, splits, scratch, stream));
}

inline size_t decode_attention_scratch_floats(int num_heads, int head_dim, int splits) {
  return lcr_decode_attention_scratch_floats(num_heads, head_dim, splits);
}

inline int choose_attention_splits(int num_kv_heads, int seq_len, int multiprocessors) {
  return lcr_choose_attention_splits(num_kv_heads, seq_len, multiprocessors);
}

inline void launch_sample(int32_t* out_id, const float* logits, int vocab, float temperature,
                          int top_k, float top_p, float uniform, float* scratch,
                          hipStream_t stream) {
  check_kernel_status(
      lcr_sample(out_id, logits, vocab, temperature, top_k, top_p, uniform, scratch, stream));
}

inline size_t sample_scratch_floats(int vocab, int top_k) {
  return lcr_sample_scratch_floats(vocab, top_k);
}

// The projections the reference sends to cuBLAS (src/model.cu:38-45).
inline void launch_gemv(void* y, bool y_fp32, const elem_t* W, const elem_t* x, int N, int K,
                        hipStream_t stream) {
  check_kernel_status(lcr_gemv(y, y_fp32 ? 1 : 0, W, x, N, K, stream));
}

inline void launch_gemm(void* Y, bool y_fp32, const elem_t* X, const elem_t* W, int T, int N,
                        int K, hipStream_t stream) {
  check_kernel_status(lcr_gemm(Y, y_fp32 ? 1 : 0, X, W, T, N, K, stream));
}

inline void launch_gemm(void* Y, bool y_fp32, const elem_t* X, const elem_t* W, int T, int N,
                        int K, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  check_kernel_status(lcr_gemm_ws(Y, y_fp32 ? 1 : 0, X, W, T, N, K, workspace, workspace_bytes, stream));
}

inline void launch_gemm_swiglu(elem_t* act, const elem_t* X, const elem_t* W_gate_up, int T, int ffn,
                               int K, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  check_kernel_status(lcr_gemm_swiglu_ws(act, X, W_gate_up, T, ffn, K, workspace, workspace_bytes, stream));
}

inline void launch_gemm_residual_rmsnorm(elem_t* out, elem_t* x, elem_t* delta, const elem_t* X, const elem_t* W,
                                         const elem_t* weight, int T, int N, int K, float eps, void* workspace,
                                         size_t workspace_bytes, hipStream_t stream) {
  check_kernel_status(
      lcr_gemm_residual_rmsnorm_ws(out, x, delta, X, W, weight, T, N, K, eps, workspace, workspace_bytes, stream));
}

inline void launch_gemm_qkv_rope(elem_t* q_heads, const KvCacheView& view, const elem_t* X, const elem_t* W_qkv,
                                 const float2* rope_table, int T, int num_heads, int K, int start_position,
                                 bool paged, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const lcr_kv_view v = view.to_c();
  check_kernel_status(lcr_gemm_qkv_rope_ws(q_heads, &v, X, W_qkv, reinterpret_cast<const float*>(rope_table), T,
                                           num_heads, K, start_position, paged ? 1 : 0, workspace,
                                           workspace_bytes, stream));
}

inline void launch_prefill_attention(elem_t* out, const elem_t* q_heads, const KvCacheView& view,
                                     int num_heads, int heads_per_kv, int tokens,
                                     int start_position, float scale, bool paged,
                                     hipStream_t stream) {
  const lcr_kv_view v = view.to_c();
  check_kernel_status(lcr_prefill_attention(out, q_heads, &v, num_heads, heads_per_kv, tokens,
                                            start_position, scale, paged ? 1 : 0, stream));
}

}  // namespace lcr
