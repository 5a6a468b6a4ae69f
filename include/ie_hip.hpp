/* C++17 face of libie_hip.so for the engine: the reference's launcher names
 * and argument order (src/cuda/kernels.cuh:33-38,69-102), calling the C ABI of
 * ie_hip.h, with failures turned into std::runtime_error carrying the
 * library's message, as the reference's check() does (src/cuda/kernels.cu:18-23,
 * src/cuda/cuda_runner.cu:45-48). Header-only; nothing here launches work of
 * its own. */
#ifndef IE_HIP_HPP_
#define IE_HIP_HPP_

#include <stdexcept>
#include <string>

#include "ie_hip.h"

namespace ie::hip {

inline void check(int rc) {
  if (rc != IE_HIP_OK) throw std::runtime_error(ie_hip_last_error());
}

inline void check(hipError_t err, const char* what) {
  if (err != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(err));
}

constexpr int kPageSize = IE_HIP_PAGE_SIZE;

/* KvLayout{tables, max_pages, page_size, f16} (src/cuda/kernels.cuh:33-38): the
 * boolean f16 becomes a KV dtype (IE_KV_F32 / F16 / BF16) and the pool size is
 * added, so kernels skip page ids outside the pool. Passed by value. */
struct KvLayout {
  const int32_t* tables = nullptr;
  int max_pages = 0;
  int page_size = kPageSize;
  int kv_dtype = IE_KV_F32;
  int num_pages = 0;
  ie_kv_layout c() const { return ie_kv_layout{tables, max_pages, page_size, kv_dtype, num_pages}; }
};

inline int kv_elem_bytes(int kv_dtype) { return kv_dtype == IE_KV_F32 ? 4 : 2; }

/* rope_and_cache (kernels.cuh:69-74) with the host-built cos/sin table in
 * place of inv_freq: [table_positions, head_dim] from ie_hip_rope_table. */
inline void rope_and_cache(float* q, const float* k, const float* v, void* k_pool, void* v_pool,
                           const float* rope_table, int table_positions, int T,
                           const int* row_pos, const int* row_seq, const KvLayout& kv,
                           int n_heads, int n_kv_heads, int head_dim, hipStream_t stream) {
  check(ie_hip_rope_and_cache(q, k, v, k_pool, v_pool, rope_table, table_positions, T, row_pos,
                              row_seq, kv.c(), n_heads, n_kv_heads, head_dim, stream));
}

/* attention (kernels.cuh:76-87): part_o + part_ml become one workspace of
 * attention_workspace_bytes(); chunk_tokens is the partition length the
 * chunk count was computed with. */
inline void attention(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                      const int* row_pos, const int* row_seq, const KvLayout& kv, int num_chunks,
                      int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                      int head_dim, hipStream_t stream) {
  check(ie_hip_attention(out, q, k_pool, v_pool, T, row_pos, row_seq, kv.c(), num_chunks,
                         chunk_tokens, workspace, n_heads, n_kv_heads, head_dim, stream));
}

/* The decode work list built on the host (ie_hip_attention_plan) and the calls
 * that read it; results are those of attention / rope_cache_attention. */
inline size_t attention_plan_ints(int T, int num_chunks, int chunk_tokens) {
  return ie_hip_attention_plan_ints(T, num_chunks, chunk_tokens);
}
inline void attention_plan(int32_t* plan, size_t plan_capacity, int T, const int* row_pos,
                           const int* row_seq, const int32_t* tables, int max_seqs, int max_pages,
                           int num_chunks, int chunk_tokens) {
  check(ie_hip_attention_plan(plan, plan_capacity, T, row_pos, row_seq, tables, max_seqs,
                              max_pages, num_chunks, chunk_tokens));
}
inline void attention_planned(float* out, const float* q, const void* k_pool, const void* v_pool,
                              int T, const int* row_pos, const int* row_seq, const KvLayout& kv,
                              int num_chunks, int chunk_tokens, void* workspace,
                              const int32_t* plan, size_t plan_capacity, int n_heads,
                              int n_kv_heads, int head_dim, hipStream_t stream) {
  check(ie_hip_attention_planned(out, q, k_pool, v_pool, T, row_pos, row_seq, kv.c(), num_chunks,
                                 chunk_tokens, workspace, plan, plan_capacity, n_heads,
                                 n_kv_heads, head_dim, stream));
}

/* rope_and_cache followed by attention for a decode step, in one launch
 * (rows of distinct sequences; see ie_hip_rope_cache_attention). */
inline bool rope_cache_attention_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                           int head_dim, int chunk_tokens) {
  return ie_hip_rope_cache_attention_supported(kv_dtype, n_heads, n_kv_heads, head_dim,
                                               chunk_tokens) != 0;
}
inline void rope_cache_attention(float* out, const float* q, const float* k, const float* v,
                                 void* k_pool, void* v_pool, const float* rope_table,
                                 int table_positions, int T, const int* row_pos,
                                 const int* row_seq, const KvLayout& kv, int num_chunks,
                                 int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                                 int head_dim, hipStream_t stream) {
  check(ie_hip_rope_cache_attention(out, q, k, v, k_pool, v_pool, rope_table, table_positions, T,
                                    row_pos, row_seq, kv.c(), num_chunks, chunk_tokens, workspace,
                                    n_heads, n_kv_heads, head_dim, stream));
}

inline void rope_cache_attention_planned(float* out, const float* q, const float* k,
                                         const float* v, void* k_pool, void* v_pool,
                                         const float* rope_table, int table_positions, int T,
                                         const int* row_pos, const int* row_seq,
                                         const KvLayout& kv, int num_chunks, int chunk_tokens,
                                         void* workspace, const int32_t* plan,
                                         size_t plan_capacity, int n_heads, int n_kv_heads,
                                         int head_dim, hipStream_t stream) {
  check(ie_hip_rope_cache_attention_planned(out, q, k, v, k_pool, v_pool, rope_table,
                                            table_positions, T, row_pos, row_seq, kv.c(),
                                            num_chunks, chunk_tokens, workspace, plan,
                                            plan_capacity, n_heads, n_kv_heads, head_dim, stream));
}

/* attention_prefill_supported / attention_prefill (kernels.cuh:89-96). */
inline bool attention_prefill_supported(int n_heads, int n_kv_heads, int head_dim) {
  return ie_hip_attention_prefill_supported(n_heads, n_kv_heads, head_dim) != 0;
}
inline void attention_prefill(float* out, const float* q, const void* k_pool, const void* v_pool,
                              int T, const int* row_pos, const int* row_seq, const KvLayout& kv,
                              int n_heads, int n_kv_heads, int head_dim, hipStream_t stream) {
  check(ie_hip_attention_prefill(out, q, k_pool, v_pool, T, row_pos, row_seq, kv.c(), n_heads,
                                 n_kv_heads, head_dim, stream));
}

/* rope_and_cache followed by attention_prefill for a prompt chunk, q rotated
 * inside the prefill kernel (see ie_hip_rope_cache_attention_prefill). */
inline bool rope_cache_attention_prefill_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                                   int head_dim) {
  return ie_hip_rope_cache_attention_prefill_supported(kv_dtype, n_heads, n_kv_heads,
                                                       head_dim) != 0;
}
inline void rope_cache_attention_prefill(float* out, const float* q, const float* k,
                                         const float* v, void* k_pool, void* v_pool,
                                         const float* rope_table, int table_positions, int T,
                                         const int* row_pos, const int* row_seq,
                                         const KvLayout& kv, int n_heads, int n_kv_heads,
                                         int head_dim, hipStream_t stream) {
  check(ie_hip_rope_cache_attention_prefill(out, q, k, v, k_pool, v_pool, rope_table,
                                            table_positions, T, row_pos, row_seq, kv.c(), n_heads,
                                            n_kv_heads, head_dim, stream));
}

/* attention_chunks (kernels.cuh:98-99), for a given partition length. */
inline int attention_chunks(int context_tokens, int chunk_tokens) {
  const int n = ie_hip_attention_chunks(context_tokens, chunk_tokens);
  if (n <= 0) throw std::runtime_error("attention_chunks: context and chunk must be positive");
  return n;
}
inline int attention_chunk_tokens(int T, int max_context, int kv_dtype) {
  return ie_hip_attention_chunk_tokens(T, max_context, kv_dtype);
}
inline size_t attention_workspace_bytes(int T, int n_heads, int head_dim, int num_chunks) {
  return ie_hip_attention_workspace_bytes(T, n_heads, head_dim, num_chunks);
}

/* embedding / rmsnorm / matmul / gate_up_silu (kernels.cuh:48-66) over an
 * ie_matrix (DeviceMatrix, kernels.cuh:40-46). */
inline void embedding(float* x, const int32_t* ids, const ie_matrix& e, int T, hipStream_t stream) {
  check(ie_hip_embedding(x, ids, e, T, stream));
}
inline void rmsnorm(float* y, const float* x, const float* weight, int T, int dim, float eps,
                    hipStream_t stream) {
  check(ie_hip_rmsnorm(y, x, weight, T, dim, eps, stream));
}
inline void matmul(float* y, const float* x, const ie_matrix& w, const float* bias, int T,
                   bool accumulate, hipStream_t stream) {
  check(ie_hip_matmul(y, x, w, bias, T, accumulate ? 1 : 0, stream));
}
inline void qkv_proj(float* q, float* k, float* v, const float* x, const ie_matrix& w_qkv,
                     const float* b_qkv, int T, int q_dim, int kv_dim, hipStream_t stream) {
  check(ie_hip_qkv_proj(q, k, v, x, w_qkv, b_qkv, T, q_dim, kv_dim, stream));
}
inline void gate_up_silu(float* out, const float* x, const ie_matrix& wg, const ie_matrix& wu,
                         int T, hipStream_t stream) {
  check(ie_hip_gate_up_silu(out, x, wg, wu, T, stream));
}
/* rmsnorm folded into qkv_proj / gate_up_silu (no reference counterpart). */
inline void rmsnorm_qkv_proj(float* q, float* k, float* v, const float* x, const float* norm,
                             float eps, const ie_matrix& w_qkv, const float* b_qkv, int T,
                             int q_dim, int kv_dim, hipStream_t stream) {
  check(ie_hip_rmsnorm_qkv_proj(q, k, v, x, norm, eps, w_qkv, b_qkv, T, q_dim, kv_dim, stream));
}
inline void rmsnorm_gate_up_silu(float* out, const float* x, const float* norm, float eps,
                                 const ie_matrix& wg, const ie_matrix& wu, int T,
                                 hipStream_t stream) {
  check(ie_hip_rmsnorm_gate_up_silu(out, x, norm, eps, wg, wu, T, stream));
}

/* gather_rows (kernels.cuh:101-102). */
inline void gather_rows(float* dst, const float* src, const int* rows, int R, int dim,
                        hipStream_t stream) {
  check(ie_hip_gather_rows(dst, src, rows, R, dim, stream));
}

/* argmax_rows (kernels.cuh:106): the greedy token of each logit row. */
inline void argmax_rows(int32_t* out, const float* logits, int R, int n, hipStream_t stream) {
  check(ie_hip_argmax_rows(out, logits, R, n, stream));
}

}  // namespace ie::hip

#endif  // IE_HIP_HPP_
