// Internal interface of the decode-attention kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "ie_hip.h"

namespace iehip {

inline size_t align256(size_t n) { return (n + 255) & ~size_t(255); }

// The caller-owned decode workspace, carved into its parts.
// The decode step's RoPE + append folded into the 16-bit attention launch:
// the rows' new k/v (float32, unrotated), the pools to write them into, and
// the host cos/sin table (ie_hip_rope_cache_attention).
struct FusedAppend {
  const float* k = nullptr;
  const float* v = nullptr;
  uint16_t* k_pool = nullptr;
  uint16_t* v_pool = nullptr;
  const float* table = nullptr;
  int table_positions = 0;
};

// A decode work list built on the host (ie_hip_attention_plan), one item per
// workgroup of the 16-bit kernel in its dispatch order: int32 header
// [items, chunk_tokens, num_chunks, rows], then per item [row, chunk, position,
// sequence, the chunk's page ids (-1 past the row's position or its table
// row)], padded to a multiple of 4 ints so every item is 16-byte aligned.
constexpr int kPlanHeader = 4;
__host__ __device__ inline int plan_stride(int chunk_tokens) { return 4 + ((chunk_tokens / IE_HIP_PAGE_SIZE + 3) & ~3); }
inline size_t plan_ints(int T, int num_chunks, int chunk_tokens) {
  return kPlanHeader + size_t(T) * num_chunks * plan_stride(chunk_tokens);
}

struct Workspace {
  float* part_o = nullptr;     // [T][n_heads][num_chunks][head_dim] unnormalised partial outputs
  float* part_ml = nullptr;    // [T][n_heads][num_chunks][2] partial max (log2 units) and sum
};

Workspace carve_workspace(void* base, int T, int n_heads, int head_dim, int num_chunks);
size_t workspace_bytes(int T, int n_heads, int head_dim, int num_chunks);

int decode_merge(float* out, const Workspace& ws, const int32_t* row_pos, int T, int n_heads,
                 int num_chunks, int chunk_tokens, hipStream_t stream);

// Process-wide kernel choice (ie_hip_set_attention_impl).
int attention_impl();

// float32 KV on v_mfma_f32_16x16x4_f32 (KV rows of 128 elements, at most 16
// query heads, chunks of whole pages up to 1024 tokens); `plan`: a device copy of
// ie_hip_attention_plan's work list, or nullptr.
bool decode_mfma_f32_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                               int chunk_tokens);
int decode_mfma_f32(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                    const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                    int num_chunks, int chunk_tokens, void* workspace, int n_heads,
                    int n_kv_heads, hipStream_t stream, const int32_t* plan);
bool decode_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                           int chunk_tokens);
int decode_mfma(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream,
                const FusedAppend* fused = nullptr, const int32_t* plan = nullptr);

int decode_valu(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream);

}  // namespace iehip
