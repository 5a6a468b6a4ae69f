// Internal interface of the prefill-attention kernels.
#pragma once

#include <cstdint>

#include "ie_hip.h"

namespace iehip {

int prefill_valu_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream);

// The RoPE table (ie_hip_rope_table layout, device memory, positions rows) when
// the prefill kernel rotates q itself; table == nullptr: q is already rotated.
struct PrefillRope {
  const float* table = nullptr;
  int positions = 0;
};

// QK^T and PV on MFMA (prefill_mfma.hip): 16-bit caches in their own type,
// float32 caches on the f32 matrix instructions.
bool prefill_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim);
int prefill_mfma_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, const PrefillRope& rope, hipStream_t stream);

}  // namespace iehip
