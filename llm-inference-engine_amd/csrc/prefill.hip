// Prefill (prompt-chunk) attention into pages (gfx950).
//
// Rows are consecutive positions of one sequence (row_pos[t] = row_pos[0] + t),
// already appended to the cache. Row t attends causally to positions
// 0..row_pos[t] (reference semantics: src/ops.cpp:70-108).
//
// The matrix-core kernels (prefill_mfma.hip) take every shape this entry
// point accepts. prefill_wave is the float32 VALU kernel that
// IE_HIP_IMPL_VALU selects, as an independent implementation to check them
// against: a short, plain kernel rather than a fast one.
//
// prefill_wave: one wave per (query row, KV head), streaming the row's
// positions in tiles of 64:
//   scores  -- lane j takes position s0 + j: its key row (64 dims of the KV
//              head, widened to f32) in registers, dotted with each of the
//              group's G queries (pre-scaled by 1/8, exact) read from LDS;
//   softmax -- per head, the tile's max and sum by wave64 butterflies, the
//              running (max, sum) rescaled when the max rises;
//   values  -- the lanes switch roles: lane d owns output dim d and adds, for
//              each of the tile's positions, the position's weights (from
//              LDS) times its value row's dim d (64 lanes read the row's 64
//              contiguous elements).
// Positions whose page lies outside the pool are not attended.
#include <algorithm>

#include "common.hpp"
#include "prefill.hpp"
#include "decode.hpp"

namespace iehip {
namespace {

constexpr int kPwWaves = 4;   // waves (query rows) per workgroup
constexpr int kPwMaxGroup = 8;

__device__ __forceinline__ float wave_max64(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int KV, int G>
__global__ void __launch_bounds__(64 * kPwWaves)
prefill_wave(float* __restrict__ out, const float* __restrict__ q,
             const typename Kv<KV>::elem* __restrict__ k_pool,
             const typename Kv<KV>::elem* __restrict__ v_pool, int T,
             const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
             const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
             int n_kv_heads) {
  constexpr int HD = 64;
  using K = Kv<KV>;
  __shared__ float q_s[kPwWaves][G][HD];
  __shared__ float w_s[kPwWaves][G][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * kPwWaves + wave;
  const int h = blockIdx.y;  // KV head
  if (t >= T) return;        // uniform per wave; no workgroup barrier below
  const int p = row_pos[t], seq = row_seq[t];
  const int kv_dim = n_kv_heads * HD;
  float* orow = out + (size_t(t) * n_heads + size_t(h) * G) * HD;
  if (p < 0) {
#pragma unroll
    for (int g = 0; g < G; ++g) orow[g * HD + lane] = 0.0f;
    return;
  }
#pragma unroll
  for (int g = 0; g < G; ++g)
    q_s[wave][g][lane] = q[(size_t(t) * n_heads + size_t(h) * G + g) * HD + lane] * 0.125f;
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");

  float m[G], l[G], acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
    acc[g] = 0.0f;
  }
  const int32_t* tab = tables + size_t(seq) * max_pages;
  for (int s0 = 0; s0 <= p; s0 += 64) {
    // Scores: lane = position s0 + lane.
    const int pos = s0 + lane;
    const int pi = pos / IE_HIP_PAGE_SIZE;
    const int page = (pos <= p && pi < max_pages) ? tab[pi] : -1;
    const bool ok = page >= 0 && page < num_pages;
    float s[G];
#pragma unroll
    for (int g = 0; g < G; ++g) s[g] = -INFINITY;
    if (ok) {
      const typename K::elem* kr =
          k_pool + (size_t(page) * IE_HIP_PAGE_SIZE + pos % IE_HIP_PAGE_SIZE) * kv_dim + h * HD;
      float kk[HD];
#pragma unroll
      for (int d8 = 0; d8 < HD / 8; ++d8) K::load8(kr + 8 * d8, kk + 8 * d8);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        float a = 0.0f;
#pragma unroll
        for (int d = 0; d < HD; ++d) a = __builtin_fmaf(q_s[wave][g][d], kk[d], a);
        s[g] = a;
      }
    }
    // Online softmax per head; the tile's weights to LDS for the value pass.
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float m_new = fmaxf(m[g], wave_max64(s[g]));
      const float e = m_new == -INFINITY ? 0.0f : expf(s[g] - m_new);
      const float corr = m[g] == -INFINITY ? 0.0f : expf(m[g] - m_new);
      l[g] = __builtin_fmaf(l[g], corr, wave_sum64(e));
      acc[g] *= corr;
      m[g] = m_new;
      w_s[wave][g][lane] = e;
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    // Values: lane = output dim.
    const int n = min(64, p + 1 - s0);
    for (int j = 0; j < n; ++j) {
      const int pg = __builtin_amdgcn_readlane(page, j);
      if (pg < 0 || pg >= num_pages) continue;
      const int pj = s0 + j;
      const float v = K::load1(
          v_pool + (size_t(pg) * IE_HIP_PAGE_SIZE + pj % IE_HIP_PAGE_SIZE) * kv_dim + h * HD + lane);
#pragma unroll
      for (int g = 0; g < G; ++g) acc[g] = __builtin_fmaf(w_s[wave][g][j], v, acc[g]);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
#pragma unroll
  for (int g = 0; g < G; ++g) orow[g * HD + lane] = l[g] > 0.0f ? acc[g] / l[g] : 0.0f;
}

template <int KV, int G>
int launch_prefill_wave(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream) {
  using E = typename Kv<KV>::elem;
  const dim3 grid((T + kPwWaves - 1) / kPwWaves, n_kv_heads);
  hipLaunchKernelGGL((prefill_wave<KV, G>), grid, dim3(64 * kPwWaves), 0, stream, out, q,
                     static_cast<const E*>(k_pool), static_cast<const E*>(v_pool), T, row_pos,
                     row_seq, kv.tables, kv.max_pages, kv.num_pages, n_heads, n_kv_heads);
  return check_launch("attention_prefill_valu");
}

template <int KV>
int dispatch_prefill_group(int group, float* out, const float* q, const void* k_pool,
                           const void* v_pool, int T, const int32_t* row_pos,
                           const int32_t* row_seq, const ie_kv_layout& kv, int n_heads,
                           int n_kv_heads, hipStream_t stream) {
  switch (group) {
#define IE_PW_CASE(G)                                                                       \
  case G:                                                                                   \
    return launch_prefill_wave<KV, G>(out, q, k_pool, v_pool, T, row_pos, row_seq, kv,      \
                                      n_heads, n_kv_heads, stream);
    IE_PW_CASE(1)
    IE_PW_CASE(2)
    IE_PW_CASE(3)
    IE_PW_CASE(4)
    IE_PW_CASE(5)
    IE_PW_CASE(6)
    IE_PW_CASE(7)
    IE_PW_CASE(8)
#undef IE_PW_CASE
  }
  return fail(IE_HIP_EINVAL, "attention_prefill: at most 8 query heads per KV head");
}

}  // namespace

int prefill_valu_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream) {
  const int group = n_heads / n_kv_heads;
  switch (kv.kv_dtype) {
    case IE_KV_F32:
      return dispatch_prefill_group<IE_KV_F32>(group, out, q, k_pool, v_pool, T, row_pos,
                                               row_seq, kv, n_heads, n_kv_heads, stream);
    case IE_KV_F16:
      return dispatch_prefill_group<IE_KV_F16>(group, out, q, k_pool, v_pool, T, row_pos,
                                               row_seq, kv, n_heads, n_kv_heads, stream);
    case IE_KV_BF16:
      return dispatch_prefill_group<IE_KV_BF16>(group, out, q, k_pool, v_pool, T, row_pos,
                                                row_seq, kv, n_heads, n_kv_heads, stream);
  }
  return fail(IE_HIP_EINVAL, "attention_prefill: unsupported kv_dtype");
}

}  // namespace iehip

using namespace iehip;

extern "C" {

int ie_hip_attention_prefill_supported(int n_heads, int n_kv_heads, int head_dim) {
  return head_dim == 64 && n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0 &&
         n_heads / n_kv_heads <= kPwMaxGroup;
}

int ie_hip_attention_prefill(float* out, const float* q, const void* k_pool, const void* v_pool,
                             int T, const int32_t* row_pos, const int32_t* row_seq,
                             ie_kv_layout kv, int n_heads, int n_kv_heads, int head_dim,
                             hipStream_t stream) {
  clear_error();
  if (int rc = check_layout(kv, "attention_prefill")) return rc;
  if (!ie_hip_attention_prefill_supported(n_heads, n_kv_heads, head_dim))
    return fail(IE_HIP_EINVAL,
                "attention_prefill: needs head_dim 64 and at most 8 query heads per KV head");
  if (T < 0) return fail(IE_HIP_EINVAL, "attention_prefill: negative row count");
  if (T == 0) return IE_HIP_OK;
  if (!out || !q || !k_pool || !v_pool || !row_pos || !row_seq)
    return fail(IE_HIP_EINVAL, "attention_prefill: null pointer");
  const int impl = attention_impl();
  if (impl != IE_HIP_IMPL_VALU &&
      prefill_mfma_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim))
    return prefill_mfma_launch(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, n_heads,
                               n_kv_heads, PrefillRope{}, stream);
  if (impl == IE_HIP_IMPL_MFMA)
    return fail(IE_HIP_EINVAL, "attention_prefill: the MFMA kernels do not support this shape");
  return prefill_valu_launch(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, n_heads, n_kv_heads,
                             stream);
}

int ie_hip_rope_cache_attention_prefill_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                                   int head_dim) {
  return attention_impl() != IE_HIP_IMPL_VALU && kv_dtype != IE_KV_F32 &&
         prefill_mfma_supported(kv_dtype, n_heads, n_kv_heads, head_dim);
}

int ie_hip_rope_cache_attention_prefill(float* out, const float* q, const float* k, const float* v,
                                        void* k_pool, void* v_pool, const float* rope_table,
                                        int table_positions, int T, const int32_t* row_pos,
                                        const int32_t* row_seq, ie_kv_layout kv, int n_heads,
                                        int n_kv_heads, int head_dim, hipStream_t stream) {
  clear_error();
  if (int rc = check_layout(kv, "rope_cache_attention_prefill")) return rc;
  if (!ie_hip_rope_cache_attention_prefill_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim))
    return fail(IE_HIP_EINVAL,
                "rope_cache_attention_prefill: needs a 16-bit cache and the matrix-core prefill "
                "kernel (head_dim 64, at most 8 query heads per KV head, not IE_HIP_IMPL_VALU); "
                "use rope_and_cache + attention_prefill");
  if (T < 0) return fail(IE_HIP_EINVAL, "rope_cache_attention_prefill: negative row count");
  if (T == 0) return IE_HIP_OK;
  if (!out || !q || !k || !v || !k_pool || !v_pool || !rope_table || !row_pos || !row_seq)
    return fail(IE_HIP_EINVAL, "rope_cache_attention_prefill: null pointer");
  if (table_positions <= 0)
    return fail(IE_HIP_EINVAL, "rope_cache_attention_prefill: empty RoPE table");
  // K and V rotated (K) and stored; q is left as it is and rotated by the prefill
  // kernel as it loads it.
  if (int rc = ie_hip_rope_and_cache(nullptr, k, v, k_pool, v_pool, rope_table, table_positions, T,
                                     row_pos, row_seq, kv, n_heads, n_kv_heads, head_dim, stream))
    return rc;
  return prefill_mfma_launch(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, n_heads, n_kv_heads,
                             PrefillRope{rope_table, table_positions}, stream);
}

}  // extern "C"
