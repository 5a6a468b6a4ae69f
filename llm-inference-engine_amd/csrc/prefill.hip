// Prefill (prompt-chunk) attention into pages (gfx950).
//
// Rows are consecutive positions of one sequence (row_pos[t] = row_pos[0] + t),
// already appended to the cache. Row t attends causally to positions
// 0..row_pos[t] (reference semantics: src/ops.cpp:70-108; the reference's GPU
// prompt kernels are src/cuda/kernels.cu:527-776).
//
// prefill_valu: float32 arithmetic on the VALU, used for the f32 KV cache
// (where 1e-5 relative error rules out 16-bit matrix inputs). A workgroup takes
// 32 consecutive query rows and all query heads of one KV head; thread
// (row, head slot) keeps its query (pre-scaled by 1/sqrt(64) = 2^-3, exact)
// and its output row in registers. K/V tiles of 32 positions are staged in LDS
// (widened to f32) and shared by the 32 x group queries; softmax is online
// (running max and sum, rescaled when the max rises).
#include <algorithm>

#include "common.hpp"
#include "prefill.hpp"
#include "decode.hpp"

namespace iehip {
namespace {

constexpr int kPfThreads = 256;
constexpr int kPfRows = 32;   // query rows per workgroup
constexpr int kPfSlots = 8;   // head slots per row (group <= 8)
constexpr int kPfKeys = 32;   // positions per LDS tile

template <int KV, int HD>
__global__ void __launch_bounds__(kPfThreads)
prefill_valu(float* __restrict__ out, const float* __restrict__ q,
             const typename Kv<KV>::elem* __restrict__ k_pool,
             const typename Kv<KV>::elem* __restrict__ v_pool, int T,
             const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
             const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
             int n_kv_heads, float scale) {
  using K = Kv<KV>;
  static_assert(HD == 64, "8 threads x 8 elements stage one 64-wide row");
  __shared__ __align__(16) float ks[kPfKeys][HD];
  __shared__ __align__(16) float vs[kPfKeys][HD];
  __shared__ int kvis[kPfKeys];  // key j of the tile exists: at most max_pos, page in the pool
  const int group = n_heads / n_kv_heads;
  const int kvh = blockIdx.y, t0 = blockIdx.x * kPfRows;
  const int tid = threadIdx.x, qi = tid / kPfSlots, g = tid % kPfSlots;
  const int t = t0 + qi;
  const bool active = g < group && t < T;
  const int seq = row_seq[0];
  const int max_pos = row_pos[min(t0 + kPfRows, T) - 1];
  const int pos = active ? row_pos[t] : -1;
  const int h = kvh * group + g;
  const int kv_dim = n_kv_heads * HD;

  float qr[HD], acc[HD];
#pragma unroll
  for (int d = 0; d < HD; d += 4) {
    float4 x = make_float4(0.f, 0.f, 0.f, 0.f);
    if (active) x = *reinterpret_cast<const float4*>(q + (size_t(t) * n_heads + h) * HD + d);
    qr[d] = x.x * scale;
    qr[d + 1] = x.y * scale;
    qr[d + 2] = x.z * scale;
    qr[d + 3] = x.w * scale;
  }
#pragma unroll
  for (int d = 0; d < HD; ++d) acc[d] = 0.0f;
  float m = -INFINITY, l = 0.0f;

  for (int s0 = 0; s0 <= max_pos; s0 += kPfKeys) {
    __syncthreads();  // the previous tile is no longer read
    {
      const int j = tid / 8, d8 = (tid % 8) * 8;
      const int s = s0 + j;
      float kx[8] = {0, 0, 0, 0, 0, 0, 0, 0}, vx[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      bool vis = false;
      if (s <= max_pos) {
        const int pi = s / IE_HIP_PAGE_SIZE;
        const int page = pi < max_pages ? tables[size_t(seq) * max_pages + pi] : -1;
        if (page >= 0 && page < num_pages) {  // a page outside the pool is not attended
          const size_t off = (size_t(page) * IE_HIP_PAGE_SIZE + s % IE_HIP_PAGE_SIZE) * kv_dim +
                             size_t(kvh) * HD + d8;
          K::load8(k_pool + off, kx);
          K::load8(v_pool + off, vx);
          vis = true;
        }
      }
      if (d8 == 0) kvis[j] = vis;
      *reinterpret_cast<float4*>(&ks[j][d8]) = make_float4(kx[0], kx[1], kx[2], kx[3]);
      *reinterpret_cast<float4*>(&ks[j][d8 + 4]) = make_float4(kx[4], kx[5], kx[6], kx[7]);
      *reinterpret_cast<float4*>(&vs[j][d8]) = make_float4(vx[0], vx[1], vx[2], vx[3]);
      *reinterpret_cast<float4*>(&vs[j][d8 + 4]) = make_float4(vx[4], vx[5], vx[6], vx[7]);
    }
    __syncthreads();

    float sc[kPfKeys];
    float tile_max = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPfKeys; ++j) {
      float dot = 0.0f;
#pragma unroll
      for (int d = 0; d < HD; d += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(&ks[j][d]);
        dot = __builtin_fmaf(qr[d], kk.x, dot);
        dot = __builtin_fmaf(qr[d + 1], kk.y, dot);
        dot = __builtin_fmaf(qr[d + 2], kk.z, dot);
        dot = __builtin_fmaf(qr[d + 3], kk.w, dot);
      }
      sc[j] = (s0 + j <= pos && kvis[j]) ? dot : -INFINITY;
      tile_max = fmaxf(tile_max, sc[j]);
    }
    const float m_new = fmaxf(m, tile_max);
    if (m_new == -INFINITY) continue;  // nothing visible yet (or an inactive slot)
    const float corr = expf(m - m_new);
    l *= corr;
#pragma unroll
    for (int d = 0; d < HD; ++d) acc[d] *= corr;
#pragma unroll
    for (int j = 0; j < kPfKeys; ++j) {
      const float pj = expf(sc[j] - m_new);
      l += pj;
#pragma unroll
      for (int d = 0; d < HD; d += 4) {
        const float4 vv = *reinterpret_cast<const float4*>(&vs[j][d]);
        acc[d] = __builtin_fmaf(pj, vv.x, acc[d]);
        acc[d + 1] = __builtin_fmaf(pj, vv.y, acc[d + 1]);
        acc[d + 2] = __builtin_fmaf(pj, vv.z, acc[d + 2]);
        acc[d + 3] = __builtin_fmaf(pj, vv.w, acc[d + 3]);
      }
    }
    m = m_new;
  }

  if (!active) return;
  const float inv_l = 1.0f / l;
  float* o = out + (size_t(t) * n_heads + h) * HD;
#pragma unroll
  for (int d = 0; d < HD; d += 4)
    *reinterpret_cast<float4*>(o + d) =
        make_float4(acc[d] * inv_l, acc[d + 1] * inv_l, acc[d + 2] * inv_l, acc[d + 3] * inv_l);
}

template <int KV>
int launch_prefill_valu(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream) {
  using E = typename Kv<KV>::elem;
  constexpr int HD = 64;
  const dim3 grid((T + kPfRows - 1) / kPfRows, n_kv_heads);
  hipLaunchKernelGGL((prefill_valu<KV, HD>), grid, dim3(kPfThreads), 0, stream, out, q,
                     static_cast<const E*>(k_pool), static_cast<const E*>(v_pool), T, row_pos,
                     row_seq, kv.tables, kv.max_pages, kv.num_pages, n_heads, n_kv_heads,
                     1.0f / sqrtf(float(HD)));
  return check_launch("attention_prefill_valu");
}

}  // namespace

int prefill_valu_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream) {
  switch (kv.kv_dtype) {
    case IE_KV_F32:
      return launch_prefill_valu<IE_KV_F32>(out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                            n_heads, n_kv_heads, stream);
    case IE_KV_F16:
      return launch_prefill_valu<IE_KV_F16>(out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                            n_heads, n_kv_heads, stream);
    case IE_KV_BF16:
      return launch_prefill_valu<IE_KV_BF16>(out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                             n_heads, n_kv_heads, stream);
  }
  return fail(IE_HIP_EINVAL, "attention_prefill: unsupported kv_dtype");
}

}  // namespace iehip

using namespace iehip;

extern "C" {

int ie_hip_attention_prefill_supported(int n_heads, int n_kv_heads, int head_dim) {
  return head_dim == 64 && n_kv_heads > 0 && n_heads > 0 && n_heads % n_kv_heads == 0 &&
         n_heads / n_kv_heads <= kPfSlots;
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
  if (impl != IE_HIP_IMPL_VALU && prefill_mfma_enabled() &&
      prefill_mfma_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim))
    return prefill_mfma_launch(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, n_heads,
                               n_kv_heads, stream);
  if (impl == IE_HIP_IMPL_MFMA)
    return fail(IE_HIP_EINVAL, "attention_prefill: the MFMA kernels do not support this shape");
  return prefill_valu_launch(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, n_heads, n_kv_heads,
                             stream);
}

}  // extern "C"
