// Fused RoPE + paged KV append (gfx950).
//
// Reference semantics: the CPU rope (src/ops.cpp:34-55) applied to each row at
// its own position, then the K/V rows written into the row's page slot
// (src/cuda/kernels.cu:183-186,278-307; CPU append src/model.cpp:70-75).
//
// Layout of the work: one thread per "item" of a row, items numbered
//   [0, q_items)                     4 rotation pairs (i..i+3, i+half..i+half+3) of a query head
//   [q_items, q_items + kv_rot)      4 rotation pairs of a key head
//   [.., + n_kv_heads*head_dim/4)    4 consecutive values of v
// so consecutive threads touch consecutive 16-byte pieces of q, k, v and of
// the destination page row (one 256-byte f16 row per token at Qwen2.5 shape).
// The angle's cos/sin come from the host table (ie_hip_rope_table), and the
// rotation is written with explicit fmaf in the order GCC compiles the
// reference expression; the library is built with -ffp-contract=off, so the
// result is bit-identical to the reference CPU path.
#include "common.hpp"

namespace iehip {
namespace {

constexpr int kThreads = 256;

template <int KV, int HD>
__global__ void __launch_bounds__(kThreads)
rope_append_kernel(float* __restrict__ q, const float* __restrict__ k, const float* __restrict__ v,
                   typename Kv<KV>::elem* __restrict__ k_pool,
                   typename Kv<KV>::elem* __restrict__ v_pool, const float* __restrict__ table,
                   int table_positions, int T, const int32_t* __restrict__ row_pos,
                   const int32_t* __restrict__ row_seq, const int32_t* __restrict__ tables,
                   int max_pages, int num_pages, int n_heads, int n_kv_heads, int q_items,
                   int items_per_row) {
  using K = Kv<KV>;
  constexpr int kHalf = HD / 2, kItemsPerHead = kHalf / 4;
  const int64_t gid = int64_t(blockIdx.x) * kThreads + threadIdx.x;
  const int t = int(gid / items_per_row);
  if (t >= T) return;
  const int j = int(gid - int64_t(t) * items_per_row);
  const int pos = row_pos[t];
  if (pos < 0 || pos >= table_positions) return;  // outside the table: row skipped
  const int kv_dim = n_kv_heads * HD;
  const int kv_rot_end = q_items + n_kv_heads * kItemsPerHead;

  // Destination slot (seq, pos) -> page tables[seq * max_pages + pos / 16], row pos % 16.
  const int page_index = pos / IE_HIP_PAGE_SIZE;
  int page = -1;
  if (j >= q_items && page_index < max_pages)
    page = tables[size_t(row_seq[t]) * max_pages + page_index];
  const bool page_ok = page >= 0 && page < num_pages;
  const size_t dst_row = (size_t(page_ok ? page : 0) * IE_HIP_PAGE_SIZE + pos % IE_HIP_PAGE_SIZE) * kv_dim;

  if (j < kv_rot_end) {
    const int head = j / kItemsPerHead, i = (j % kItemsPerHead) * 4;
    const float4 c4 = *reinterpret_cast<const float4*>(table + size_t(pos) * HD + i);
    const float4 s4 = *reinterpret_cast<const float4*>(table + size_t(pos) * HD + kHalf + i);
    const float c[4] = {c4.x, c4.y, c4.z, c4.w}, s[4] = {s4.x, s4.y, s4.z, s4.w};
    const float* src;
    if (j < q_items)
      src = q + (size_t(t) * n_heads + head) * HD;
    else
      src = k + size_t(t) * kv_dim + size_t(head - n_heads * (q_items > 0)) * HD;
    const float4 a4 = *reinterpret_cast<const float4*>(src + i);
    const float4 b4 = *reinterpret_cast<const float4*>(src + kHalf + i);
    const float x0[4] = {a4.x, a4.y, a4.z, a4.w}, x1[4] = {b4.x, b4.y, b4.z, b4.w};
    float r0[4], r1[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      r0[u] = __builtin_fmaf(x0[u], c[u], -(x1[u] * s[u]));  // x0*c - x1*s
      r1[u] = __builtin_fmaf(x1[u], c[u], x0[u] * s[u]);     // x1*c + x0*s
    }
    if (j < q_items) {
      float* dst = q + (size_t(t) * n_heads + head) * HD;
      *reinterpret_cast<float4*>(dst + i) = make_float4(r0[0], r0[1], r0[2], r0[3]);
      *reinterpret_cast<float4*>(dst + kHalf + i) = make_float4(r1[0], r1[1], r1[2], r1[3]);
    } else if (page_ok) {
      typename K::elem* dst = k_pool + dst_row + size_t(head - n_heads * (q_items > 0)) * HD;
      K::store4(dst + i, r0);
      K::store4(dst + kHalf + i, r1);
    }
  } else if (page_ok) {
    const int i = (j - kv_rot_end) * 4;
    const float4 x = *reinterpret_cast<const float4*>(v + size_t(t) * kv_dim + i);
    const float xs[4] = {x.x, x.y, x.z, x.w};
    K::store4(v_pool + dst_row + i, xs);
  }
}

template <int KV, int HD>
int launch(float* q, const float* k, const float* v, void* k_pool, void* v_pool,
           const float* table, int table_positions, int T, const int32_t* row_pos,
           const int32_t* row_seq, const ie_kv_layout& kv, int n_heads, int n_kv_heads,
           hipStream_t stream) {
  using E = typename Kv<KV>::elem;
  const int per_head = HD / 8;
  const int q_items = q ? n_heads * per_head : 0;
  const int items = q_items + n_kv_heads * per_head + n_kv_heads * HD / 4;
  const int64_t threads = int64_t(T) * items;
  const int64_t blocks = (threads + kThreads - 1) / kThreads;
  if (blocks > 0x7fffffff) return fail(IE_HIP_EINVAL, "rope_and_cache: too many rows");
  hipLaunchKernelGGL((rope_append_kernel<KV, HD>), dim3(unsigned(blocks)), dim3(kThreads), 0,
                     stream, q, k, v, static_cast<E*>(k_pool), static_cast<E*>(v_pool), table,
                     table_positions, T, row_pos, row_seq, kv.tables, kv.max_pages, kv.num_pages,
                     n_heads, n_kv_heads, q_items, items);
  return check_launch("rope_and_cache");
}

}  // namespace
}  // namespace iehip

using namespace iehip;

extern "C" int ie_hip_rope_and_cache(float* q, const float* k, const float* v, void* k_pool,
                                     void* v_pool, const float* rope_table, int table_positions,
                                     int T, const int32_t* row_pos, const int32_t* row_seq,
                                     ie_kv_layout kv, int n_heads, int n_kv_heads, int head_dim,
                                     hipStream_t stream) {
  clear_error();
  if (int rc = check_layout(kv, "rope_and_cache")) return rc;
  if (T < 0 || n_heads <= 0 || n_kv_heads <= 0)
    return fail(IE_HIP_EINVAL, "rope_and_cache: bad row or head counts");
  if (head_dim != 64 && head_dim != 128)
    return fail(IE_HIP_EINVAL, "rope_and_cache: head_dim must be 64 or 128");
  if (!k || !v || !k_pool || !v_pool || !rope_table || !row_pos || !row_seq)
    return fail(IE_HIP_EINVAL, "rope_and_cache: null pointer");
  if (table_positions <= 0) return fail(IE_HIP_EINVAL, "rope_and_cache: empty RoPE table");
  if (T == 0) return IE_HIP_OK;
#define IE_ROPE_CASE(KVT, HDV)                                                                    \
  if (kv.kv_dtype == KVT && head_dim == HDV)                                                      \
    return launch<KVT, HDV>(q, k, v, k_pool, v_pool, rope_table, table_positions, T, row_pos,     \
                            row_seq, kv, n_heads, n_kv_heads, stream);
  IE_ROPE_CASE(IE_KV_F32, 64)
  IE_ROPE_CASE(IE_KV_F16, 64)
  IE_ROPE_CASE(IE_KV_BF16, 64)
  IE_ROPE_CASE(IE_KV_F32, 128)
  IE_ROPE_CASE(IE_KV_F16, 128)
  IE_ROPE_CASE(IE_KV_BF16, 128)
#undef IE_ROPE_CASE
  return fail(IE_HIP_EINVAL, "rope_and_cache: unsupported kv_dtype");
}
