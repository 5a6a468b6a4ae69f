// Flash-decoding attention over block-tabled KV pages (gfx950, wave64).
//
// Reference semantics: each row's causal GQA attention over its cached
// positions, src/ops.cpp:70-108; the reference GPU path splits positions into
// chunks and merges by log-sum-exp (src/cuda/kernels.cu:309-507).
//
// This file: the VALU partial kernel (all KV dtypes) and the merge.
//   grid (T, n_kv_heads, num_chunks): rows vary fastest, so the dispatcher
//   hands out chunk 0 of every row first and the empty tail chunks of short
//   rows last; one 256-thread workgroup (4 waves) per (row, kv head, chunk).
//   1. page ids of the chunk -> LDS; the group's queries -> LDS.
//   2. scores: one lane per position, the position's key row read with 16-byte
//      loads, dot products against the LDS queries (broadcast reads) for all
//      query heads of the group; scores -> LDS.
//   3. chunk max and sum of exp per head: wave64 butterfly reductions, then
//      across the 4 waves through LDS.
//   4. values: lanes = 8 positions x 8 dim-slices of 8 (16-byte loads), every
//      value row read once for all heads of the group; butterfly-reduced over
//      the 8 positions, then across waves through LDS.
//   A row whose context fits one chunk writes `out` directly; otherwise the
//   chunk writes (o, m, l), m in log2 units (every partial kernel: the VALU one
//   here converts its natural-log max), and decode_merge_kernel combines them:
//   M = max m_c, L = sum l_c 2^(m_c - M), out = sum o_c 2^(m_c - M) / L.
#include <algorithm>
#include <atomic>
#include <mutex>
#include <vector>

#include "common.hpp"
#include "decode.hpp"
#include "mfma.hpp"

namespace iehip {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunk = 1024;
constexpr float kLog2eMerge = 1.4426950408889634f;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <int KV, int HD, int G>
__global__ void __launch_bounds__(kThreads)
decode_partial_valu(float* __restrict__ out, float* __restrict__ part_o,
                    float* __restrict__ part_ml, const float* __restrict__ q,
                    const typename Kv<KV>::elem* __restrict__ k_pool,
                    const typename Kv<KV>::elem* __restrict__ v_pool,
                    const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                    const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
                    int n_kv_heads, int num_chunks, int chunk_tokens, float scale) {
  using K = Kv<KV>;
  static_assert(HD == 64, "lanes 0..7 of a position group cover 64 dims in 8-element slices");
  extern __shared__ float scores[];  // [G][chunk_tokens]
  __shared__ __align__(16) float q_s[G][HD];
  __shared__ int pages_s[kMaxChunk / IE_HIP_PAGE_SIZE];
  __shared__ float red[kWaves][G];
  __shared__ float red_o[kWaves][G][HD];
  __shared__ float stat[2][G];

  const int t = blockIdx.x, kvh = blockIdx.y, c = blockIdx.z;
  const int p = row_pos[t];
  const int s0 = c * chunk_tokens;
  if (p < 0 || s0 > p) return;  // chunk in the future: nothing to do (uniform exit)
  const int n = min(s0 + chunk_tokens, p + 1) - s0;
  const int chunks_row = min(p / chunk_tokens + 1, num_chunks);
  const int seq = row_seq[t];
  const int h0 = kvh * G;
  const int kv_dim = n_kv_heads * HD;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  for (int i = tid; i < (n + IE_HIP_PAGE_SIZE - 1) / IE_HIP_PAGE_SIZE; i += kThreads) {
    const int pi = s0 / IE_HIP_PAGE_SIZE + i;
    const int page = pi < max_pages ? tables[size_t(seq) * max_pages + pi] : -1;
    pages_s[i] = (page >= 0 && page < num_pages) ? page : -1;  // -1: outside the pool, skipped
  }
  for (int i = tid; i < G * HD; i += kThreads)
    q_s[i / HD][i % HD] = q[(size_t(t) * n_heads + h0) * HD + i];
  __syncthreads();

  // 2. scores, one lane per position.
  float mx[G];
#pragma unroll
  for (int g = 0; g < G; ++g) mx[g] = -INFINITY;
  for (int tl = tid; tl < n; tl += kThreads) {
    const int page = pages_s[tl / IE_HIP_PAGE_SIZE];
    if (page < 0) {  // a page outside the pool: its positions are not attended
#pragma unroll
      for (int g = 0; g < G; ++g) scores[g * chunk_tokens + tl] = -INFINITY;
      continue;
    }
    const typename K::elem* kr =
        k_pool + (size_t(page) * IE_HIP_PAGE_SIZE + tl % IE_HIP_PAGE_SIZE) * kv_dim + kvh * HD;
    float kk[HD];
#pragma unroll
    for (int d8 = 0; d8 < HD / 8; ++d8) K::load8(kr + 8 * d8, kk + 8 * d8);
    float acc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] = 0.0f;
#pragma unroll
    for (int d4 = 0; d4 < HD / 4; ++d4) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 qa = *reinterpret_cast<const float4*>(&q_s[g][4 * d4]);
        acc[g] = __builtin_fmaf(qa.x, kk[4 * d4 + 0], acc[g]);
        acc[g] = __builtin_fmaf(qa.y, kk[4 * d4 + 1], acc[g]);
        acc[g] = __builtin_fmaf(qa.z, kk[4 * d4 + 2], acc[g]);
        acc[g] = __builtin_fmaf(qa.w, kk[4 * d4 + 3], acc[g]);
      }
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float s = acc[g] * scale;
      scores[g * chunk_tokens + tl] = s;
      mx[g] = fmaxf(mx[g], s);
    }
  }

  // 3. max, then exp and sum, per head.
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float m = wave_max(mx[g]);
    if (lane == 0) red[wave][g] = m;
  }
  __syncthreads();
  float M[G], ls[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    M[g] = red[0][g];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) M[g] = fmaxf(M[g], red[w][g]);
    ls[g] = 0.0f;
  }
  if (tid < G) {
    float m = red[0][tid];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) m = fmaxf(m, red[w][tid]);
    stat[0][tid] = m;
  }
  for (int tl = tid; tl < n; tl += kThreads) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      // M = -inf: every position of the chunk was skipped; its weights are 0.
      const float e = M[g] == -INFINITY ? 0.0f : expf(scores[g * chunk_tokens + tl] - M[g]);
      scores[g * chunk_tokens + tl] = e;
      ls[g] += e;
    }
  }
  __syncthreads();  // every lane has read `red` (maxima) before it is reused
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const float s = wave_sum(ls[g]);
    if (lane == 0) red[wave][g] = s;
  }
  __syncthreads();  // sums and the exp'd scores are visible
  if (tid < G) {
    float L = 0.0f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) L += red[w][tid];
    stat[1][tid] = L;
  }

  // 4. values: lane = (position group pg, dim slice ds), 8 dims per lane.
  const int pg = lane >> 3, ds = lane & 7;
  float acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[g][u] = 0.0f;
#pragma unroll 2
  for (int tl = wave * 8 + pg; tl < n; tl += kWaves * 8) {
    const int page = pages_s[tl / IE_HIP_PAGE_SIZE];
    if (page < 0) continue;  // skipped position (weight 0; its memory is never read)
    const typename K::elem* vr =
        v_pool + (size_t(page) * IE_HIP_PAGE_SIZE + tl % IE_HIP_PAGE_SIZE) * kv_dim + kvh * HD +
        ds * 8;
    float vv[8];
    K::load8(vr, vv);
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float w = scores[g * chunk_tokens + tl];
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[g][u] = __builtin_fmaf(w, vv[u], acc[g][u]);
    }
  }
#pragma unroll
  for (int off = 8; off < 64; off <<= 1)
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int u = 0; u < 8; ++u) acc[g][u] += __shfl_xor(acc[g][u], off, 64);
  if (pg == 0) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int u = 0; u < 8; ++u) red_o[wave][g][ds * 8 + u] = acc[g][u];
  }
  __syncthreads();

  for (int i = tid; i < G * HD; i += kThreads) {
    const int g = i / HD, d = i % HD;
    float o = red_o[0][g][d];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) o += red_o[w][g][d];
    const size_t head = size_t(t) * n_heads + h0 + g;
    if (chunks_row == 1)
      out[head * HD + d] = o / stat[1][g];
    else
      part_o[(head * num_chunks + c) * HD + d] = o;
  }
  if (chunks_row > 1 && tid < G) {
    const size_t slot = (size_t(t) * n_heads + h0 + tid) * num_chunks + c;
    part_ml[2 * slot] = stat[0][tid] * kLog2eMerge;  // log2 units, as the merge takes them
    part_ml[2 * slot + 1] = stat[1][tid];
  }
}

// Split-K merge: out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M), M = max m_c
// (m in log2 units).
//
// The order of the sums is fixed by the row alone, so a row's result does not
// depend on the batch, the launch shape or the chunk count the caller sizes
// the workspace for: the leaves are the row's chunks 0 .. nc-1 (nc from its
// position and chunk_tokens); block b = chunks [8b, 8b+8) is folded in chunk
// order, and the blocks are combined by a binary tree over b -- node (b, b+1),
// then (b..b+1, b+2..b+3), ... each as merge(left, right). Slots past nc and
// chunks that saw no position (m = -inf) are identities that every merge
// passes through unchanged, so padding the tree to any width changes nothing.
//
// A workgroup takes one (head, row) and a slice of 64/S output dims (S = 1 to
// 16 slices, more slices when rows x heads alone would leave compute units
// idle or the row has more chunks than one wave's lanes hold). In a wave, lane = (dim quad, block lane): the slice's Q quads of
// float4, each over CL = 64/Q consecutive lanes; block lane i of wave w owns
// block w * CL + i and loads its 8 chunks at once. The tree runs over the
// block lanes -- node (b, b + k) forms in b's lane from lane b + k, a VALU
// lane move (DPP within a row of 16 lanes, the permlane swaps across rows) --
// and then over the waves through LDS.
constexpr int kMergeBlock = 8;
constexpr int kMergeMaxWaves = 16;

struct MergeAcc {
  float m, l;
  float4 a;
};

// (M1, L1, A1) + (M2, L2, A2) = (M, L1 2^(M1-M) + L2 2^(M2-M), A1 2^(M1-M) +
// A2 2^(M2-M)), M = max(M1, M2); an identity side (M = -inf) returns the
// other side bit for bit.
__device__ __forceinline__ MergeAcc merge_pair(const MergeAcc& x, const MergeAcc& y) {
  if (y.m == -INFINITY) return x;
  if (x.m == -INFINITY) return y;
  const float m = fmaxf(x.m, y.m);
  const float ex = __builtin_amdgcn_exp2f(x.m - m), ey = __builtin_amdgcn_exp2f(y.m - m);
  MergeAcc r;
  r.m = m;
  r.l = __builtin_fmaf(x.l, ex, y.l * ey);
  r.a.x = __builtin_fmaf(x.a.x, ex, y.a.x * ey);
  r.a.y = __builtin_fmaf(x.a.y, ex, y.a.y * ey);
  r.a.z = __builtin_fmaf(x.a.z, ex, y.a.z * ey);
  r.a.w = __builtin_fmaf(x.a.w, ex, y.a.w * ey);
  return r;
}

// The value of lane + K, for the lanes where that lane is in the same group of
// 2K (the lanes whose bit K is clear); other lanes get an unspecified value.
// K < 16: a DPP move within the row of 16 lanes (quad_perm for 1 and 2,
// row_shl for 4 and 8); K = 16, 32: v_permlane16/32_swap.
template <int K>
__device__ __forceinline__ float lane_from_above(float x) {
  if constexpr (K == 16 || K == 32) {
    float a, b;  // a: the lower lane's value, b: the upper lane's, in both lanes
    if constexpr (K == 16)
      lane_pair16(x, a, b);
    else
      lane_pair32(x, a, b);
    return b;
  } else {
    constexpr int ctrl = K == 1   ? 0xB1    // quad_perm [1, 0, 3, 2]
                         : K == 2 ? 0x4E    // quad_perm [2, 3, 0, 1]
                                  : 0x100 + K;  // row_shl:K
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                         0, __builtin_bit_cast(int, x), ctrl, 0xF, 0xF, false));
  }
}

template <int K>
__device__ __forceinline__ MergeAcc acc_from_above(const MergeAcc& x) {
  MergeAcc r;
  r.m = lane_from_above<K>(x.m);
  r.l = lane_from_above<K>(x.l);
  r.a.x = lane_from_above<K>(x.a.x);
  r.a.y = lane_from_above<K>(x.a.y);
  r.a.z = lane_from_above<K>(x.a.z);
  r.a.w = lane_from_above<K>(x.a.w);
  return r;
}

// Levels K, 2K, ... below CL of the tree over a wave's block lanes.
template <int K, int CL>
__device__ __forceinline__ void lane_tree(MergeAcc& acc) {
  if constexpr (K < CL) {
    acc = merge_pair(acc, acc_from_above<K>(acc));
    lane_tree<2 * K, CL>(acc);
  }
}

// Q = dim quads per slice (16, 8, 4, 2 or 1 for S = 16 / Q = 1 .. 16 slices).
// One slice: blockIdx = (head, row). Several slices: a 1-D grid in which all
// slices of one (row, head) run on the same XCD. MI355X hands workgroup w to
// XCD w mod 8, so workgroup w = x + 8 j takes (row, head) pair x + 8 (j / S)
// and slice j % S. The slices share the 128-byte lines of their pair's
// partials and all of its (m, l) values; on one XCD those lines come from HBM
// once and from that XCD's L2 after, where slices spread over four XCDs
// fetched every line four times. Workgroups past the last pair leave at once.
// Where workgroups land changes no sum, only the traffic.
template <int Q>
__global__ void __launch_bounds__(64 * kMergeMaxWaves)
decode_merge_kernel(float* __restrict__ out, const float* __restrict__ part_o,
                    const float* __restrict__ part_ml, const int32_t* __restrict__ row_pos,
                    int T, int n_heads, int num_chunks, int chunk_tokens) {
  constexpr int HD = 64, CL = 64 / Q, S = 16 / Q;
  __shared__ MergeAcc red[kMergeMaxWaves][Q];
  int h, t, s;
  if constexpr (S == 1) {
    h = blockIdx.x;
    t = blockIdx.y;
    s = 0;
  } else {
    const int x = blockIdx.x & 7, j = blockIdx.x >> 3;
    const int pair = x + 8 * (j / S);
    if (pair >= T * n_heads) return;
    h = pair % n_heads;
    t = pair / n_heads;
    s = j % S;
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int qd = lane / CL, bl = lane % CL;
  const int p = row_pos[t];
  if (p < 0) return;
  const int nc = min(p / chunk_tokens + 1, num_chunks);
  if (nc <= 1) return;  // written by the partial kernel
  const size_t base = (size_t(t) * n_heads + h) * num_chunks;
  const int dim = s * 4 * Q + 4 * qd;
  const float2* ml = reinterpret_cast<const float2*>(part_ml) + base;
  const float4* po = reinterpret_cast<const float4*>(part_o + base * HD + dim);

  // This lane's block, folded in chunk order.
  const int b = w * CL + bl;
  const int c0 = b * kMergeBlock;
  float2 mlc[kMergeBlock];
  float4 oc[kMergeBlock];
#pragma unroll
  for (int j = 0; j < kMergeBlock; ++j) {
    const bool ok = c0 + j < nc;
    mlc[j] = ok ? ml[c0 + j] : make_float2(-INFINITY, 0.0f);
    oc[j] = ok ? po[size_t(c0 + j) * (HD / 4)] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  MergeAcc acc{-INFINITY, 0.0f, make_float4(0.0f, 0.0f, 0.0f, 0.0f)};
  float mb = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMergeBlock; ++j) mb = fmaxf(mb, mlc[j].x);
  if (mb != -INFINITY) {
    acc.m = mb;
#pragma unroll
    for (int j = 0; j < kMergeBlock; ++j) {
      const float e = mlc[j].x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mlc[j].x - mb);
      acc.l = __builtin_fmaf(mlc[j].y, e, acc.l);
      acc.a.x = __builtin_fmaf(oc[j].x, e, acc.a.x);
      acc.a.y = __builtin_fmaf(oc[j].y, e, acc.a.y);
      acc.a.z = __builtin_fmaf(oc[j].z, e, acc.a.z);
      acc.a.w = __builtin_fmaf(oc[j].w, e, acc.a.w);
    }
  }
  // Tree over the wave's blocks: the lanes with bl = 0 end up with the wave's node.
  lane_tree<1, CL>(acc);
  float4* dst = reinterpret_cast<float4*>(out + (size_t(t) * n_heads + h) * HD + dim);
  if (W > 1) {  // the tree continues over the waves, node (w, w + stride)
    if (bl == 0) red[w][qd] = acc;
    __syncthreads();
    for (int stride = 1; stride < W; stride <<= 1) {
      if (bl == 0 && (w & (2 * stride - 1)) == 0 && w + stride < W)
        red[w][qd] = merge_pair(red[w][qd], red[w + stride][qd]);
      __syncthreads();
    }
    if (w != 0) return;
    acc = red[0][qd];
  }
  if (bl == 0)
    *dst = make_float4(acc.a.x / acc.l, acc.a.y / acc.l, acc.a.z / acc.l, acc.a.w / acc.l);
}

template <int KV, int G>
int launch_valu(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, const Workspace& ws, int n_heads,
                int n_kv_heads, hipStream_t stream) {
  using E = typename Kv<KV>::elem;
  constexpr int HD = 64;
  const float scale = 1.0f / sqrtf(float(HD));
  const size_t lds = size_t(G) * chunk_tokens * sizeof(float);
  hipLaunchKernelGGL((decode_partial_valu<KV, HD, G>), dim3(T, n_kv_heads, num_chunks),
                     dim3(kThreads), lds, stream, out, ws.part_o, ws.part_ml, q,
                     static_cast<const E*>(k_pool), static_cast<const E*>(v_pool), row_pos, row_seq,
                     kv.tables, kv.max_pages, kv.num_pages, n_heads, n_kv_heads, num_chunks,
                     chunk_tokens, scale);
  if (int rc = check_launch("attention_partial")) return rc;
  return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
}

template <int KV>
int dispatch_group(int group, float* out, const float* q, const void* k_pool, const void* v_pool,
                   int T, const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                   int num_chunks, int chunk_tokens, const Workspace& ws, int n_heads,
                   int n_kv_heads, hipStream_t stream) {
  switch (group) {
#define IE_GROUP_CASE(G)                                                                           \
  case G:                                                                                          \
    return launch_valu<KV, G>(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks,        \
                              chunk_tokens, ws, n_heads, n_kv_heads, stream);
    IE_GROUP_CASE(1)
    IE_GROUP_CASE(2)
    IE_GROUP_CASE(3)
    IE_GROUP_CASE(4)
    IE_GROUP_CASE(5)
    IE_GROUP_CASE(6)
    IE_GROUP_CASE(7)
    IE_GROUP_CASE(8)
#undef IE_GROUP_CASE
  }
  return fail(IE_HIP_EINVAL, "attention: at most 8 query heads per KV head");
}

}  // namespace

int decode_merge(float* out, const Workspace& ws, const int32_t* row_pos, int T, int n_heads,
                 int num_chunks, int chunk_tokens, hipStream_t stream) {
  if (num_chunks <= 1) return IE_HIP_OK;
  // Dim slices: enough (head, row, slice) workgroups to reach every compute unit
  // when rows x heads alone cannot (long-context batches of a few rows), and
  // enough block lanes for the longest row: a wave holds 4 x slices blocks of
  // 8 chunks, a workgroup at most 16 waves. Neither choice changes the sums.
  const int64_t pairs = int64_t(T) * n_heads;
  const int cus = device_compute_units();
  int slices = pairs >= cus ? 1 : (2 * pairs >= cus ? 2 : 4);
  // Few rows: as many slices as make every workgroup one wave (up to 16), so
  // that the tree ends in registers, without the LDS stage and its barriers.
  if (pairs < cus)
    while (slices < 16 && 4 * slices * kMergeBlock < num_chunks) slices *= 2;
  while (slices < 16 && int64_t(kMergeMaxWaves) * 4 * slices * kMergeBlock < num_chunks)
    slices *= 2;
  const int blocks_per_wave = 4 * slices;
  const int blocks = (num_chunks + kMergeBlock - 1) / kMergeBlock;
  const int waves = (blocks + blocks_per_wave - 1) / blocks_per_wave;
  if (waves > kMergeMaxWaves)
    return fail(IE_HIP_EINVAL, "attention: more than 8,192 chunks per row");
  // Several slices: 8 XCD lanes x ceil(pairs / 8) pairs each x slices (see the kernel).
  const dim3 grid = slices == 1 ? dim3(n_heads, T) : dim3(8 * ((pairs + 7) / 8) * slices);
  const dim3 block(64 * waves);
#define IE_MERGE_CASE(S)                                                                     \
  case S:                                                                                    \
    hipLaunchKernelGGL((decode_merge_kernel<16 / S>), grid, block, 0, stream, out, ws.part_o, \
                       ws.part_ml, row_pos, T, n_heads, num_chunks, chunk_tokens);           \
    break;
  switch (slices) {
    IE_MERGE_CASE(1)
    IE_MERGE_CASE(2)
    IE_MERGE_CASE(4)
    IE_MERGE_CASE(8)
    IE_MERGE_CASE(16)
  }
#undef IE_MERGE_CASE
  return check_launch("attention_merge");
}

Workspace carve_workspace(void* base, int T, int n_heads, int head_dim, int num_chunks) {
  Workspace ws;
  char* p = static_cast<char*>(base);
  const size_t slots = size_t(T) * n_heads * num_chunks;
  ws.part_o = reinterpret_cast<float*>(p);
  p += align256(slots * head_dim * sizeof(float));
  ws.part_ml = reinterpret_cast<float*>(p);
  return ws;
}

size_t workspace_bytes(int T, int n_heads, int head_dim, int num_chunks) {
  const size_t slots = size_t(T) * n_heads * num_chunks;
  return align256(slots * head_dim * sizeof(float)) + align256(slots * 2 * sizeof(float));
}

int device_compute_units() {
  // Per device: the count of the device current on the calling thread, looked
  // up once per device (a launch on another device must not reuse another's).
  constexpr int kDevices = 64;
  static std::atomic<int> known[kDevices] = {};
  int dev = 0, n = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return 256;  // no device visible (host-only callers): MI355X's count
  }
  if (dev >= 0 && dev < kDevices && (n = known[dev].load(std::memory_order_relaxed)) > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      n <= 0) {
    (void)hipGetLastError();
    n = 256;
  }
  if (dev >= 0 && dev < kDevices) known[dev].store(n, std::memory_order_relaxed);
  return n;
}

int decode_valu(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream) {
  const int group = n_heads / n_kv_heads;
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  switch (kv.kv_dtype) {
    case IE_KV_F32:
      return dispatch_group<IE_KV_F32>(group, out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                       num_chunks, chunk_tokens, ws, n_heads, n_kv_heads, stream);
    case IE_KV_F16:
      return dispatch_group<IE_KV_F16>(group, out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                       num_chunks, chunk_tokens, ws, n_heads, n_kv_heads, stream);
    case IE_KV_BF16:
      return dispatch_group<IE_KV_BF16>(group, out, q, k_pool, v_pool, T, row_pos, row_seq, kv,
                                        num_chunks, chunk_tokens, ws, n_heads, n_kv_heads, stream);
  }
  return fail(IE_HIP_EINVAL, "attention: unsupported kv_dtype");
}

}  // namespace iehip

using namespace iehip;

extern "C" {

int ie_hip_attention_chunks(int context_tokens, int chunk_tokens) {
  if (context_tokens <= 0 || chunk_tokens <= 0) return 0;
  return (context_tokens + chunk_tokens - 1) / chunk_tokens;
}

int ie_hip_attention_chunk_tokens(int T, int max_context, int kv_dtype) {
  const int cus = device_compute_units();
  const int64_t rows = std::max(T, 1);
  const int ctx = std::max(max_context, 1);
  if (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) {
    // Matrix-core kernel (measured on MI355X): 192-position chunks where rows x
    // chunks at full context still reach 4 workgroups per compute unit (64 rows
    // of 4,096: 18.5 us per call against 19.5 at 256, 21.0 at 128, 25.1 at 512);
    // 64 where even 64-position chunks give at most two workgroups per compute
    // unit (one row of 32,768: 10.2 us per call against 10.5 at 128, the fused
    // decode layer 11.1 against 11.9; one row of 8,192: 7.9 against 9.4; 4 rows
    // of 4,096: 8.5 against 9.7); else 128 (2 rows of 32,768, 16 of 4,096: 13.1
    // and 12.7 us against 14.5 and 13.3 at 64; 48 rows of 2,049: 16.0 against
    // 18.6 at 64 and 16.0 at 192). Where the grid gives two workgroups per
    // compute unit one wave streams each chunk; on smaller grids each of a
    // chunk's page pairs gets its own wave (same result), so all are in flight
    // at once.
    if (rows * ie_hip_attention_chunks(ctx, 192) >= 4 * int64_t(cus)) return 192;
    return rows * ie_hip_attention_chunks(ctx, 64) <= 2 * int64_t(cus) ? 64 : 128;
  }
  // float32 (matrix-core kernel, one page in flight per wave; measured on
  // MI355X): 192 positions where that gives 4 workgroups per compute unit (64
  // rows of 4,096: 33.6 us per call at 192, 35.6 at 256, 40.5 at 128), else the
  // largest of 128 and 64 that still gives two (48 rows of 2,049: 25.0 us at 128
  // against 29.5 at 192; one row of 32,768: 64) -- long chains of pages per wave
  // where the grid is large, short ones where few rows must fill the device.
  if (rows * ie_hip_attention_chunks(ctx, 192) >= 4 * int64_t(cus)) return 192;
  for (int ct : {128, 64})
    if (rows * ie_hip_attention_chunks(ctx, ct) >= 2 * cus) return ct;
  return 32;
}

size_t ie_hip_attention_workspace_bytes(int T, int n_heads, int head_dim, int num_chunks) {
  if (T <= 0 || n_heads <= 0 || head_dim <= 0 || num_chunks <= 0) return 0;
  return workspace_bytes(T, n_heads, head_dim, num_chunks);
}

size_t ie_hip_attention_plan_ints(int T, int num_chunks, int chunk_tokens) {
  if (T <= 0 || num_chunks <= 0 || chunk_tokens < IE_HIP_PAGE_SIZE || chunk_tokens > 1024 ||
      chunk_tokens % IE_HIP_PAGE_SIZE)
    return 0;
  return plan_ints(T, num_chunks, chunk_tokens);
}

int ie_hip_attention_plan(int32_t* plan, size_t plan_capacity, int T, const int32_t* row_pos,
                          const int32_t* row_seq, const int32_t* tables, int max_seqs,
                          int max_pages, int num_chunks, int chunk_tokens) {
  clear_error();
  if (T < 0 || num_chunks <= 0 || max_seqs <= 0 || max_pages <= 0)
    return fail(IE_HIP_EINVAL, "attention_plan: bad row, chunk, sequence or page count");
  if (chunk_tokens < IE_HIP_PAGE_SIZE || chunk_tokens > 1024 || chunk_tokens % IE_HIP_PAGE_SIZE)
    return fail(IE_HIP_EINVAL, "attention_plan: chunk_tokens must be a multiple of 16 in [16, 1024]");
  if (!plan || (T > 0 && (!row_pos || !row_seq || !tables)))
    return fail(IE_HIP_EINVAL, "attention_plan: null pointer");
  const size_t need = plan_ints(std::max(T, 1), num_chunks, chunk_tokens);
  if (plan_capacity < need)
    return fail(IE_HIP_EINVAL, "attention_plan: the plan holds " + std::to_string(plan_capacity) +
                                   " ints; " + std::to_string(T) + " rows x " +
                                   std::to_string(num_chunks) + " chunks need " +
                                   std::to_string(need) + " (ie_hip_attention_plan_ints)");
  const int stride = plan_stride(chunk_tokens), pages = chunk_tokens / IE_HIP_PAGE_SIZE;
  // min(p / chunk + 1, num_chunks) chunks per row. Items in dispatch order:
  // longer chunks first -- every row's full chunks, then the shorter last
  // chunks, longest first -- each group in row and chunk order, so the short
  // workgroups fill the end of the launch instead of holding its start (the
  // order changes no result: every item writes its own (row, chunk) slot).
  struct Item {
    int n, t, c;  // positions in the chunk, row, chunk
  };
  std::vector<Item> order;
  for (int t = 0; t < T; ++t) {
    const int p = row_pos[t];
    if (p < 0) continue;
    const int seq = row_seq[t];
    if (seq < 0 || seq >= max_seqs)
      return fail(IE_HIP_EINVAL, "attention_plan: row " + std::to_string(t) + " has sequence " +
                                     std::to_string(seq) + " outside the table's " +
                                     std::to_string(max_seqs) + " rows");
    const int nc = std::min(p / chunk_tokens + 1, num_chunks);
    for (int c = 0; c < nc; ++c)
      order.push_back(Item{std::min(chunk_tokens, p + 1 - c * chunk_tokens), t, c});
  }
  std::stable_sort(order.begin(), order.end(),
                   [](const Item& a, const Item& b) { return a.n > b.n; });
  int items = 0;
  for (const Item& e : order) {
    const int t = e.t, c = e.c;
    const int p = row_pos[t], seq = row_seq[t];
    int32_t* it = plan + kPlanHeader + size_t(items) * stride;
    it[0] = t;
    it[1] = c;
    it[2] = p;
    it[3] = seq;
    for (int j = 0; j < stride - 4; ++j) {
      const int pi = c * pages + j;
      const bool in = j < pages && pi * IE_HIP_PAGE_SIZE <= p && pi < max_pages;
      it[4 + j] = in ? tables[size_t(seq) * max_pages + pi] : -1;
    }
    ++items;
  }
  plan[0] = items;
  plan[1] = chunk_tokens;
  plan[2] = num_chunks;
  plan[3] = T;
  return IE_HIP_OK;
}

}  // extern "C"

namespace {

int attention_call(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                   const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                   int num_chunks, int chunk_tokens, void* workspace, int n_heads,
                   int n_kv_heads, int head_dim, hipStream_t stream, const int32_t* plan) {
  if (int rc = check_layout(kv, "attention")) return rc;
  if (head_dim != 64) return fail(IE_HIP_EINVAL, "attention: head_dim must be 64");
  if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0 || n_heads / n_kv_heads > 8)
    return fail(IE_HIP_EINVAL, "attention: at most 8 query heads per KV head");
  if (chunk_tokens < IE_HIP_PAGE_SIZE || chunk_tokens > 1024 || chunk_tokens % IE_HIP_PAGE_SIZE)
    return fail(IE_HIP_EINVAL, "attention: chunk_tokens must be a multiple of 16 in [16, 1024]");
  if (num_chunks <= 0 || T < 0) return fail(IE_HIP_EINVAL, "attention: bad chunk or row count");
  if (T == 0) return IE_HIP_OK;
  if (!out || !q || !k_pool || !v_pool || !row_pos || !row_seq || !workspace)
    return fail(IE_HIP_EINVAL, "attention: null pointer");
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(workspace)) & 15)
    return fail(IE_HIP_EINVAL, "attention: out and the workspace must be 16-byte aligned");
  const int impl = attention_impl();
  if (impl != IE_HIP_IMPL_VALU &&
      decode_mfma_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim, chunk_tokens))
    return decode_mfma(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks, chunk_tokens,
                       workspace, n_heads, n_kv_heads, stream, nullptr, plan);
  if (impl != IE_HIP_IMPL_VALU &&
      decode_mfma_f32_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim, chunk_tokens))
    return decode_mfma_f32(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks,
                           chunk_tokens, workspace, n_heads, n_kv_heads, stream, plan);
  if (impl == IE_HIP_IMPL_MFMA)
    return fail(IE_HIP_EINVAL, "attention: the MFMA kernels do not support this shape "
                               "(kv_dim 128, n_heads <= 16; 16-bit KV: chunk a multiple of 64 "
                               "up to 1024; f32 KV: a multiple of 16 up to 1024)");
  return decode_valu(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks, chunk_tokens,
                     workspace, n_heads, n_kv_heads, stream);
}

int check_plan(const int32_t* plan, size_t plan_capacity, int T, int num_chunks, int chunk_tokens,
               const char* who) {
  if (!plan) return fail(IE_HIP_EINVAL, std::string(who) + ": null plan");
  if (reinterpret_cast<uintptr_t>(plan) & 15)
    return fail(IE_HIP_EINVAL, std::string(who) + ": the plan must be 16-byte aligned");
  const size_t need = ie_hip_attention_plan_ints(T, num_chunks, chunk_tokens);
  if (plan_capacity < need)
    return fail(IE_HIP_EINVAL, std::string(who) + ": the plan holds " +
                                   std::to_string(plan_capacity) + " ints, the grid needs " +
                                   std::to_string(need));
  return IE_HIP_OK;
}

}  // namespace

extern "C" {

int ie_hip_attention(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                     const int32_t* row_pos, const int32_t* row_seq, ie_kv_layout kv,
                     int num_chunks, int chunk_tokens, void* workspace, int n_heads,
                     int n_kv_heads, int head_dim, hipStream_t stream) {
  clear_error();
  return attention_call(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks, chunk_tokens,
                        workspace, n_heads, n_kv_heads, head_dim, stream, nullptr);
}

int ie_hip_attention_planned(float* out, const float* q, const void* k_pool, const void* v_pool,
                             int T, const int32_t* row_pos, const int32_t* row_seq,
                             ie_kv_layout kv, int num_chunks, int chunk_tokens, void* workspace,
                             const int32_t* plan, size_t plan_capacity, int n_heads,
                             int n_kv_heads, int head_dim, hipStream_t stream) {
  clear_error();
  if (T > 0)
    if (int rc = check_plan(plan, plan_capacity, T, num_chunks, chunk_tokens, "attention_planned"))
      return rc;
  return attention_call(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks, chunk_tokens,
                        workspace, n_heads, n_kv_heads, head_dim, stream, plan);
}

}  // extern "C"

// ------------------------------------------------- no-allocation variant ---
// ie_hip_attention for callers that cannot allocate (HIP graph capture, tight
// serving loops): the split-K partials go to `scratch`, a fixed device array of
// IE_HIP_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds until
// the process ends. Host code never passes `scratch` itself (its name is a host
// stand-in, not a device address): the first call on a device looks up that
// device's copy with hipGetSymbolAddress, once, and every later call passes
// the address kept for it. The partials need no initialisation (a call reads
// only the slots it wrote), so nothing is cleared. Calls that overlap on one
// GPU share the array and race.
static __device__ __align__(256) unsigned char scratch[IE_HIP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

int scratch_address(void** out) {
  static std::mutex mu;
  static void* addr[kMaxDevices] = {};
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "attention_noalloc: hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices)
    return fail(IE_HIP_EINVAL, "attention_noalloc: device index above 63");
  std::lock_guard<std::mutex> lock(mu);
  if (!addr[dev]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                           "attention_noalloc: hipGetSymbolAddress(scratch)"))
      return rc;
    addr[dev] = p;
  }
  *out = addr[dev];
  return IE_HIP_OK;
}

}  // namespace

extern "C" int ie_hip_attention_noalloc(float* out, const float* q, const void* k_pool,
                                        const void* v_pool, int T, const int32_t* row_pos,
                                        const int32_t* row_seq, ie_kv_layout kv, int num_chunks,
                                        int chunk_tokens, int n_heads, int n_kv_heads,
                                        int head_dim, hipStream_t stream) {
  clear_error();
  if (T < 0 || num_chunks <= 0 || n_heads <= 0 || head_dim <= 0)
    return fail(IE_HIP_EINVAL, "attention_noalloc: bad row, chunk or head count");
  if (T == 0) return IE_HIP_OK;
  const size_t need = workspace_bytes(T, n_heads, head_dim, num_chunks);
  if (need > IE_HIP_NOALLOC_SCRATCH_BYTES)
    return fail(IE_HIP_EINVAL,
                "attention_noalloc: " + std::to_string(T) + " rows x " + std::to_string(n_heads) +
                    " heads x " + std::to_string(num_chunks) + " chunks need " +
                    std::to_string(need) + " bytes of split-K scratch; the fixed scratch holds " +
                    std::to_string(size_t(IE_HIP_NOALLOC_SCRATCH_BYTES)) +
                    " (use ie_hip_attention with a workspace)");
  void* ws = nullptr;
  if (int rc = scratch_address(&ws)) return rc;
  return ie_hip_attention(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks,
                          chunk_tokens, ws, n_heads, n_kv_heads, head_dim, stream);
}

extern "C" {

static bool fused_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                            int chunk_tokens) {
  return attention_impl() != IE_HIP_IMPL_VALU &&
         decode_mfma_supported(kv_dtype, n_heads, n_kv_heads, head_dim, chunk_tokens);
}

int ie_hip_rope_cache_attention_supported(int kv_dtype, int n_heads, int n_kv_heads,
                                          int head_dim, int chunk_tokens) {
  return fused_supported(kv_dtype, n_heads, n_kv_heads, head_dim, chunk_tokens) ? 1 : 0;
}

static int rope_cache_attention_call(float* out, const float* q, const float* k, const float* v,
                                     void* k_pool, void* v_pool, const float* rope_table,
                                     int table_positions, int T, const int32_t* row_pos,
                                     const int32_t* row_seq, const ie_kv_layout& kv,
                                     int num_chunks, int chunk_tokens, void* workspace,
                                     int n_heads, int n_kv_heads, int head_dim,
                                     hipStream_t stream, const int32_t* plan) {
  if (int rc = check_layout(kv, "rope_cache_attention")) return rc;
  if (n_kv_heads <= 0 || n_heads <= 0 || n_heads % n_kv_heads != 0)
    return fail(IE_HIP_EINVAL, "rope_cache_attention: bad head counts");
  if (num_chunks <= 0 || T < 0) return fail(IE_HIP_EINVAL, "rope_cache_attention: bad chunk or row count");
  if (table_positions <= 0) return fail(IE_HIP_EINVAL, "rope_cache_attention: empty RoPE table");
  if (!fused_supported(kv.kv_dtype, n_heads, n_kv_heads, head_dim, chunk_tokens))
    return fail(IE_HIP_EINVAL,
                "rope_cache_attention: needs a 16-bit KV cache and the matrix-core decode shapes "
                "(head_dim 64, kv_dim 128, n_heads <= 16, chunk a multiple of 64 up to 1024); "
                "use ie_hip_rope_and_cache + ie_hip_attention");
  if (T == 0) return IE_HIP_OK;
  if (!out || !q || !k || !v || !k_pool || !v_pool || !rope_table || !row_pos || !row_seq ||
      !workspace)
    return fail(IE_HIP_EINVAL, "rope_cache_attention: null pointer");
  if ((reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(workspace) |
       reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
       reinterpret_cast<uintptr_t>(rope_table)) & 15)
    return fail(IE_HIP_EINVAL,
                "rope_cache_attention: out, k, v, the table and the workspace must be 16-byte "
                "aligned");
  FusedAppend fa;
  fa.k = k;
  fa.v = v;
  fa.k_pool = static_cast<uint16_t*>(k_pool);
  fa.v_pool = static_cast<uint16_t*>(v_pool);
  fa.table = rope_table;
  fa.table_positions = table_positions;
  return decode_mfma(out, q, k_pool, v_pool, T, row_pos, row_seq, kv, num_chunks, chunk_tokens,
                     workspace, n_heads, n_kv_heads, stream, &fa, plan);
}

int ie_hip_rope_cache_attention(float* out, const float* q, const float* k, const float* v,
                                void* k_pool, void* v_pool, const float* rope_table,
                                int table_positions, int T, const int32_t* row_pos,
                                const int32_t* row_seq, ie_kv_layout kv, int num_chunks,
                                int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                                int head_dim, hipStream_t stream) {
  clear_error();
  return rope_cache_attention_call(out, q, k, v, k_pool, v_pool, rope_table, table_positions, T,
                                   row_pos, row_seq, kv, num_chunks, chunk_tokens, workspace,
                                   n_heads, n_kv_heads, head_dim, stream, nullptr);
}

int ie_hip_rope_cache_attention_planned(float* out, const float* q, const float* k,
                                        const float* v, void* k_pool, void* v_pool,
                                        const float* rope_table, int table_positions, int T,
                                        const int32_t* row_pos, const int32_t* row_seq,
                                        ie_kv_layout kv, int num_chunks, int chunk_tokens,
                                        void* workspace, const int32_t* plan,
                                        size_t plan_capacity, int n_heads, int n_kv_heads,
                                        int head_dim, hipStream_t stream) {
  clear_error();
  if (T > 0)
    if (int rc = check_plan(plan, plan_capacity, T, num_chunks, chunk_tokens,
                            "rope_cache_attention_planned"))
      return rc;
  return rope_cache_attention_call(out, q, k, v, k_pool, v_pool, rope_table, table_positions, T,
                                   row_pos, row_seq, kv, num_chunks, chunk_tokens, workspace,
                                   n_heads, n_kv_heads, head_dim, stream, plan);
}

}  // extern "C"
