// Flash-decoding attention over pages on the matrix cores (gfx950), for f16
// and bf16 KV caches whose rows hold 128 elements (2 KV heads x 64) and at
// most 16 query heads -- Qwen2.5-0.5B: 14 query heads, 2 KV heads.
//
// Reference semantics: each row's causal GQA attention, src/ops.cpp:70-108;
// split-K chunks merged by log-sum-exp as in src/cuda/kernels.cu:309-507.
//
// Why MFMA for decode: every KV row is used by all 7 query heads of its group,
// so per 16-token page the work is two dense products,
//     S^T[16 tok x 16 heads] = K_page[16 x 128] . Qbd^T[128 x 16]
//     O[16 heads x 128]     += P[16 heads x 32 tok] . V_pair[32 tok x 128]
// where Qbd is block-diagonal: head h carries its query in the 64 dims of its
// own KV head and zeros elsewhere, so ONE 16-row tile serves all 14 heads of
// both KV heads and each K/V row is read exactly once. On the VALU the same
// work costs ~1,800 FMAs per position -- as much time as streaming the cache.
// The only extra work is the off-diagonal half of O, discarded at the end.
//
// Precision (2e-3 absolute bound for 16-bit caches): K and V enter the MFMA in
// their stored format, exactly. Q (pre-scaled by 1/8, exact) and P are split
// into hi + lo halves of the same 16-bit type (x = hi + lo, |x - hi - lo| ~
// 2^-22 |x|), each product done twice: float32-level scores and weights.
//
// Layout of the work:
//   grid (T, num_chunks), rows fastest; chunk_tokens / 64 (<= 8) waves per workgroup,
//   each wave owns 64 consecutive positions = 4 pages = 2 page pairs.
//   1. All K and V loads of the wave are issued first (one memory round trip).
//      K goes straight into the MFMA A-operand registers (4 x 16-byte loads per
//      page; lanes 0-15 hold tokens 0-15, the 4 lane groups hold the 4 16-byte
//      slices of each 64-byte quarter row). 8 MFMA 16x16x32 per page.
//   2. softmax over the chunk: wave-local max/sum by shuffles, across waves
//      through LDS (scores kept in registers; base-2 exponent).
//   3. V: each page pair (8 KB) is staged in a per-wave LDS tile with 16-byte
//      coalesced loads and read back transposed (one 2-byte element per lane per
//      slot) as the B operand; 16 MFMA 16x16x32 per pair.
//   4. O: per-wave tiles summed through LDS; a row whose context fits one chunk
//      writes `out` directly, otherwise the chunk writes (o, m, l) and the last
//      chunk of the row to finish merges them (atomic counter per row in the
//      workspace, reset by that chunk): one launch, no separate merge kernel.
#include <cstdlib>

#include "common.hpp"
#include "decode.hpp"

namespace iehip {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kKvd = 128;                 // elements per KV row (n_kv_heads * 64)
constexpr int kWaveTokens = 128;          // positions per wave: 8 pages = 4 page pairs
constexpr int kWavePages = kWaveTokens / IE_HIP_PAGE_SIZE;
constexpr int kWaveLds = 8192;            // per-wave LDS: one V page-pair tile, then the O tile
// How chunk partials are combined.
constexpr int kMergeKernel = 0;    // a separate merge kernel
constexpr int kMergeFence = 1;     // fused: last chunk merges; device-scope fences
constexpr int kMergeCoherent = 2;  // fused: last chunk merges; device-coherent stores/loads
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxWaves = 4;
constexpr int kMaxLds = kMaxWaves * (kWaveLds + 16 * 2 * 4);

template <int KV>
struct Mfma;

template <>
struct Mfma<IE_KV_F16> {
  using op = f16x8;
  using elem = _Float16;
  __device__ __forceinline__ static f32x4 mma(op a, op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<IE_KV_BF16> {
  using op = bf16x8;
  using elem = __bf16;
  __device__ __forceinline__ static f32x4 mma(op a, op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// Wave-local pieces of the kernel, one page pair (32 positions) at a time.
template <int KV>
struct PairIo {
  using op = typename Mfma<KV>::op;
  op k[2][4];   // K of the pair's two pages, A-operand layout
  uint4 v[8];   // V of the pair in coalesced 16-byte pieces
};

// Issues the loads of one page pair (pages p0, p1) into `io`.
template <int KV>
__device__ __forceinline__ void load_pair(PairIo<KV>& io, const uint16_t* __restrict__ k_pool,
                                          const uint16_t* __restrict__ v_pool, int p0, int p1,
                                          int lane) {
  using op = typename Mfma<KV>::op;
  const int g = lane >> 4, r = lane & 15;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int tok = 4 * u + (lane >> 4), piece = lane & 15;  // 0..31 within the pair
    io.v[u] = *reinterpret_cast<const uint4*>(
        v_pool + (size_t(tok < 16 ? p0 : p1) * IE_HIP_PAGE_SIZE + (tok & 15)) * kKvd + 8 * piece);
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const uint16_t* krow = k_pool + (size_t(h ? p1 : p0) * IE_HIP_PAGE_SIZE + r) * kKvd + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) io.k[h][ks] = *reinterpret_cast<const op*>(krow + 32 * ks);
  }
}

template <int KV>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 2)))
decode_partial_mfma(float* __restrict__ out, float* __restrict__ part_o,
                    float* __restrict__ part_ml, int32_t* __restrict__ counters,
                    const float* __restrict__ q, const uint16_t* __restrict__ k_pool,
                    const uint16_t* __restrict__ v_pool, const int32_t* __restrict__ row_pos,
                    const int32_t* __restrict__ row_seq, const int32_t* __restrict__ tables,
                    int max_pages, int num_pages, int n_heads, int group, int num_chunks,
                    int chunk_tokens, int merge_mode) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ int s_last;
  const int waves = blockDim.x >> 6;
  float* red_m = reinterpret_cast<float*>(smem + size_t(waves) * kWaveLds);
  float* red_l = red_m + waves * 16;

  const int t = blockIdx.x, c = blockIdx.y;
  const int p = row_pos[t];
  const int s0 = c * chunk_tokens;
  if (p < 0 || s0 > p) return;  // future chunk: the whole workgroup leaves
  const int n = min(s0 + chunk_tokens, p + 1) - s0;
  const int chunks_row = min(p / chunk_tokens + 1, num_chunks);
  const int seq = row_seq[t];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;
  const int wt0 = wave * kWaveTokens;  // first position of this wave within the chunk
  const int wn = min(max(n - wt0, 0), kWaveTokens);  // this wave's positions
  const int npairs = (wn + 31) / 32;                  // wave-uniform
  E* vt = reinterpret_cast<E*>(smem + size_t(wave) * kWaveLds);

  // Page ids of this wave's pages; a page past the context or outside the pool
  // is replaced by the wave's first page (read again from cache, then masked).
  int page[kWavePages];
  bool page_ok[kWavePages];
  {
    const int32_t* row_tab = tables + size_t(seq) * max_pages;
    int first_page = 0;
#pragma unroll
    for (int pg = 0; pg < kWavePages; ++pg) {
      const int first = wt0 + 16 * pg;
      const int pi = (s0 + first) / IE_HIP_PAGE_SIZE;
      int id = -1;
      if (first < n && pi < max_pages) id = row_tab[pi];
      page_ok[pg] = id >= 0 && id < num_pages;
      page[pg] = id;
      if (pg == 0 && page_ok[0]) first_page = id;
    }
#pragma unroll
    for (int pg = 0; pg < kWavePages; ++pg)
      if (!page_ok[pg]) page[pg] = first_page;
  }

  // Two page pairs in flight from the start; each later pair is requested as
  // soon as the registers of the pair two steps back are free.
  PairIo<KV> io[2];
  if (npairs > 0) load_pair<KV>(io[0], k_pool, v_pool, page[0], page[1], lane);
  if (npairs > 1) load_pair<KV>(io[1], k_pool, v_pool, page[2], page[3], lane);

  // Block-diagonal query tile as the B operand, hi + lo: lane (g, r) holds
  // head r's query (times 1/8) at dims [32 ks + 8 g, +8) of the KV row when
  // those dims belong to head r's KV head, zeros otherwise.
  op qhi[4], qlo[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int d0 = 32 * ks + 8 * g;
    const int kvh = d0 / 64;
    const bool mine = r < n_heads && r / group == kvh;
    float x[8];
    if (mine) {
      const float4* src =
          reinterpret_cast<const float4*>(q + (size_t(t) * n_heads + r) * 64 + (d0 - 64 * kvh));
      const float4 a = src[0], b = src[1];
      x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
      x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) x[j] = 0.0f;
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const float v = x[j] * 0.125f;
      const E hi = static_cast<E>(v);
      qhi[ks][j] = hi;
      qlo[ks][j] = static_cast<E>(v - static_cast<float>(hi));
    }
  }

  // Online softmax over the wave's pairs: running max m (base 2), sum l, O.
  float m_run = -INFINITY, l_run = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int pp = 0; pp < kWavePages / 2; ++pp) {
    if (pp < npairs) {
      PairIo<KV>& cur = io[pp & 1];
      // S^T of the pair's two pages: lane (g, r) gets tokens 4g..4g+3, head r.
      f32x4 s[2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        s[h] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          s[h] = M::mma(cur.k[h][ks], qhi[ks], s[h]);
          s[h] = M::mma(cur.k[h][ks], qlo[ks], s[h]);
        }
      }
      float mloc = -INFINITY;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int pg = 2 * pp + h;
          const int tok = wt0 + 16 * pg + 4 * g + i;
          const float v = (page_ok[pg] && tok < n) ? s[h][i] * kLog2e : -INFINITY;
          s[h][i] = v;
          mloc = fmaxf(mloc, v);
        }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float m_new = fmaxf(m_run, mloc);
      // rows of O belong to heads 4g+i: fetch their rescale factors from lane 4g+i
      const float corr = m_new == -INFINITY ? 1.0f : exp2f(m_run - m_new);
      m_run = m_new;
      op phi, plo;
      float lsum = 0.0f;
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float e = m_new == -INFINITY ? 0.0f : exp2f(s[h][i] - m_new);
          lsum += e;
          const E hi = static_cast<E>(e);
          phi[4 * h + i] = hi;
          plo[4 * h + i] = static_cast<E>(e - static_cast<float>(hi));
        }
      lsum += __shfl_xor(lsum, 16, 64);
      lsum += __shfl_xor(lsum, 32, 64);
      l_run = l_run * corr + lsum;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ci = __shfl(corr, 4 * g + i, 64);
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) o[nt][i] *= ci;
      }
      // V of the pair through the wave's LDS tile (swizzled: 16-byte piece k of
      // row `tok` at slot k ^ 2*((tok >> 2) & 3)), read back transposed.
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int tok = 4 * u + (lane >> 4), piece = lane & 15;
        const int slot = piece ^ (2 * ((tok >> 2) & 3));
        *reinterpret_cast<uint4*>(vt + tok * kKvd + 8 * slot) = cur.v[u];
      }
      // the pair two steps ahead may now reuse these registers
      if (pp + 2 < npairs) {
        __builtin_amdgcn_sched_barrier(0);
        load_pair<KV>(cur, k_pool, v_pool, page[2 * pp + 4], page[2 * pp + 5], lane);
        __builtin_amdgcn_sched_barrier(0);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        op b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int tok = (j < 4) ? (4 * g + j) : (16 + 4 * g + j - 4);
          const int slot = (2 * nt + (r >> 3)) ^ (2 * ((tok >> 2) & 3));
          b[j] = vt[tok * kKvd + slot * 8 + (r & 7)];
        }
        o[nt] = M::mma(phi, b, o[nt]);
        o[nt] = M::mma(plo, b, o[nt]);
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // Per-wave O tile [16 heads][128] floats into the wave's own LDS area, per-wave
  // (m, l); then the waves are merged for the diagonal blocks (head h, its KV
  // head's 64 dims).
  float* ot = reinterpret_cast<float*>(smem + size_t(wave) * kWaveLds);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) ot[(4 * g + i) * kKvd + 16 * nt + r] = o[nt][i];
  if (g == 0) {
    red_m[wave * 16 + r] = m_run;
    red_l[wave * 16 + r] = l_run;
  }
  __syncthreads();
  for (int idx = tid; idx < n_heads * 64; idx += blockDim.x) {
    const int h = idx >> 6, d = idx & 63;
    const int col = (h / group) * 64 + d;
    float mx = -INFINITY;
    for (int w = 0; w < waves; ++w) mx = fmaxf(mx, red_m[w * 16 + h]);
    float acc = 0.0f, l = 0.0f;
    for (int w = 0; w < waves; ++w) {
      const float mwh = red_m[w * 16 + h];
      if (mwh == -INFINITY) continue;  // a wave with no positions
      const float sc = exp2f(mwh - mx);
      acc = __builtin_fmaf(reinterpret_cast<const float*>(smem + size_t(w) * kWaveLds)[h * kKvd + col],
                           sc, acc);
      l = __builtin_fmaf(red_l[w * 16 + h], sc, l);
    }
    const size_t head = size_t(t) * n_heads + h;
    if (chunks_row == 1) {
      out[head * 64 + d] = acc / l;
    } else {
      const size_t slot = head * num_chunks + c;
      if (merge_mode == kMergeCoherent) {  // written through to the device coherence point
        __hip_atomic_store(part_o + slot * 64 + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (d == 0) {
          __hip_atomic_store(part_ml + 2 * slot, mx * kLn2, __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_AGENT);
          __hip_atomic_store(part_ml + 2 * slot + 1, l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      } else {
        part_o[slot * 64 + d] = acc;
        if (d == 0) {
          part_ml[2 * slot] = mx * kLn2;  // natural-log units
          part_ml[2 * slot + 1] = l;
        }
      }
    }
  }
  if (chunks_row == 1 || merge_mode == kMergeKernel) return;

  // 5. Merge, fused: the last chunk of the row to finish combines all chunks
  //    (M = max m_c, L = sum l_c e^(m_c - M), out = sum o_c e^(m_c - M) / L) and
  //    resets the row's counter for the next launch.
  //    kMergeFence: release/acquire fences at device scope (these write back and
  //      invalidate the XCD's whole L2).
  //    kMergeCoherent: partials are stored and loaded with device-scope relaxed
  //      atomics (coherent at the device level, no L2 flush); the stores are
  //      waited for before the counter is bumped, and the merging workgroup only
  //      loads them after it has seen the final count.
  if (merge_mode == kMergeFence) {
    __threadfence();
  } else {
    __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores are complete
  }
  __syncthreads();
  if (tid == 0) {
    const int done = merge_mode == kMergeFence
                         ? __hip_atomic_fetch_add(counters + t, 1, __ATOMIC_ACQ_REL,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                         : __hip_atomic_fetch_add(counters + t, 1, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
    s_last = done == chunks_row - 1;
  }
  __syncthreads();
  if (!s_last) return;
  if (merge_mode == kMergeFence) __threadfence();
  for (int idx = tid; idx < n_heads * 64; idx += blockDim.x) {
    const int h = idx >> 6, d = idx & 63;
    const size_t base = (size_t(t) * n_heads + h) * num_chunks;
    auto ld = [&](const float* ptr) {
      return merge_mode == kMergeFence
                 ? *ptr
                 : __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    float mx = -INFINITY;
    for (int cc = 0; cc < chunks_row; ++cc) mx = fmaxf(mx, ld(part_ml + 2 * (base + cc)));
    float L = 0.0f, acc = 0.0f;
    for (int cc = 0; cc < chunks_row; ++cc) {
      const float w = expf(ld(part_ml + 2 * (base + cc)) - mx);
      L = __builtin_fmaf(ld(part_ml + 2 * (base + cc) + 1), w, L);
      acc = __builtin_fmaf(ld(part_o + (base + cc) * 64 + d), w, acc);
    }
    out[(size_t(t) * n_heads + h) * 64 + d] = acc / L;
  }
  if (tid == 0) __hip_atomic_store(counters + t, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

bool decode_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                           int chunk_tokens) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) && head_dim == 64 &&
         n_kv_heads * head_dim == kKvd && n_heads <= 16 &&
         n_heads % n_kv_heads == 0 && chunk_tokens % kWaveTokens == 0 &&
         chunk_tokens >= kWaveTokens && chunk_tokens <= kMaxWaves * kWaveTokens;
}

int decode_mfma(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream) {
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  const int waves = chunk_tokens / kWaveTokens;
  const size_t lds = size_t(waves) * (kWaveLds + 16 * 2 * sizeof(float));
  const dim3 grid(T, num_chunks), block(64 * waves);
  static const int mode = [] {
    const char* e = getenv("IE_HIP_DECODE_MERGE");
    return e ? atoi(e) : kMergeKernel;
  }();
  const int group = n_heads / n_kv_heads;
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  // Keep the dynamic-LDS cap explicit (4 waves use 33 KB).
  static const hipError_t attr_f16 = hipFuncSetAttribute(
      reinterpret_cast<const void*>(decode_partial_mfma<IE_KV_F16>),
      hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
  static const hipError_t attr_bf16 = hipFuncSetAttribute(
      reinterpret_cast<const void*>(decode_partial_mfma<IE_KV_BF16>),
      hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);
  if (int rc = check_hip(kv.kv_dtype == IE_KV_F16 ? attr_f16 : attr_bf16,
                         "hipFuncSetAttribute(attention_partial_mfma)"))
    return rc;
  if (kv.kv_dtype == IE_KV_F16)
    hipLaunchKernelGGL(decode_partial_mfma<IE_KV_F16>, grid, block, lds, stream, out, ws.part_o,
                       ws.part_ml, ws.counters, q, kp, vp, row_pos, row_seq, kv.tables,
                       kv.max_pages, kv.num_pages, n_heads, group, num_chunks, chunk_tokens,
                       mode);
  else
    hipLaunchKernelGGL(decode_partial_mfma<IE_KV_BF16>, grid, block, lds, stream, out, ws.part_o,
                       ws.part_ml, ws.counters, q, kp, vp, row_pos, row_seq, kv.tables,
                       kv.max_pages, kv.num_pages, n_heads, group, num_chunks, chunk_tokens,
                       mode);
  if (int rc = check_launch("attention_mfma")) return rc;
  if (mode == kMergeKernel)
    return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
  return IE_HIP_OK;
}

}  // namespace iehip
