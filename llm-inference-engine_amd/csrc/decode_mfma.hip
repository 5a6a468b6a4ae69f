// Flash-decoding attention over pages on the matrix cores (gfx950), for f16
// and bf16 KV caches whose rows hold at most 128 elements (n_kv_heads * 64)
// and at most 16 query heads -- Qwen2.5-0.5B: 14 query heads, 2 KV heads.
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
//   1. K: each lane loads its token row's 16-byte pieces straight into the MFMA
//      A-operand registers (4 x global_load_dwordx4 per page; lanes 0-15 hold
//      tokens 0-15, the 4 lane groups hold the 4 16-byte slices of each 64-byte
//      quarter row). 8 MFMA 16x16x32 per page.
//   2. softmax over the chunk: wave-local max/sum by shuffles, across waves
//      through LDS (scores kept in registers; base-2 exponent).
//   3. V: each page pair (8 KB) is staged in a per-wave LDS tile with 16-byte
//      coalesced loads and read back transposed (one 2-byte element per lane per
//      slot) as the B operand; 16 MFMA 16x16x32 per pair.
//   4. O: per-wave tiles summed through LDS; a row whose context fits one chunk
//      writes `out` directly, otherwise the chunk writes (o, m, l) for the merge.
#include "common.hpp"
#include "decode.hpp"

namespace iehip {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kKvd = 128;                 // elements per KV row (n_kv_heads * 64)
constexpr int kVStride = kKvd + 4;        // LDS row stride of a staged V pair (halfs)
constexpr int kVTileHalfs = 32 * kVStride;  // one page pair
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxLds = 8 * (kVTileHalfs * 2 + 16 * 2 * 4);  // 8 waves

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

template <int KV>
__global__ void __launch_bounds__(512)
decode_partial_mfma(float* __restrict__ out, float* __restrict__ part_o,
                    float* __restrict__ part_ml, const float* __restrict__ q,
                    const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
                    const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                    const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
                    int group, int kv_dim, int num_chunks, int chunk_tokens) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  extern __shared__ __align__(16) unsigned char smem[];
  const int waves = blockDim.x >> 6;
  // LDS: per-wave V tile / O tile, then per-wave head maxima and sums.
  E* vtile_all = reinterpret_cast<E*>(smem);
  float* red_m = reinterpret_cast<float*>(smem + size_t(waves) * kVTileHalfs * sizeof(E));
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
  const int wt0 = wave * 64;  // first position of this wave within the chunk
  const int ks_count = kv_dim / 32;

  // Page ids of this wave's 4 pages; pages past the context (or outside the
  // pool) are not loaded, and their positions are masked.
  int page[4];
  bool page_ok[4];
#pragma unroll
  for (int pg = 0; pg < 4; ++pg) {
    const int first = wt0 + 16 * pg;
    const int pi = (s0 + first) / IE_HIP_PAGE_SIZE;
    int id = -1;
    if (first < n && pi < max_pages) id = tables[size_t(seq) * max_pages + pi];
    page_ok[pg] = id >= 0 && id < num_pages;
    page[pg] = page_ok[pg] ? id : 0;
  }

  // Block-diagonal query tile as the B operand, hi + lo: lane (g, r) holds
  // head r's query (times 1/8) at dims [32 ks + 8 g, +8) of the KV row when
  // those dims belong to head r's KV head, zeros otherwise.
  op qhi[4], qlo[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int d0 = 32 * ks + 8 * g;
    const int kvh = d0 / 64;
    const bool mine = ks < ks_count && r < n_heads && r / group == kvh;
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

  // 1. S^T per page: lane (g, r) gets tokens 4g..4g+3 of the page for head r.
  f32x4 s[4];
#pragma unroll
  for (int pg = 0; pg < 4; ++pg) {
    s[pg] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (page_ok[pg]) {
      const uint16_t* krow = k_pool + (size_t(page[pg]) * IE_HIP_PAGE_SIZE + r) * kv_dim + 8 * g;
      op ka[4];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        if (ks < ks_count) ka[ks] = *reinterpret_cast<const op*>(krow + 32 * ks);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        if (ks < ks_count) {
          s[pg] = M::mma(ka[ks], qhi[ks], s[pg]);
          s[pg] = M::mma(ka[ks], qlo[ks], s[pg]);
        }
      }
    }
  }

  // 2. Softmax statistics per head (base 2).
  float mloc = -INFINITY;
#pragma unroll
  for (int pg = 0; pg < 4; ++pg)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int tok = wt0 + 16 * pg + 4 * g + i;
      const float v = (page_ok[pg] && tok < n) ? s[pg][i] * kLog2e : -INFINITY;
      s[pg][i] = v;
      mloc = fmaxf(mloc, v);
    }
  mloc = fmaxf(mloc, __shfl_xor(mloc, 16, 64));
  mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
  if (g == 0) red_m[wave * 16 + r] = mloc;
  __syncthreads();
  float m2 = -INFINITY;
  for (int w = 0; w < waves; ++w) m2 = fmaxf(m2, red_m[w * 16 + r]);

  op phi[2], plo[2];  // A operands of the two page pairs
  float lsum = 0.0f;
#pragma unroll
  for (int pg = 0; pg < 4; ++pg)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = exp2f(s[pg][i] - m2);  // masked: exp2(-inf) = 0
      lsum += e;
      const E hi = static_cast<E>(e);
      phi[pg >> 1][(pg & 1) * 4 + i] = hi;
      plo[pg >> 1][(pg & 1) * 4 + i] = static_cast<E>(e - static_cast<float>(hi));
    }
  lsum += __shfl_xor(lsum, 16, 64);
  lsum += __shfl_xor(lsum, 32, 64);
  if (g == 0) red_l[wave * 16 + r] = lsum;

  // 3. O += P V, one page pair at a time through this wave's LDS tile.
  E* vt = vtile_all + size_t(wave) * kVTileHalfs;
  f32x4 o[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int row_chunks = kv_dim / 8;  // 16-byte pieces per KV row
#pragma unroll
  for (int pp = 0; pp < 2; ++pp) {
    if (pp) __syncthreads();  // every lane has read the previous pair's tile
    // stage: 32 rows x kv_dim, lane-contiguous 16-byte pieces
    for (int id = lane; id < 32 * row_chunks; id += 64) {
      const int tok = id / row_chunks, piece = id % row_chunks;
      const int pg = 2 * pp + tok / 16;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (page_ok[pg])
        val = *reinterpret_cast<const uint4*>(
            v_pool + (size_t(page[pg]) * IE_HIP_PAGE_SIZE + tok % 16) * kv_dim + 8 * piece);
      uint2* dst = reinterpret_cast<uint2*>(vt + tok * kVStride + 8 * piece);
      dst[0] = make_uint2(val.x, val.y);
      dst[1] = make_uint2(val.z, val.w);
    }
    __syncthreads();
    // B operand slot j of lane group g holds pair token 4g+j (j<4) or 16+4g+j-4.
#pragma unroll
    for (int nt = 0; nt < 8; ++nt) {
      if (nt * 16 < kv_dim) {
        op b;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int tok = (j < 4) ? (4 * g + j) : (16 + 4 * g + j - 4);
          b[j] = vt[tok * kVStride + 16 * nt + r];
        }
        o[nt] = M::mma(phi[pp], b, o[nt]);
        o[nt] = M::mma(plo[pp], b, o[nt]);
      }
    }
  }
  __syncthreads();  // V tiles are free: reuse them for the O tiles

  // 4. Per-wave O tiles -> LDS [wave][16 heads][kv_dim] floats, then summed.
  float* ot = reinterpret_cast<float*>(vtile_all) + size_t(wave) * 16 * kKvd;
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
    if (nt * 16 < kv_dim)
#pragma unroll
      for (int i = 0; i < 4; ++i) ot[(4 * g + i) * kKvd + 16 * nt + r] = o[nt][i];
  __syncthreads();
  const float* ot_all = reinterpret_cast<const float*>(vtile_all);
  for (int idx = tid; idx < n_heads * 64; idx += blockDim.x) {
    const int h = idx >> 6, d = idx & 63;
    const int col = (h / group) * 64 + d;
    float acc = 0.0f, l = 0.0f;
    for (int w = 0; w < waves; ++w) {
      acc += ot_all[(size_t(w) * 16 + h) * kKvd + col];
      l += red_l[w * 16 + h];
    }
    const size_t head = size_t(t) * n_heads + h;
    if (chunks_row == 1) {
      out[head * 64 + d] = acc / l;
    } else {
      const size_t slot = head * num_chunks + c;
      part_o[slot * 64 + d] = acc;
      if (d == 0) {
        float mm = -INFINITY;
        for (int w = 0; w < waves; ++w) mm = fmaxf(mm, red_m[w * 16 + h]);
        part_ml[2 * slot] = mm * kLn2;  // natural-log units, as the merge expects
        part_ml[2 * slot + 1] = l;
      }
    }
  }
}

}  // namespace

bool decode_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                           int chunk_tokens) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) && head_dim == 64 &&
         n_kv_heads >= 1 && n_kv_heads * head_dim <= kKvd && n_heads <= 16 &&
         n_heads % n_kv_heads == 0 && chunk_tokens % 64 == 0 && chunk_tokens >= 64 &&
         chunk_tokens <= 512;
}

int decode_mfma(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream) {
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  const int waves = chunk_tokens / 64;
  const int kv_dim = n_kv_heads * 64;
  const size_t lds = size_t(waves) * kVTileHalfs * 2 + size_t(waves) * 16 * 2 * sizeof(float);
  const dim3 grid(T, num_chunks), block(64 * waves);
  const int group = n_heads / n_kv_heads;
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  // 8 waves need ~69 KB of LDS: above the 64 KB default cap for dynamic LDS,
  // within gfx950's 160 KB per workgroup. Raise the cap once per kernel.
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
                       ws.part_ml, q, kp, vp, row_pos, row_seq, kv.tables, kv.max_pages,
                       kv.num_pages, n_heads, group, kv_dim, num_chunks, chunk_tokens);
  else
    hipLaunchKernelGGL(decode_partial_mfma<IE_KV_BF16>, grid, block, lds, stream, out, ws.part_o,
                       ws.part_ml, q, kp, vp, row_pos, row_seq, kv.tables, kv.max_pages,
                       kv.num_pages, n_heads, group, kv_dim, num_chunks, chunk_tokens);
  if (int rc = check_launch("attention_partial_mfma")) return rc;
  return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
}

}  // namespace iehip
