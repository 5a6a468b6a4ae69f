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
//   grid (T, num_chunks), rows fastest; chunk_tokens / 64 waves per workgroup
//   (2 at the default 128-token chunk), each wave owns 64 consecutive
//   positions = 4 pages = 2 page pairs. A workgroup takes exactly 16 KB of LDS
//   per wave and ~136 VGPRs per lane, so 5 two-wave workgroups fit on a CU and a
//   whole batch-64 decode step is resident at once (one round of workgroups,
//   every load of the step in flight from the start).
//   1. All K and V loads of the wave are issued first (one memory round trip).
//      K goes straight into the MFMA A-operand registers (4 x 16-byte loads per
//      page; lanes 0-15 hold tokens 0-15, the 4 lane groups hold the 4 16-byte
//      slices of each 64-byte quarter row). 8 MFMA 16x16x32 per page.
//   2. softmax over the chunk: wave-local max/sum by shuffles, across waves
//      through LDS (scores kept in registers; base-2 exponent).
//   3. V: each page pair (8 KB) is staged in a per-wave LDS tile with 16-byte
//      coalesced loads and read back transposed (one 2-byte element per lane per
//      slot) as the B operand; 16 MFMA 16x16x32 per pair.
//   4. O: per-wave tiles merged through LDS (log-sum-exp across the waves); a row
//      whose context fits one chunk writes `out` directly, otherwise the chunk
//      writes (o, m, l) and decode_merge_kernel (decode.hip) combines the chunks.
//      Merging inside this kernel instead (last chunk of a row, atomic counter)
//      was measured slower on MI355X: device-scope fences write back and
//      invalidate the XCD's L2, and the per-row counter serialises the chunks.
#include "common.hpp"
#include "decode.hpp"

namespace iehip {
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s4 __attribute__((ext_vector_type(4)));

constexpr int kKvd = 128;                 // elements per KV row (n_kv_heads * 64)
constexpr int kWaveLds = 16384;           // per-wave LDS: two 8 KB V page-pair tiles;
                                          // later the O tile (8 KB) and the wave's (m, l)
constexpr int kMaxWaves = 8;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
constexpr int kMaxLds = kMaxWaves * kWaveLds;

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
                    int group, int num_chunks, int chunk_tokens) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  extern __shared__ __align__(16) unsigned char smem[];
  const int waves = blockDim.x >> 6;
  // LDS per wave (16 KB): two 8 KB V page-pair tiles; after the PV products the
  // first 8 KB hold the wave's O tile [16 heads][128] and the next bytes its
  // per-head (m, l). Wave 0's area also holds the per-(wave, head) merge scales.
  auto red_m = [&](int w) { return reinterpret_cast<float*>(smem + size_t(w) * kWaveLds + 8192); };
  auto red_l = [&](int w) { return red_m(w) + 16; };
  float* comb_sc = reinterpret_cast<float*>(smem + 8192 + 256);  // [kMaxWaves][16]
  float* comb_il = comb_sc + kMaxWaves * 16;                       // [16] 1 / L

  const int t = blockIdx.x, c = blockIdx.y;
  const int p = row_pos[t];
  const int seq = row_seq[t];
  const int s0 = c * chunk_tokens;
  if (p < 0 || s0 > p) return;  // future chunk: the whole workgroup leaves
  const int n = min(s0 + chunk_tokens, p + 1) - s0;
  const bool single = s0 == 0 && p < chunk_tokens;  // the row fits this one chunk
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;
  const int wt0 = wave * 64;      // first position of this wave within the chunk
  const bool active = wt0 < n;    // wave-uniform: the wave has positions to read
  unsigned char* warea = smem + size_t(wave) * kWaveLds;

  // Page ids of this wave's 4 pages. A page past the context or outside the
  // pool is replaced by the wave's first page (re-read from cache, masked).
  int page[4];
  bool page_ok[4];
  {
    const int32_t* row_tab = tables + size_t(seq) * max_pages + (s0 + wt0) / IE_HIP_PAGE_SIZE;
    const int pi0 = (s0 + wt0) / IE_HIP_PAGE_SIZE;
#pragma unroll
    for (int pg = 0; pg < 4; ++pg) {
      int id = -1;
      if (wt0 + 16 * pg < n && pi0 + pg < max_pages) id = row_tab[pg];
      page_ok[pg] = id >= 0 && id < num_pages;
      page[pg] = id;
    }
#pragma unroll
    for (int pg = 0; pg < 4; ++pg)
      if (!page_ok[pg]) page[pg] = page_ok[0] ? page[0] : 0;
  }

  // 1. Every load of the wave is issued before any math (one memory round trip):
  //    V straight into LDS by DMA (global_load_lds_dwordx4: lane l of a load lands
  //    at base + 16 l), K into the MFMA A-operand registers (lane (g, r): token r
  //    of the page, 16-byte slice g of each 64-byte quarter row).
  //    V tile of a page pair: 32 rows of 256 bytes; 16-byte piece k of row `tok`
  //    is stored at slot k ^ 2*(tok & 7), so that the transposed reads below (8
  //    rows x 32 bytes per half-wave) fall into distinct banks.
  op ka[4][4];
  if (active) {
#pragma unroll
    for (int pp = 0; pp < 2; ++pp)
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int tok = 4 * u + g;                           // 0..31 within the pair
        const int piece = r ^ (2 * (tok & 7));               // global piece for slot r
        const uint16_t* src = v_pool +
            (size_t(page[2 * pp + (tok >> 4)]) * IE_HIP_PAGE_SIZE + (tok & 15)) * kKvd + 8 * piece;
        __builtin_amdgcn_global_load_lds(
            (const void __attribute__((address_space(1)))*)(src),
            (void __attribute__((address_space(3)))*)(warea + pp * 8192 + u * 1024), 16, 0, 0);
      }
#pragma unroll
    for (int pg = 0; pg < 4; ++pg) {
      const uint16_t* krow = k_pool + (size_t(page[pg]) * IE_HIP_PAGE_SIZE + r) * kKvd + 8 * g;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ka[pg][ks] = *reinterpret_cast<const op*>(krow + 32 * ks);
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // keep all loads ahead of the math

  // Block-diagonal query tile as the B operand, hi + lo: lane (g, r) holds
  // head r's query (times 1/8) at dims [32 ks + 8 g, +8) of the KV row when
  // those dims belong to head r's KV head (ks / 2), zeros otherwise.
  op qhi[4], qlo[4];
  {
    const int r_kvh = r >= group;  // kv head of query head r (two KV heads)
    const float* qrow = q + (size_t(t) * n_heads + r) * 64 + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      float4 a = make_float4(0.f, 0.f, 0.f, 0.f), b = a;
      if (r < n_heads && r_kvh == (ks >> 1)) {
        const float4* src = reinterpret_cast<const float4*>(qrow + 32 * (ks & 1));
        a = src[0];
        b = src[1];
      }
      const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float v = x[j] * 0.125f;
        const E hi = static_cast<E>(v);
        qhi[ks][j] = hi;
        qlo[ks][j] = static_cast<E>(v - static_cast<float>(hi));
      }
    }
  }

  // 2. S^T per page (lane (g, r): tokens 4g..4g+3 of the page, head r), then the
  //    wave's own softmax statistics (base 2); waves are merged at the end.
  float mw = -INFINITY, lw = 0.0f;
  f32x4 o[8];
#pragma unroll
  for (int nt = 0; nt < 8; ++nt) o[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
  if (active) {
    f32x4 s[4];
#pragma unroll
    for (int pg = 0; pg < 4; ++pg) {
      s[pg] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s[pg] = M::mma(ka[pg][ks], qhi[ks], s[pg]);
        s[pg] = M::mma(ka[pg][ks], qlo[ks], s[pg]);
      }
    }
#pragma unroll
    for (int pg = 0; pg < 4; ++pg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int tok = wt0 + 16 * pg + 4 * g + i;
        const float v = (page_ok[pg] && tok < n) ? s[pg][i] * kLog2e : -INFINITY;
        s[pg][i] = v;
        mw = fmaxf(mw, v);
      }
    mw = fmaxf(mw, __shfl_xor(mw, 16, 64));
    mw = fmaxf(mw, __shfl_xor(mw, 32, 64));
    op phi[2], plo[2];  // A operands of the two page pairs
#pragma unroll
    for (int pg = 0; pg < 4; ++pg)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float e = exp2f(s[pg][i] - mw);  // masked: exp2(-inf) = 0
        lw += e;
        const E hi = static_cast<E>(e);
        phi[pg >> 1][(pg & 1) * 4 + i] = hi;
        plo[pg >> 1][(pg & 1) * 4 + i] = static_cast<E>(e - static_cast<float>(hi));
      }
    lw += __shfl_xor(lw, 16, 64);
    lw += __shfl_xor(lw, 32, 64);

    // 3. O += P V. The B operand (pair token 4g+j in slot j < 4, 16+4g+j-4 in
    //    slot j >= 4; dim 16 nt + r) comes from two transposing LDS reads
    //    (ds_read_b64_tr_b16): in each 16-lane group, lane 4a+b receives element
    //    b of the 8-byte reads of lanes a, a+4, a+8, a+12; lane L reads row
    //    4g + L/4, dims 16 nt + 4 (L%4) .. +3, so lane r receives dim 16 nt + r of
    //    rows 4g..4g+3 (and 16+4g.. for the second read).
    __builtin_amdgcn_s_waitcnt(0);  // the LDS DMA of V has landed
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const int rtok = 4 * g + (r >> 2);  // row this lane reads (first read)
    const int rsw = rtok & 7;           // its swizzle key
    const int rlo = (r & 1) * 8;        // byte within the 16-byte piece
    const int rpc = (r >> 1) & 1;       // piece parity within the 32-byte unit
#pragma unroll
    for (int pp = 0; pp < 2; ++pp) {
      const unsigned char* vt = warea + pp * 8192 + rtok * 256 + rlo;
#pragma unroll
      for (int nt = 0; nt < 8; ++nt) {
        const int slot = 2 * (nt ^ rsw) + rpc;
        const s4 lo4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s4*)(vt + slot * 16));
        const s4 hi4 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (__attribute__((address_space(3))) s4*)(vt + 16 * 256 + slot * 16));
        // Joined as whole vectors: element-wise extraction of these results
        // miscompiles (it broadcasts element 0) with this toolchain.
        const op b = __builtin_bit_cast(op, __builtin_shufflevector(lo4, hi4, 0, 1, 2, 3, 4, 5, 6, 7));
        o[nt] = M::mma(phi[pp], b, o[nt]);
        o[nt] = M::mma(plo[pp], b, o[nt]);
      }
    }
  }

  // 4. Per-wave O tile [16 heads][128] floats into the wave's own area (its V
  //    reads are done) and per-wave (m, l); then the waves are merged
  //    (log-sum-exp) for the diagonal blocks (head h, its KV head's 64 dims).
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  float* ot = reinterpret_cast<float*>(warea);
#pragma unroll
  for (int nt = 0; nt < 8; ++nt)
#pragma unroll
    for (int i = 0; i < 4; ++i) ot[(4 * g + i) * kKvd + 16 * nt + r] = o[nt][i];
  if (g == 0) {
    red_m(wave)[r] = mw;
    red_l(wave)[r] = lw;
  }
  __syncthreads();
  if (tid < n_heads) {  // per head: chunk max, merge scale of each wave, sum, 1 / sum
    const int h = tid;
    float mx = -INFINITY;
    for (int w = 0; w < waves; ++w) mx = fmaxf(mx, red_m(w)[h]);
    float l = 0.0f;
    for (int w = 0; w < waves; ++w) {
      const float mwh = red_m(w)[h];
      const float sc = mwh == -INFINITY ? 0.0f : exp2f(mwh - mx);
      comb_sc[w * 16 + h] = sc;
      l = __builtin_fmaf(red_l(w)[h], sc, l);
    }
    comb_il[h] = 1.0f / l;
    if (!single) {
      const size_t slot = (size_t(t) * n_heads + h) * num_chunks + c;
      part_ml[2 * slot] = mx * kLn2;  // natural-log units
      part_ml[2 * slot + 1] = l;
    }
  }
  __syncthreads();
  // Each thread owns outputs idx = tid + k * blockDim (head idx / 64, dim idx % 64).
#pragma unroll 4
  for (int idx = tid; idx < n_heads * 64; idx += blockDim.x) {
    {
      const int h = idx >> 6, d = idx & 63;
      const int col = (h >= group ? 64 : 0) + d;
      float acc = 0.0f;
#pragma unroll
      for (int w = 0; w < kMaxWaves; ++w)
        if (w < waves)
          acc = __builtin_fmaf(
              reinterpret_cast<const float*>(smem + size_t(w) * kWaveLds)[h * kKvd + col],
              comb_sc[w * 16 + h], acc);
      const size_t head = size_t(t) * n_heads + h;
      if (single)
        out[head * 64 + d] = acc * comb_il[h];
      else
        part_o[(head * num_chunks + c) * 64 + d] = acc;
    }
  }
}

}  // namespace

bool decode_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                           int chunk_tokens) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) && head_dim == 64 &&
         n_kv_heads * head_dim == kKvd && n_heads <= 16 &&
         n_heads % n_kv_heads == 0 && chunk_tokens % 64 == 0 && chunk_tokens >= 64 &&
         chunk_tokens <= 512;
}

int decode_mfma(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream) {
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  const int waves = chunk_tokens / 64;
  const size_t lds = size_t(waves) * kWaveLds;
  const dim3 grid(T, num_chunks), block(64 * waves);
  const int group = n_heads / n_kv_heads;
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  // 8 waves (512-token chunks) need 128 KB of LDS: above the 64 KB default cap
  // for dynamic LDS, within gfx950's 160 KB per workgroup. Raise it once.
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
                       kv.num_pages, n_heads, group, num_chunks, chunk_tokens);
  else
    hipLaunchKernelGGL(decode_partial_mfma<IE_KV_BF16>, grid, block, lds, stream, out, ws.part_o,
                       ws.part_ml, q, kp, vp, row_pos, row_seq, kv.tables, kv.max_pages,
                       kv.num_pages, n_heads, group, num_chunks, chunk_tokens);
  if (int rc = check_launch("attention_mfma")) return rc;
  return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
}

}  // namespace iehip
