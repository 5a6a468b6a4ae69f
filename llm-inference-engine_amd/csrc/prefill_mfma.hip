// Chunked-prefill attention into pages on the matrix cores (gfx950), for f16
// and bf16 KV caches with head_dim 64.
//
// Reference semantics: each row's causal GQA attention over positions
// 0..row_pos[t] of its sequence (src/ops.cpp:70-108); the reference's GPU
// prompt kernels are src/cuda/kernels.cu:527-776. Rows are consecutive
// positions of ONE sequence (row_pos[t] = row_pos[0] + t), already appended.
//
// Here QK^T and PV are dense tiles: a block of 16 query rows against 64-key
// tiles, per query head,
//     S^T[16 keys x 16 rows]   = K_tile[16 x 64] . Q^T[64 x 16]          (2 k-steps)
//     O^T[64 dims x 16 rows]  += V_tile^T[64 x 32 keys] . P^T[32 x 16 rows]
// on v_mfma_f32_16x16x32_{f16,bf16} in the cache's own 16-bit type. As in the
// decode kernel, lane (g, r) of every tile belongs to query row r, so the
// online-softmax statistics of a row never leave its lanes except for the
// reductions over the 4 lane groups.
//
// Precision: K and V enter exactly; q (pre-scaled by log2(e)/8) and P are split
// into hi + lo halves of the same 16-bit type and each product is done twice --
// float32-level scores and weights (the 2e-3 absolute bound for 16-bit caches
// holds with a wide margin; measured errors are ~1e-6).
//
// Layout of the work:
//   One workgroup per (pair of 16-row blocks, KV head); one wave per query head
//   of the KV head (the 7 heads of a Qwen2.5 group share every K/V tile through
//   LDS). The pair is block b and block n-1-b: the causal triangle gives block b
//   b+1 key tiles of work, so every pair carries about the same total and the
//   ceil(n/2) x n_kv_heads workgroups finish together (the heavier block goes
//   first).
//   K/V tiles of 64 keys (4 pages) are double-buffered in LDS (2 x 16 KB): while
//   the waves compute on one, the next tile's 16 KB arrive by DMA
//   (global_load_lds_dwordx4, 16 x 1 KB spread over the waves), page ids
//   prefetched a tile ahead. K rows are stored with their 16-byte pieces
//   swizzled (piece ^ (row/2 % 8)) so the A-operand reads (16 rows, one piece
//   each) hit distinct banks; V rows with piece ^ 2*(row/2 % 4) so the
//   transposed reads (ds_read_b64_tr_b16: 8 rows x 32 bytes per half-wave) do.
//   Keys past the block's last position and pages outside the pool are masked
//   (-inf scores, and their V rows zeroed in LDS before use, so stale or
//   non-finite memory cannot reach the output through 0 * x).
#include <algorithm>

#include "common.hpp"
#include "mfma.hpp"
#include "prefill.hpp"

namespace iehip {
namespace {

constexpr int kRows = 16;                  // query rows per block (one MFMA column tile)
constexpr int kKeys = 64;                  // keys per LDS tile
constexpr int kTileBytes = kKeys * 128;    // 64 keys x 64 dims x 2 B
constexpr int kBufBytes = 2 * kTileBytes;  // K tile + V tile
constexpr int kLdsBytes = 2 * kBufBytes;   // double-buffered
constexpr int kMaxGroup = 8;
constexpr float kLog2e = 1.4426950408889634f;

template <int KV>
__global__ void __launch_bounds__(64 * kMaxGroup)
prefill_mfma_kernel(float* __restrict__ out, const float* __restrict__ q,
                    const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
                    int T, const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                    const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
                    int n_kv_heads, int n_blocks) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  extern __shared__ __align__(16) unsigned char smem[];
  const int waves = blockDim.x >> 6;  // = query heads per KV head
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int g = lane >> 4, r = lane & 15;
  const int h = kvh * waves + wave;
  const int kv_dim = n_kv_heads * 64;
  const int pos0 = __builtin_amdgcn_readfirstlane(row_pos[0]);
  const int seq = __builtin_amdgcn_readfirstlane(row_seq[0]);
  const int32_t* tab = tables + size_t(seq) * max_pages;

  // Page id of the tile's page j (uniform); -1 past the table row.
  auto page_id = [&](const int tile, const int j) -> int {
    const int pi = tile * (kKeys / IE_HIP_PAGE_SIZE) + j;
    return pi < max_pages ? tab[pi] : -1;
  };
  auto valid = [&](const int id) { return id >= 0 && id < num_pages; };

  // DMA of tile `tile` into buffer `buf`: 8 K loads then 8 V loads of 1 KB
  // (8 key rows of 128 bytes each), load i issued by wave i % waves. Lane l of a
  // load moves key row 8u + l/8, LDS slot l % 8 (the DMA lands lane l at base +
  // 16 l), fetching the global piece that the row's swizzle maps to that slot.
  auto issue = [&](const int tile, const int buf, const int id0, const int id1, const int id2,
                   const int id3) {
    for (int i = wave; i < 16; i += waves) {
      const bool is_v = i >= 8;
      const int u = i & 7;
      const int row = 8 * u + (lane >> 3), slot = lane & 7;
      const int piece = is_v ? slot ^ (2 * ((row >> 1) & 3)) : slot ^ ((row >> 1) & 7);
      const int pj = u >> 1;
      const int id = pj == 0 ? id0 : pj == 1 ? id1 : pj == 2 ? id2 : id3;
      const int page = valid(id) ? id : 0;
      const uint16_t* src = (is_v ? v_pool : k_pool) +
                            (size_t(page) * IE_HIP_PAGE_SIZE + (row & 15)) * kv_dim + kvh * 64 +
                            8 * piece;
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(src),
          (void __attribute__((address_space(3)))*)(smem + buf * kBufBytes +
                                                    (is_v ? kTileBytes : 0) + u * 1024),
          16, 0, 0);
    }
  };

  for (int pass = 0; pass < 2; ++pass) {
    const int hi_block = n_blocks - 1 - int(blockIdx.x);
    const int rb = pass == 0 ? hi_block : int(blockIdx.x);
    if (pass == 1 && rb == hi_block) break;  // the middle block of an odd count
    const int t0 = rb * kRows;
    const int t_last = min(t0 + kRows, T) - 1;
    const int max_pos = pos0 + t_last;  // last position any row of the block sees
    const int min_pos = pos0 + t0;      // first row's position
    const int n_tiles = max_pos / kKeys + 1;

    // Query of row t0 + r, head h, as the B operand (dims 32 ks + 8g .. +8).
    const int t = t0 + r;
    const bool row_ok = t < T;
    const int rp = pos0 + t;  // this lane's row position
    op qhi[2], qlo[2];
    {
      float4 a[2][2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        a[ks][0] = a[ks][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row_ok) {
          const float4* src =
              reinterpret_cast<const float4*>(q + (size_t(t) * n_heads + h) * 64 + 32 * ks + 8 * g);
          a[ks][0] = src[0];
          a[ks][1] = src[1];
        }
      }
      const float qs = 0.125f * kLog2e;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const float x[8] = {a[ks][0].x, a[ks][0].y, a[ks][0].z, a[ks][0].w,
                            a[ks][1].x, a[ks][1].y, a[ks][1].z, a[ks][1].w};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          E hv, lv;
          split16(x[j] * qs, hv, lv);
          qhi[ks][j] = hv;
          qlo[ks][j] = lv;
        }
      }
    }

    float m = -INFINITY, l = 0.0f;  // running max (base 2), this lane's part of the sum
    f32x4 o[4];                     // O^T: lane (g, r) holds row r, dims 16 mt + 4g + e
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    int ids[4] = {page_id(0, 0), page_id(0, 1), page_id(0, 2), page_id(0, 3)};
    issue(0, 0, ids[0], ids[1], ids[2], ids[3]);
    int nx[4] = {page_id(1, 0), page_id(1, 1), page_id(1, 2), page_id(1, 3)};
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();

    for (int kb = 0; kb < n_tiles; ++kb) {
      const int buf = kb & 1;
      const bool ok_pg[4] = {valid(ids[0]), valid(ids[1]), valid(ids[2]), valid(ids[3])};
      if (kb + 1 < n_tiles) {  // the next tile into the other buffer (free since the last barrier)
        issue(kb + 1, buf ^ 1, nx[0], nx[1], nx[2], nx[3]);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          ids[j] = nx[j];
          nx[j] = page_id(kb + 2, j);
        }
      }
      const int kbase = kb * kKeys;
      const unsigned char* kt = smem + buf * kBufBytes;
      const unsigned char* vt = kt + kTileBytes;
      const bool pages_ok = ok_pg[0] && ok_pg[1] && ok_pg[2] && ok_pg[3];
      // Keys past max_pos (the last tile) or in pages outside the pool: zero
      // their V rows before any wave reads the tile (uniform decision).
      if (kbase + kKeys - 1 > max_pos || !pages_ok) {
        for (int i = tid; i < kKeys * 8; i += blockDim.x) {
          const int key = i >> 3;
          if (kbase + key > max_pos || !ok_pg[key >> 4])
            *reinterpret_cast<uint4*>(const_cast<unsigned char*>(vt) + key * 128 + (i & 7) * 16) =
                make_uint4(0, 0, 0, 0);
        }
        __syncthreads();
      }

      // S^T for the tile's 4 key groups of 16: A = K rows 16 kt4 + r, dims 32 ks + 8g.
      f32x4 s[4];
#pragma unroll
      for (int kt4 = 0; kt4 < 4; ++kt4) {
        s[kt4] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int row = 16 * kt4 + r;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const int slot = (4 * ks + g) ^ ((row >> 1) & 7);
          const op a = *reinterpret_cast<const op*>(kt + row * 128 + slot * 16);
          s[kt4] = M::mma(a, qhi[ks], s[kt4]);
          s[kt4] = M::mma(a, qlo[ks], s[kt4]);
        }
      }
      // Causal mask (and masked pages) where the tile is not entirely visible.
      if (kbase + kKeys - 1 > min_pos || !pages_ok) {
#pragma unroll
        for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int kp = kbase + 16 * kt4 + 4 * g + e;
            s[kt4][e] = (kp <= rp && ok_pg[kt4]) ? s[kt4][e] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt4 = 0; kt4 < 4; ++kt4)
        mx = fmaxf(mx, fmaxf(fmaxf(s[kt4][0], s[kt4][1]), fmaxf(s[kt4][2], s[kt4][3])));
      mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
      mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
      const float m_new = fmaxf(m, mx);
      const float mref = m_new == -INFINITY ? 0.0f : m_new;  // nothing visible yet: weights 0
      const float corr = exp2f(m - mref);                     // m = -inf: 0
      l *= corr;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) o[mt] *= corr;
      m = m_new;
      // P^T operands per 32-key group kg: slots 0-3 = keys 32kg + 4g + e (group
      // 2kg), slots 4-7 = keys 32kg + 16 + 4g + e (group 2kg+1).
      op phi[2], plo[2];
#pragma unroll
      for (int kg = 0; kg < 2; ++kg)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pa = exp2f(s[2 * kg][e] - mref), pb = exp2f(s[2 * kg + 1][e] - mref);
          l += pa + pb;
          E ha, la, hb, lb;
          split16(pa, ha, la);
          split16(pb, hb, lb);
          phi[kg][e] = ha;
          plo[kg][e] = la;
          phi[kg][4 + e] = hb;
          plo[kg][4 + e] = lb;
        }
      // O^T += V^T P^T. Lane L reads tile row 32kg + 4g + L/4 (and +16), dims
      // 16 mt + 4 (L%4) .. +3: after the transpose lane r holds dim 16 mt + r of
      // keys 32kg + 4g + e and 32kg + 16 + 4g + e -- P^T's slots.
      const int rbyte = (r & 1) * 8;
#pragma unroll
      for (int kg = 0; kg < 2; ++kg) {
        const int vrow = 32 * kg + 4 * g + (r >> 2);
        const int sw = 2 * ((vrow >> 1) & 3);  // same for vrow + 16
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) {
          const int slot = (2 * mt + ((r >> 1) & 1)) ^ sw;
          const s16x4 lo4 = lds_read_tr16(vt + vrow * 128 + slot * 16 + rbyte);
          const s16x4 hi4 = lds_read_tr16(vt + (vrow + 16) * 128 + slot * 16 + rbyte);
          const op a = join_tr<op>(lo4, hi4);
          o[mt] = M::mma(a, phi[kg], o[mt]);
          o[mt] = M::mma(a, plo[kg], o[mt]);
        }
      }
      __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA of the next tile has landed
      __syncthreads();                // every wave's DMA landed, every wave done with `buf`
    }

    l += __shfl_xor(l, 16, 64);
    l += __shfl_xor(l, 32, 64);
    if (row_ok) {
      const float il = 1.0f / l;
      float* dst = out + (size_t(t) * n_heads + h) * 64 + 4 * g;
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4*>(dst + 16 * mt) = o[mt] * il;
    }
  }
}

}  // namespace

bool prefill_mfma_enabled() { return true; }

bool prefill_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) && head_dim == 64 && n_kv_heads > 0 &&
         n_heads % n_kv_heads == 0 && n_heads / n_kv_heads <= kMaxGroup;
}

int prefill_mfma_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, hipStream_t stream) {
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return fail(IE_HIP_EINVAL, "attention_prefill: q, out and the pools must be 16-byte aligned");
  const int group = n_heads / n_kv_heads;
  const int n_blocks = (T + kRows - 1) / kRows;
  const dim3 grid((n_blocks + 1) / 2, n_kv_heads), block(64 * group);
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  if (kv.kv_dtype == IE_KV_F16)
    hipLaunchKernelGGL(prefill_mfma_kernel<IE_KV_F16>, grid, block, kLdsBytes, stream, out, q, kp,
                       vp, T, row_pos, row_seq, kv.tables, kv.max_pages, kv.num_pages, n_heads,
                       n_kv_heads, n_blocks);
  else
    hipLaunchKernelGGL(prefill_mfma_kernel<IE_KV_BF16>, grid, block, kLdsBytes, stream, out, q, kp,
                       vp, T, row_pos, row_seq, kv.tables, kv.max_pages, kv.num_pages, n_heads,
                       n_kv_heads, n_blocks);
  return check_launch("attention_prefill_mfma");
}

}  // namespace iehip
