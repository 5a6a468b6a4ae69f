// Flash-decoding attention over pages on the matrix cores (gfx950), for KV
// caches whose rows hold 128 elements (2 KV heads x 64) and at most 16 query
// heads -- Qwen2.5-0.5B: 14 query heads, 2 KV heads. 16-bit caches:
// decode_partial_mfma, described here (with kFused, the decode step's RoPE +
// append rides along); f32 caches: decode_partial_mfma_f32, further down.
//
// Reference semantics: each row's causal GQA attention, src/ops.cpp:70-108;
// split-K chunks merged by log-sum-exp as in src/cuda/kernels.cu:309-507.
//
// Why MFMA for decode: every KV row is used by all 7 query heads of its group,
// so per 16-token page the work is two dense products,
//     S^T[16 tok x 16 heads]   = K_page[16 x 128] . Qbd^T[128 x 16]
//     O^T[128 dims x 16 heads] += V_pair^T[128 x 32 tok] . P^T[32 tok x 16 heads]
// where Qbd is block-diagonal: head h carries its query in the 64 dims of its
// own KV head and zeros elsewhere, so ONE 16-column tile serves all 14 heads of
// both KV heads and each K/V row is read exactly once. On the VALU the same
// work costs ~1,800 FMAs per position -- as much time as streaming the cache.
// The only extra work is the off-diagonal half of O^T, discarded at the end.
// With both products in this orientation, lane (g, r) of every tile belongs to
// head r: the scores it holds (S^T), the weights it feeds (P^T) and the output
// it accumulates (O^T) are all head r's, so softmax statistics never move
// between lanes except for the reductions over the 4 lane groups.
//
// Precision (2e-3 absolute bound for 16-bit caches): K and V enter the MFMA in
// their stored format, exactly. Q (pre-scaled by log2(e)/8) and P are split
// into hi + lo halves of the same 16-bit type, each product done twice:
// |x - hi - lo| <= u^2 |x| for the type's unit roundoff u (f16 2^-11, so
// 2^-22: float32-level; bf16 2^-8, so 2^-16).
//
// Layout of the work:
//   One workgroup per non-empty (row, chunk) pair. The 1-D grid covers the
//   chunks each row actually has, so all real work comes first in dispatch
//   order and the slots past the batch's total exit at once. A workgroup finds
//   its (row, chunk) and page ids either in a host-built work list (one load;
//   items ordered longer chunks first, so the rows' short last chunks fill the
//   end of the launch) or by a prefix sum of the rows' chunk counts from
//   row_pos followed by the row's table (two dependent loads; row by row).
//   A chunk is streamed as page pairs (32 tokens, 2 pages), and each pair
//   yields its own partial: its max per head, weights relative to that max,
//   their sum and V^T P^T from zero (fold_pair folds it into the running
//   result). Large grids: one wave streams the chunk's pairs, keeping the next
//   pair's loads in flight while it computes the current one. Small grids (few,
//   long rows): one wave per pair, every pair in flight at once, and wave 0
//   folds the others' partials through LDS in pair order -- the same fold, so
//   the same bits (decode_mfma_waves). A wave takes 16 KB of LDS (two V
//   page-pair tiles, double-buffered).
//   1. The query, then page pair 0: K straight into the MFMA A-operand
//      registers (lanes 0-15 hold tokens 0-15, the 4 lane groups the 4 16-byte
//      slices of each 64-byte quarter row), V into an LDS tile by DMA.
//   2. Per page pair, as its data lands: S^T (8 MFMA 16x16x32 per page); the
//      next pair's loads into the K registers and the other LDS tile; the
//      pair's max, weights and sum; V^T P^T with V^T read back from the tile
//      transposed (ds_read_b64_tr_b16) as the A operand (16 MFMA per pair);
//      the fold.
//   3. A row whose context fits one chunk writes `out` directly; otherwise the
//      chunk writes its partial (o, m, l) to the workspace and
//      decode_merge_kernel (decode.hip) combines the row's chunks. Fusing that
//      merge into this kernel (the row's last chunk to finish merges, through a
//      per-row atomic counter) was measured slower on MI355X, also with every
//      chunk of a row placed on one XCD so the partials stay in its L2: the
//      store acknowledgements and the atomic cost what the launch saves.
//   Positions past the row's context (the tail of its last page) and pages
//   whose id lies outside the pool are masked: their scores are -inf and their
//   V elements are zeroed before the product, so stale or non-finite memory in
//   those rows cannot reach the output. Page pairs with no such position skip
//   the masking.
#include <algorithm>

#include "common.hpp"
#include "decode.hpp"
#include "mfma.hpp"

namespace iehip {
namespace {

constexpr int kKvd = 128;          // elements per KV row (n_kv_heads * 64)
constexpr int kPair = 8192;        // one V page-pair tile [32 tok][256 B]
constexpr int kTile = 2 * kPair;   // per-wave LDS: the two page-pair tiles; after the
                                   // products, the wave's output tile [16][64] f32
constexpr int kMaxWaves = 8;
constexpr int kOutTile = 16 * 64 * 4;        // a wave's output tile [16 heads][64] f32
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxLds = kMaxWaves * kTile;

__device__ __forceinline__ int wave_inclusive_scan(int v, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int u = __shfl_up(v, off, 64);
    if (lane >= off) v += u;
  }
  return v;
}

// Folds a page pair's partial (max mj in log2 units, this lane's part lj of the
// sum of its weights 2^(s - mj), and pv = V^T P^T of those weights) into the
// running (m, l, o). A side with max -inf saw no position and passes the other
// side through unchanged; otherwise both are rescaled to the larger max. The
// same function, in the same pair order, serves one wave folding its pairs and
// wave 0 folding one pair per wave, so the two layouts give the same bits.
__device__ __forceinline__ void fold_pair(float& m, float& l, f32x4 (&o)[8], const float mj,
                                          const float lj, const f32x4 (&pv)[8]) {
  if (mj == -INFINITY) return;
  if (m == -INFINITY) {
    m = mj;
    l = lj;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] = pv[mt];
    return;
  }
  const float mn = fmaxf(m, mj);
  const float a = exp2_weight(m - mn), b = exp2_weight(mj - mn);
  m = mn;
  l = __builtin_fmaf(l, a, lj * b);
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int e = 0; e < 4; ++e) o[mt][e] = __builtin_fmaf(o[mt][e], a, pv[mt][e] * b);
}

// Workgroup `wg` -> (row t, chunk c, position p, sequence seq) in the order
// "row 0's chunks, row 1's chunks, ...", where row t has min(p / chunk + 1,
// num_chunks) chunks (none if p < 0). Every wave computes the same answer.
// Returns false when wg lies past the batch's last chunk.
__device__ __forceinline__ bool locate_chunk(int wg, int T, const int32_t* __restrict__ row_pos,
                                             const int32_t* __restrict__ row_seq, int num_chunks,
                                             int chunk_tokens, int lane, int& t, int& c, int& p,
                                             int& seq) {
  int base = 0;
  for (int r0 = 0; r0 < T; r0 += 64) {
    const int rr = r0 + lane;
    const int pr = rr < T ? row_pos[rr] : -1;
    const int sr = rr < T ? row_seq[rr] : 0;
    const int n = pr < 0 ? 0 : min(pr / chunk_tokens + 1, num_chunks);
    const int incl = wave_inclusive_scan(n, lane);
    const int total = __builtin_amdgcn_readfirstlane(__shfl(incl, 63, 64));
    if (wg < base + total) {
      const unsigned long long m = __ballot(wg < base + incl);
      const int L = __ffsll(m) - 1;  // first lane whose chunks reach past wg
      t = r0 + L;
      p = __builtin_amdgcn_readfirstlane(__shfl(pr, L, 64));
      seq = __builtin_amdgcn_readfirstlane(__shfl(sr, L, 64));
      c = wg - base - __builtin_amdgcn_readfirstlane(__shfl(incl - n, L, 64));
      return true;
    }
    base += total;
  }
  return false;
}

// kOneWave: one-wave workgroups (a wave streams the whole chunk) -- its fold
// is the chunk's result, so the epilogue writes straight from the accumulators
// and the workgroup needs no LDS beyond its V tiles. Otherwise one wave per
// page pair, and wave 0 folds the other waves' pair partials through LDS.
template <int KV, bool kOneWave, bool kFused>
__global__ void __launch_bounds__(kOneWave ? 64 : 512)
__attribute__((amdgpu_waves_per_eu(2)))  // ~206 registers: a pair partial beside the running one
decode_partial_mfma(float* __restrict__ out, float* __restrict__ part_o,
                    float* __restrict__ part_ml, const float* __restrict__ q,
                    const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
                    const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                    const int32_t* __restrict__ tables, int T, int max_pages, int num_pages,
                    int n_heads, int group, int num_chunks, int chunk_tokens, FusedAppend fa,
                    const int32_t* __restrict__ plan) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  extern __shared__ __align__(16) unsigned char smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = kOneWave ? 0 : __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int waves = kOneWave ? 1 : blockDim.x >> 6;
  const int tw = chunk_tokens / waves;              // positions per wave (a multiple of 32)
  const int wt0 = wave * tw;                        // first position of this wave in the chunk

  // Which (row, chunk) this workgroup takes, and the page ids of the wave's
  // pages, one per lane (lane i: page i of the wave's positions; -1 past them
  // or past the table row). With a host-built plan both come from the
  // workgroup's item in one round trip (the header and this lane's page id are
  // loaded together, before the item count is checked: every item slot of the
  // grid lies inside the plan). Without one, every wave prefix-sums the rows'
  // chunk counts (locate_chunk) and then reads the row's table: two dependent
  // round trips before the first K/V load. A pair's ids are read from this
  // register (readlane): a scalar load of the table inside the pair loop would
  // share lgkmcnt with the transposed V reads, so the first V wait of every
  // pair would also wait for the table's round trip. A wave covers at most 64
  // pages (1,024 positions, the largest chunk).
  int t, c, p, seq;
  int pid_plan = -1;
  if (plan) {
    const int32_t* item = plan + kPlanHeader + size_t(blockIdx.x) * plan_stride(chunk_tokens);
    const int pg = wt0 / IE_HIP_PAGE_SIZE + lane;
    pid_plan = pg < chunk_tokens / IE_HIP_PAGE_SIZE ? item[4 + pg] : -1;
    const int4 head = *reinterpret_cast<const int4*>(plan);  // [items, chunk, chunks, rows]
    const int items = __builtin_amdgcn_readfirstlane(head.x);
    t = __builtin_amdgcn_readfirstlane(item[0]);
    c = __builtin_amdgcn_readfirstlane(item[1]);
    p = __builtin_amdgcn_readfirstlane(item[2]);
    seq = __builtin_amdgcn_readfirstlane(item[3]);
    if (int(blockIdx.x) >= items) return;  // past the plan's last item
    // A plan built for another launch (another chunk size, chunk count or row
    // count) would address other slots: such a launch writes nothing. So does
    // an item naming a row or chunk outside this launch's.
    if (__builtin_amdgcn_readfirstlane(head.y) != chunk_tokens ||
        __builtin_amdgcn_readfirstlane(head.z) != num_chunks ||
        __builtin_amdgcn_readfirstlane(head.w) != T || t < 0 || t >= T || c < 0 ||
        c >= num_chunks || p < c * chunk_tokens)
      return;
  } else if (!locate_chunk(blockIdx.x, T, row_pos, row_seq, num_chunks, chunk_tokens, lane, t, c,
                           p, seq)) {
    return;  // past the batch's last chunk: the whole workgroup leaves
  }
  const int s0 = c * chunk_tokens;
  const int n = min(s0 + chunk_tokens, p + 1) - s0;  // positions of this chunk
  // The row has one chunk (its context fits one, or the caller sized one):
  // written here; the merge skips it, reading the same count.
  const bool single = min(p / chunk_tokens + 1, num_chunks) == 1;
  const int nw = min(max(n - wt0, 0), tw);          // positions this wave attends to
  const int np = (nw + 31) >> 5;                    // its page pairs
  unsigned char* warea = smem + size_t(wave) * kTile;
  const unsigned warea_lds = lds_address(smem) + wave * kTile;
  const int pi0 = (s0 + wt0) / IE_HIP_PAGE_SIZE;
  const int32_t* row_tab = tables + size_t(seq) * max_pages;
  const int pid_lane = plan ? (16 * lane < nw ? pid_plan : -1)
                            : (16 * lane < nw && pi0 + lane < max_pages) ? row_tab[pi0 + lane] : -1;
  auto page_id = [&](const int pw) -> int {
    return pw < 64 ? __builtin_amdgcn_readlane(pid_lane, pw) : -1;
  };

  // The query of head r (the B operand's column), dims [8g, 8g+8) and
  // [32 + 8g, 32 + 8g + 8) of its own KV head. Loaded first, so that waiting
  // for it does not wait for the K/V loads behind it.
  const bool head_ok = r < n_heads;
  const int kv_r = r >= group;  // KV head of query head r (two KV heads)
  float4 q0a = make_float4(0.f, 0.f, 0.f, 0.f), q0b = q0a, q1a = q0a, q1b = q0a;
  if (head_ok) {
    const float4* qrow = reinterpret_cast<const float4*>(q + (size_t(t) * n_heads + r) * 64 + 8 * g);
    q0a = qrow[0];
    q0b = qrow[1];
    q1a = qrow[8];
    q1b = qrow[9];
  }

  // Fused RoPE + append (kFused): every workgroup rotates its row's query in
  // registers (lane (g, r) holds the rotation pairs (8g + j, 32 + 8g + j) of
  // head r) with the table's cos/sin of position p; the wave holding position
  // p -- the row's newest, appended now -- also rotates and rounds the new k,
  // rounds v, writes both into their page slot and substitutes them for what
  // it loads from there. Same arithmetic as ie_hip_rope_and_cache (explicit
  // fmaf, no contraction; the KV type's own rounding), so pages and results
  // are bit-identical to the two calls. Rows whose position lies outside the
  // table are not appended and use their query unrotated, as there.
  // The cos/sin row and the new k and v are loaded here and used only after
  // pair 0's K/V loads are issued, so their round trip overlaps that one; the
  // slot's page id is the wave's own (page_id), not another table read.
  const bool app = kFused && p < fa.table_positions;
  const int off = p - s0 - wt0;  // position p within this wave's range
  const bool own = app && off >= 0 && off < tw;
  E kn[4][8];                    // new K row, this lane's slices (dims 8g + 32 ks + e)
  uint4 vn = make_uint4(0, 0, 0, 0);  // new V row, 16-byte piece r
  float4 tc0, tc1, tn0, tn1;          // cos and sin of position p, dims 8g .. 8g+7
  float4 kr[2][4];                    // new k, KV head hk: dims 64 hk + 8g .. +7, 32 + ..
  float4 vr0, vr1;                    // new v, dims 8r .. 8r+7
  if constexpr (kFused) {
    if (app) {
      const float* trow = fa.table + size_t(p) * 64 + 8 * g;
      tc0 = *reinterpret_cast<const float4*>(trow);
      tc1 = *reinterpret_cast<const float4*>(trow + 4);
      tn0 = *reinterpret_cast<const float4*>(trow + 32);
      tn1 = *reinterpret_cast<const float4*>(trow + 36);
      if (own) {
        const float4* krow = reinterpret_cast<const float4*>(fa.k + size_t(t) * kKvd + 8 * g);
#pragma unroll
        for (int hk = 0; hk < 2; ++hk) {
          kr[hk][0] = krow[16 * hk];
          kr[hk][1] = krow[16 * hk + 1];
          kr[hk][2] = krow[16 * hk + 8];
          kr[hk][3] = krow[16 * hk + 9];
        }
        const float4* vrow = reinterpret_cast<const float4*>(fa.v + size_t(t) * kKvd + 8 * r);
        vr0 = vrow[0];
        vr1 = vrow[1];
      }
    }
  }

  // Loads of page pair j (pages 2j, 2j+1 of the wave): K into the MFMA
  // A-operand registers `ka` (lane (g, r): token r of the page, the 16-byte
  // slice g of each 64-byte quarter row), V into LDS tile j & 1 by DMA.
  // V tile of a page pair: 32 rows of 256 bytes; 16-byte piece k of row `tok`
  // is stored at slot k ^ 2*(tok & 7), so that the transposed reads (8 rows x
  // 32 bytes per half-wave) fall into distinct banks. Lane (g, r) of DMA u moves
  // row tok = 4u + g (page u / 4 of the pair), slot r; lane l of a DMA lands at
  // base + 16 l. A page id outside the pool (or past the context) is replaced
  // by page 0 for the loads and masked in the math.
  op ka[2][4];
  auto issue = [&](const int j, const int pa, const int pb) {
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint16_t* krow = k_pool + (size_t(h ? pb : pa) * IE_HIP_PAGE_SIZE + r) * kKvd + 8 * g;
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) ka[h][ks] = load_nt16<op>(krow + 32 * ks);
    }
    __builtin_amdgcn_sched_barrier(0);
    const unsigned tile = warea_lds + (j & 1) * kPair;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int tok = 4 * u + g;
      const int piece = r ^ (2 * (tok & 7));
      const uint16_t* src = v_pool +
          (size_t((u >> 2) ? pb : pa) * IE_HIP_PAGE_SIZE + (tok & 15)) * kKvd + 8 * piece;
      dma16_nt(src, tile + u * 1024);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  auto valid = [&](const int id) { return id >= 0 && id < num_pages; };
  // Page ids of the current pair (cur_*) and of the next one (nx_*).
  int cur_a = page_id(0), cur_b = page_id(1);
  int nx_a = page_id(2), nx_b = page_id(3);
  if (np > 0) issue(0, valid(cur_a) ? cur_a : 0, valid(cur_b) ? cur_b : 0);

  if constexpr (kFused) {
    if (app) {
      const float cs[8] = {tc0.x, tc0.y, tc0.z, tc0.w, tc1.x, tc1.y, tc1.z, tc1.w};
      const float sn[8] = {tn0.x, tn0.y, tn0.z, tn0.w, tn1.x, tn1.y, tn1.z, tn1.w};
      auto rotate = [&](float4& a0, float4& a1, float4& b0, float4& b1) {
        float x0[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
        float x1[8] = {b0.x, b0.y, b0.z, b0.w, b1.x, b1.y, b1.z, b1.w};
        float r0[8], r1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          r0[e] = __builtin_fmaf(x0[e], cs[e], -(x1[e] * sn[e]));  // x0*c - x1*s
          r1[e] = __builtin_fmaf(x1[e], cs[e], x0[e] * sn[e]);     // x1*c + x0*s
        }
        a0 = make_float4(r0[0], r0[1], r0[2], r0[3]);
        a1 = make_float4(r0[4], r0[5], r0[6], r0[7]);
        b0 = make_float4(r1[0], r1[1], r1[2], r1[3]);
        b1 = make_float4(r1[4], r1[5], r1[6], r1[7]);
      };
      rotate(q0a, q0b, q1a, q1b);
      if (own) {
#pragma unroll
        for (int hk = 0; hk < 2; ++hk) {  // KV head hk: dims 64 hk + (8g .. 8g+7, 32 + ..)
          rotate(kr[hk][0], kr[hk][1], kr[hk][2], kr[hk][3]);
          const float ra[8] = {kr[hk][0].x, kr[hk][0].y, kr[hk][0].z, kr[hk][0].w,
                               kr[hk][1].x, kr[hk][1].y, kr[hk][1].z, kr[hk][1].w};
          const float rb[8] = {kr[hk][2].x, kr[hk][2].y, kr[hk][2].z, kr[hk][2].w,
                               kr[hk][3].x, kr[hk][3].y, kr[hk][3].z, kr[hk][3].w};
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            kn[2 * hk][e] = __builtin_bit_cast(E, static_cast<uint16_t>(Kv<KV>::narrow(ra[e])));
            kn[2 * hk + 1][e] = __builtin_bit_cast(E, static_cast<uint16_t>(Kv<KV>::narrow(rb[e])));
          }
        }
        vn.x = Kv<KV>::narrow(vr0.x) | (Kv<KV>::narrow(vr0.y) << 16);
        vn.y = Kv<KV>::narrow(vr0.z) | (Kv<KV>::narrow(vr0.w) << 16);
        vn.z = Kv<KV>::narrow(vr1.x) | (Kv<KV>::narrow(vr1.y) << 16);
        vn.w = Kv<KV>::narrow(vr1.z) | (Kv<KV>::narrow(vr1.w) << 16);
        // The append itself: K slices from lanes (g, p % 16), V pieces from lanes
        // (0, r); skipped, like ie_hip_rope_and_cache, when the page is outside
        // the table row or the pool. The loads of pair 0 above read the slot's
        // old contents; the loop substitutes the new row for them.
        const int pid = page_id(off >> 4);
        if (pid >= 0 && pid < num_pages) {
          const size_t row = (size_t(pid) * IE_HIP_PAGE_SIZE + (p & 15)) * kKvd;
          if (r == (p & 15)) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
              *reinterpret_cast<op*>(fa.k_pool + row + 8 * g + 32 * ks) =
                  op{kn[ks][0], kn[ks][1], kn[ks][2], kn[ks][3],
                     kn[ks][4], kn[ks][5], kn[ks][6], kn[ks][7]};
          }
          if (g == 0) *reinterpret_cast<uint4*>(fa.v_pool + row + 8 * r) = vn;
        }
      }
    }
  }

  // Query times log2(e)/8, split into hi + lo, as the B operands of the 4
  // 32-dim steps of the 128-dim KV row: head r's values in the two steps of its
  // own KV head, zeros in the other two.
  op qhi[4], qlo[4];
  {
    const float qs = 0.125f * kLog2e;
    const float x[2][8] = {{q0a.x, q0a.y, q0a.z, q0a.w, q0b.x, q0b.y, q0b.z, q0b.w},
                           {q1a.x, q1a.y, q1a.z, q1a.w, q1b.x, q1b.y, q1b.z, q1b.w}};
    op h2[2], l2[2];
#pragma unroll
    for (int k = 0; k < 2; ++k)
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        E hi, lo;
        split16(x[k][j] * qs, hi, lo);
        h2[k][j] = hi;
        l2[k][j] = lo;
      }
    const op zero = {};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bool mine = (ks >> 1) == kv_r;
      qhi[ks] = mine ? h2[ks & 1] : zero;
      qlo[ks] = mine ? l2[ks & 1] : zero;
    }
  }

  // Per page pair j, as its data lands: scores, the pair's partial (max,
  // weights, sum, V^T P^T) and its fold, with the loads of pair j+1 issued as
  // soon as pair j's K registers are consumed, so a wave always has one pair in
  // flight while it computes.
  // Lane (g, r): head r; S^T element i of the pair's page h is token
  // 32 j + 16 h + 4g + i of the wave.
  float m = -INFINITY, l = 0.0f;  // running max (base 2) and this lane's part of the sum
  f32x4 o[8];                     // O^T tiles: lane (g, r) holds head r, dims 16 mt + 4g + e
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int rtok = 4 * g + (r >> 2);  // tile row this lane reads (first of the two reads)
  const int rsw = rtok & 7;           // its swizzle key
  const int rlo = (r & 1) * 8;        // byte within the 16-byte piece
  const int rpc = (r >> 1) & 1;       // piece parity within the 32-byte unit
  for (int j = 0; j < np; ++j) {
    // Outstanding: K and V of pair j (8 + 8 loads, in that order).
    wait_vmcnt<8>();
    if constexpr (kFused) {
      if (own && j == (off >> 5) && r == (p & 15)) {  // position p's K row: the new one
#pragma unroll
        for (int h = 0; h < 2; ++h)
          if (h == ((off >> 4) & 1)) {
#pragma unroll
            for (int ks = 0; ks < 4; ++ks)
              ka[h][ks] = op{kn[ks][0], kn[ks][1], kn[ks][2], kn[ks][3],
                             kn[ks][4], kn[ks][5], kn[ks][6], kn[ks][7]};
          }
      }
    }
    f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = sa;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      sa = M::mma(ka[0][ks], qhi[ks], sa);
      sa = M::mma(ka[0][ks], qlo[ks], sa);
      sb = M::mma(ka[1][ks], qhi[ks], sb);
      sb = M::mma(ka[1][ks], qlo[ks], sb);
    }
    const bool ok_a = valid(cur_a), ok_b = valid(cur_b);
    const bool more = j + 1 < np;
    if (more) {  // pair j+1: K into `ka` (just consumed), V into the other tile
      issue(j + 1, valid(nx_a) ? nx_a : 0, valid(nx_b) ? nx_b : 0);
      cur_a = nx_a;
      cur_b = nx_b;
      nx_a = page_id(2 * j + 4);
      nx_b = page_id(2 * j + 5);
    }
    const int tj = 32 * j;  // first token of the pair within the wave
    const bool full = tj + 32 <= nw && ok_a && ok_b;
    if (!full) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ta = tj + 4 * g + i, tb = ta + 16;
        sa[i] = (ok_a && ta < nw) ? sa[i] : -INFINITY;
        sb[i] = (ok_b && tb < nw) ? sb[i] : -INFINITY;
      }
    }
    // The pair's own partial: its max (per head), weights relative to it, their
    // sum (this lane's part) and V^T P^T from zero, folded into the running
    // result by fold_pair. Each pair's partial depends on the pair alone, so a
    // chunk's result is the same whether one wave folds its pairs as they come
    // or several waves take one pair each and one of them folds the others'.
    float mx = max_nn(max3_nn(sa[0], sa[1], sa[2]),
                      max3_nn(max3_nn(sa[3], sb[0], sb[1]), sb[2], sb[3]));
    mx = group_max4(mx);
    const float mref = mx == -INFINITY ? 0.0f : mx;  // nothing visible: weights 0
    op phi, plo;
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ea = exp2_weight(sa[i] - mref), eb = exp2_weight(sb[i] - mref);
      sum += ea + eb;
      E ha, la, hb, lb;
      split16(ea, ha, la);
      split16(eb, hb, lb);
      phi[i] = ha;
      phi[4 + i] = hb;
      plo[i] = la;
      plo[4 + i] = lb;
    }

    // V^T of the pair: two transposing reads per 16-dim tile; in each 16-lane
    // group, lane 4a+b receives element b of the 8-byte reads of lanes a,
    // a+4, a+8, a+12. Lane L reads tile row 4g + L/4, dims 16 mt + 4 (L%4)..+3,
    // so lane r receives dim 16 mt + r of rows 4g..4g+3 (and 16+4g.. for the
    // second read): the A operand, token slots matching P^T's.
    if (more)
      wait_vmcnt<16>();  // V of pair j has landed; pair j+1 (16 loads) may be in flight
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    if constexpr (kFused) {
      // Position p's V row in the tile: the new one (ahead of the transposed
      // reads below in the wave's LDS queue).
      if (own && j == (off >> 5) && g == 0) {
        const int tok = off & 31;
        *reinterpret_cast<uint4*>(warea + (j & 1) * kPair + tok * 256 +
                                  16 * (r ^ (2 * (tok & 7)))) = vn;
      }
    }
    unsigned long long keep_lo = ~0ull, keep_hi = ~0ull;
    if (!full) {  // 0 * (stale inf or NaN) is not 0: zero masked V elements
      keep_lo = keep_hi = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int ta = tj + 4 * g + i, tb = ta + 16;
        if (ok_a && ta < nw) keep_lo |= 0xFFFFull << (16 * i);
        if (ok_b && tb < nw) keep_hi |= 0xFFFFull << (16 * i);
      }
    }
    const unsigned char* vt = warea + (j & 1) * kPair + rtok * 256 + rlo;
    f32x4 pv[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      const int slot = 2 * (mt ^ rsw) + rpc;
      s16x4 lo4 = lds_read_tr16(vt + slot * 16);
      s16x4 hi4 = lds_read_tr16(vt + 16 * 256 + slot * 16);
      if (!full) {
        lo4 = __builtin_bit_cast(s16x4, __builtin_bit_cast(unsigned long long, lo4) & keep_lo);
        hi4 = __builtin_bit_cast(s16x4, __builtin_bit_cast(unsigned long long, hi4) & keep_hi);
      }
      const op a = join_tr<op>(lo4, hi4);
      pv[mt] = M::mma(a, phi, f32x4{0.f, 0.f, 0.f, 0.f});
      pv[mt] = M::mma(a, plo, pv[mt]);
    }
    fold_pair(m, l, o, mx, sum, pv);
  }
  if constexpr (!kOneWave) {
    // One pair per wave: waves 1.. hand their pair's partial to wave 0 through
    // their own LDS area (their V reads are done), and wave 0 folds them in pair
    // order -- the fold one wave makes over the same pairs.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    if (wave > 0) {
      f32x4* xo = reinterpret_cast<f32x4*>(warea);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) xo[mt * 64 + lane] = o[mt];
      reinterpret_cast<float2*>(warea + kOutTile * 2)[lane] = make_float2(m, l);
    }
    __syncthreads();
    if (wave > 0) return;
    for (int w = 1; w < waves; ++w) {
      const unsigned char* wa = smem + size_t(w) * kTile;
      const float2 ml = reinterpret_cast<const float2*>(wa + kOutTile * 2)[lane];
      f32x4 ow[8];
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) ow[mt] = reinterpret_cast<const f32x4*>(wa)[mt * 64 + lane];
      fold_pair(m, l, o, ml.x, ml.y, ow);
    }
  }
  l = group_sum4(l);

  // 3. Head r's 64 output dims: tiles 4 kv_r .. 4 kv_r + 3 (its own KV head),
  //    lane group g holding dims 16 j + 4g .. +3 of tile j.
  f32x4 od[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) od[j] = kv_r ? o[4 + j] : o[j];

  // The chunk's result per (head h, dims 4 d4 .. 4 d4 + 3): a row that fits one
  // chunk writes `out`; otherwise the chunk's partial (o unnormalised, m in
  // log2 units, l) goes to the workspace for decode_merge_kernel.
  auto emit = [&](const int h, const int d4, const f32x4 acc, const float mh, const float lh) {
    const size_t head = size_t(t) * n_heads + h;
    if (single) {
      *reinterpret_cast<f32x4*>(out + head * 64 + 4 * d4) = acc * (1.0f / lh);
    } else {
      const size_t slot = head * num_chunks + c;
      *reinterpret_cast<f32x4*>(part_o + slot * 64 + 4 * d4) = acc;
      if (d4 == 0) *reinterpret_cast<float2*>(part_ml + 2 * slot) = make_float2(mh, lh);
    }
  };
  if (head_ok) {
#pragma unroll
    for (int j = 0; j < 4; ++j) emit(r, 4 * j + g, od[j], m, l);
  }
}


// ---------------------------------------------------------------------------
// float32 KV caches: the same products on v_mfma_f32_16x16x4_f32 (full fp32
// operands, so no hi + lo split), one 16-token page at a time.
//   S^T[16 tok x 16 heads] = K_page[16 x 128] . Qbd^T[128 x 16]: 32 steps of 4
//     dims. The reduction order is free, so step s takes dims 32g + s for the
//     4 lane groups g: lane (g, r) holds token r's dims 32g .. 32g+31 (128
//     contiguous bytes, 8 16-byte loads) and, as B, head r's query at the same
//     dims of the block-diagonal Qbd (zero outside its own KV head).
//   O^T[128 dims x 16 heads] += V^T[128 x 16 tok] . P^T[16 tok x 16 heads]: 8
//     tiles of 16 dims, 4 steps of 4 tokens. Step s takes tokens 4g + s, so
//     the B operand of lane (g, r) is its own weight of token 4g + s (the S^T
//     result it already holds). Row i of tile mt is dim 4i + mt (mt < 4) or
//     64 + 4i + mt - 4: lane (g, r) reads dims 4r .. 4r+3 and 64 + 4r .. +3 of
//     token 4g + s, two 16-byte LDS reads that 16 lanes take from 256
//     contiguous bytes, and ends up holding head r's dims 16g + 4t + e of its
//     own KV head's 64 (o[4 kv_r + e][t]).
// K goes straight into registers; V into LDS by DMA (8 KB per page, two page
// buffers per wave), the next page's loads in flight while the wave computes.
// One wave per (row, chunk); the grid is numbered as for the 16-bit kernel.
constexpr int kPageF32 = 16 * kKvd * 4;  // bytes of one f32 page of one pool

__global__ void __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(3)))
decode_partial_mfma_f32(float* __restrict__ out, float* __restrict__ part_o,
                        float* __restrict__ part_ml, const float* __restrict__ q,
                        const float* __restrict__ k_pool, const float* __restrict__ v_pool,
                        const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                        const int32_t* __restrict__ tables, int T, int max_pages, int num_pages,
                        int n_heads, int group, int num_chunks, int chunk_tokens,
                        const int32_t* __restrict__ plan) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x;
  const int g = lane >> 4, r = lane & 15;
  // Which (row, chunk) this workgroup takes and the chunk's page ids, one per
  // lane: from a host-built work list in one round trip (header, item and the
  // lane's page id loaded together, as in the 16-bit kernel, with the same
  // checks of the list against the launch), or located from row_pos and then
  // read from the row's table (two dependent round trips).
  int t, c, p, seq;
  int pid_plan = -1;
  if (plan) {
    const int32_t* item = plan + kPlanHeader + size_t(blockIdx.x) * plan_stride(chunk_tokens);
    pid_plan = lane < chunk_tokens / IE_HIP_PAGE_SIZE ? item[4 + lane] : -1;
    const int4 head = *reinterpret_cast<const int4*>(plan);  // [items, chunk, chunks, rows]
    const int items = __builtin_amdgcn_readfirstlane(head.x);
    t = __builtin_amdgcn_readfirstlane(item[0]);
    c = __builtin_amdgcn_readfirstlane(item[1]);
    p = __builtin_amdgcn_readfirstlane(item[2]);
    seq = __builtin_amdgcn_readfirstlane(item[3]);
    if (int(blockIdx.x) >= items) return;  // past the plan's last item
    if (__builtin_amdgcn_readfirstlane(head.y) != chunk_tokens ||
        __builtin_amdgcn_readfirstlane(head.z) != num_chunks ||
        __builtin_amdgcn_readfirstlane(head.w) != T || t < 0 || t >= T || c < 0 ||
        c >= num_chunks || p < c * chunk_tokens)
      return;  // a list built for another launch, or an item outside this one: nothing written
  } else if (!locate_chunk(blockIdx.x, T, row_pos, row_seq, num_chunks, chunk_tokens, lane, t, c,
                           p, seq)) {
    return;  // past the batch's last chunk
  }
  const int s0 = c * chunk_tokens;
  const int n = min(s0 + chunk_tokens, p + 1) - s0;  // positions of this chunk
  // The row has one chunk (its context fits one, or the caller sized one):
  // written here; the merge skips it, reading the same count.
  const bool single = min(p / chunk_tokens + 1, num_chunks) == 1;
  const int npg = (n + IE_HIP_PAGE_SIZE - 1) / IE_HIP_PAGE_SIZE;
  // Page ids of the chunk (at most 64 pages), one per lane, loaded once and read
  // per page with readlane (no table load waits inside the page loop), as in
  // the 16-bit kernel.
  const int pi0 = s0 / IE_HIP_PAGE_SIZE;
  const int32_t* row_tab = tables + size_t(seq) * max_pages;
  const int pid_lane = plan ? (16 * lane < n ? pid_plan : -1)
                            : (16 * lane < n && pi0 + lane < max_pages) ? row_tab[pi0 + lane] : -1;
  auto page_id = [&](const int pw) -> int {
    return pw < 64 ? __builtin_amdgcn_readlane(pid_lane, pw) : -1;
  };
  auto valid = [&](const int id) { return id >= 0 && id < num_pages; };

  // Head r's query, times log2(e)/8, at dims 32 (g & 1) .. +31 of its head when
  // g / 2 is its KV head (the B operands of the 32 score steps), else zeros.
  // Every lane loads (a head in range) before page 0's loads go out, and zeros
  // what is not its own after: the loads travel together, unpredicated.
  const bool head_ok = r < n_heads;
  const int kv_r = r >= group;
  const bool mine = head_ok && (g >> 1) == kv_r;
  float4 qx[8];
  {
    const float4* qrow = reinterpret_cast<const float4*>(
        q + (size_t(t) * n_heads + (head_ok ? r : 0)) * 64 + 32 * (g & 1));
#pragma unroll
    for (int i = 0; i < 8; ++i) qx[i] = qrow[i];
  }

  // Loads of page j: K (token r, dims 32g..+31) into `kv`, V by DMA into LDS
  // buffer j & 1 in row-major order (load u moves tokens 2u, 2u+1; lane l's 16
  // bytes land at base + 16 l). A page outside the pool loads page 0 and is
  // masked in the math.
  float4 kv[8];
  const unsigned vbuf_lds = lds_address(smem);
  auto issue = [&](const int j, const int pid) {
    __builtin_amdgcn_sched_barrier(0);
    const float4* krow =
        reinterpret_cast<const float4*>(k_pool + (size_t(pid) * IE_HIP_PAGE_SIZE + r) * kKvd + 32 * g);
#pragma unroll
    for (int i = 0; i < 8; ++i) kv[i] = krow[i];  // 8 loads per 128-byte span: cached
    __builtin_amdgcn_sched_barrier(0);
    const char* vsrc = reinterpret_cast<const char*>(v_pool) + size_t(pid) * kPageF32 + 16 * lane;
    const unsigned dst = vbuf_lds + (j & 1) * kPageF32;
#pragma unroll
    for (int u = 0; u < 8; ++u) dma16_nt(vsrc + u * 1024, dst + u * 1024);
    __builtin_amdgcn_sched_barrier(0);
  };
  int cur = page_id(0), nxt = page_id(1);
  issue(0, valid(cur) ? cur : 0);  // a located chunk has at least one position
  float qb[32];
  {
    const float qm = mine ? 0.125f * kLog2e : 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      qb[4 * i + 0] = qx[i].x * qm;
      qb[4 * i + 1] = qx[i].y * qm;
      qb[4 * i + 2] = qx[i].z * qm;
      qb[4 * i + 3] = qx[i].w * qm;
    }
  }

  float m = -INFINITY, l = 0.0f;  // running max (base 2) and this lane's part of the sum
  f32x4 o[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int j = 0; j < npg; ++j) {
    // S^T of page j: lane (g, r) gets tokens 4g + e of head r.
    f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i].x, qb[4 * i + 0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i].y, qb[4 * i + 1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i].z, qb[4 * i + 2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[i].w, qb[4 * i + 3], s, 0, 0, 0);
    }
    const bool ok = valid(cur);
    const bool more = j + 1 < npg;
    if (more) {  // page j+1: K into `kv` (just consumed), V into the other buffer
      issue(j + 1, valid(nxt) ? nxt : 0);
      cur = nxt;
      nxt = page_id(j + 2);
    }
    const int tj = 16 * j;  // first token of the page within the chunk
    const bool full = tj + 16 <= n && ok;
    if (!full) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s[e] = (ok && tj + 4 * g + e < n) ? s[e] : -INFINITY;
    }
    const float mx = group_max4(fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3])));
    const float m_new = fmaxf(m, mx);
    const float mref = m_new == -INFINITY ? 0.0f : m_new;  // all masked so far: weights 0
    float pw[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) pw[e] = exp2_weight(s[e] - mref);
    const float corr = exp2_weight(m - mref);  // m = -inf (nothing seen yet): 0
    l = __builtin_fmaf(l, corr, (pw[0] + pw[1]) + (pw[2] + pw[3]));
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) o[mt] *= corr;
    m = m_new;

    // V of page j has landed once only page j+1's 16 loads may remain.
    if (more)
      wait_vmcnt<16>();
    else
      wait_vmcnt<0>();
    const float* vt = reinterpret_cast<const float*>(smem + (j & 1) * kPageF32);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int tok = 4 * g + e;
      float4 va = *reinterpret_cast<const float4*>(vt + tok * kKvd + 4 * r);
      float4 vb = *reinterpret_cast<const float4*>(vt + tok * kKvd + 64 + 4 * r);
      if (!full && !(ok && tj + tok < n)) {  // 0 * (stale inf or NaN) is not 0
        va = make_float4(0.f, 0.f, 0.f, 0.f);
        vb = va;
      }
      o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.x, pw[e], o[0], 0, 0, 0);
      o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.y, pw[e], o[1], 0, 0, 0);
      o[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.z, pw[e], o[2], 0, 0, 0);
      o[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(va.w, pw[e], o[3], 0, 0, 0);
      o[4] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb.x, pw[e], o[4], 0, 0, 0);
      o[5] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb.y, pw[e], o[5], 0, 0, 0);
      o[6] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb.z, pw[e], o[6], 0, 0, 0);
      o[7] = __builtin_amdgcn_mfma_f32_16x16x4f32(vb.w, pw[e], o[7], 0, 0, 0);
    }
  }
  l = group_sum4(l);
  if (!head_ok) return;
  // Head r's dims 16g + 4e' .. +3 of its own KV head: o[4 kv_r + 0..3][e'].
  const size_t head = size_t(t) * n_heads + r;
  const int b = 4 * kv_r;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const f32x4 v = {o[b][e], o[b + 1][e], o[b + 2][e], o[b + 3][e]};
    const int d = 16 * g + 4 * e;
    if (single) {
      *reinterpret_cast<f32x4*>(out + head * 64 + d) = v * (1.0f / l);
    } else {
      const size_t slot = head * num_chunks + c;
      *reinterpret_cast<f32x4*>(part_o + slot * 64 + d) = v;
    }
  }
  if (!single && g == 0) {
    const size_t slot = head * num_chunks + c;
    *reinterpret_cast<float2*>(part_ml + 2 * slot) = make_float2(m, l);
  }
}

}  // namespace

bool decode_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                           int chunk_tokens) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16) && head_dim == 64 &&
         n_kv_heads * head_dim == kKvd && n_heads <= 16 &&
         n_heads % n_kv_heads == 0 && chunk_tokens % 64 == 0 && chunk_tokens >= 64 &&
         chunk_tokens <= 1024;
}

// Waves per workgroup for a chunk. One wave streams the chunk as page pairs,
// one pair in flight while it computes the previous one: that hides latency
// when the grid is large. When the grid gives fewer than two workgroups per
// compute unit (few, long rows), a chunk of 2 to 8 pairs takes one wave per
// pair instead, every pair in flight at once. Either way the pairs' partials
// are folded in pair order by the same function (fold_pair), so the choice
// changes the timing and never the result.
static int decode_mfma_waves(int chunk_tokens, int64_t slots) {
  const bool small_grid = slots < 2 * int64_t(device_compute_units());
  if (small_grid && chunk_tokens >= 64 && chunk_tokens <= 32 * kMaxWaves) return chunk_tokens / 32;
  return 1;
}

int decode_mfma(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                int num_chunks, int chunk_tokens, void* workspace, int n_heads, int n_kv_heads,
                hipStream_t stream, const FusedAppend* fused, const int32_t* plan) {
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  const int64_t slots = int64_t(T) * num_chunks;  // upper bound on the non-empty chunks
  const int waves = decode_mfma_waves(chunk_tokens, slots);
  const size_t lds = size_t(waves) * kTile;
  if (chunk_tokens / waves > 1024)  // a wave's page ids live one per lane
    return fail(IE_HIP_EINVAL, "attention: more than 1,024 positions per wave");
  if (slots * n_heads * 64 * 4 > 0x7fffffff)
    return fail(IE_HIP_EINVAL, "attention: split-K workspace above 2 GB (too many rows x chunks)");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return fail(IE_HIP_EINVAL, "attention: q, out and the pools must be 16-byte aligned");
  const dim3 grid(static_cast<unsigned>(slots)), block(64 * waves);
  const int group = n_heads / n_kv_heads;
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  // 8 waves (1024-token chunks) take 128 KB of LDS: above the 64 KB default cap
  // for dynamic LDS, within gfx950's 160 KB per workgroup. Raised once per kernel.
  const FusedAppend fa = fused ? *fused : FusedAppend{};
#define IE_DECODE_LAUNCH(KVT, ONE, FUSED)                                                         \
  do {                                                                                            \
    if (!(ONE)) {                                                                                 \
      static const hipError_t attr = hipFuncSetAttribute(                                         \
          reinterpret_cast<const void*>(decode_partial_mfma<KVT, ONE, FUSED>),                    \
          hipFuncAttributeMaxDynamicSharedMemorySize, kMaxLds);                                   \
      if (int rc = check_hip(attr, "hipFuncSetAttribute(attention_partial_mfma)")) return rc;     \
    }                                                                                             \
    hipLaunchKernelGGL((decode_partial_mfma<KVT, ONE, FUSED>), grid, block, lds, stream, out,     \
                       ws.part_o, ws.part_ml, q, kp, vp, row_pos, row_seq, kv.tables, T,          \
                       kv.max_pages, kv.num_pages, n_heads, group, num_chunks, chunk_tokens, fa,  \
                       plan);                                                                     \
  } while (0)
#define IE_DECODE_LAUNCH_KV(KVT)                 \
  if (fused) {                                   \
    if (waves == 1)                              \
      IE_DECODE_LAUNCH(KVT, true, true);         \
    else                                         \
      IE_DECODE_LAUNCH(KVT, false, true);        \
  } else {                                       \
    if (waves == 1)                              \
      IE_DECODE_LAUNCH(KVT, true, false);        \
    else                                         \
      IE_DECODE_LAUNCH(KVT, false, false);       \
  }
  if (kv.kv_dtype == IE_KV_F16) {
    IE_DECODE_LAUNCH_KV(IE_KV_F16)
  } else {
    IE_DECODE_LAUNCH_KV(IE_KV_BF16)
  }
#undef IE_DECODE_LAUNCH_KV
#undef IE_DECODE_LAUNCH
  if (int rc = check_launch("attention_mfma")) return rc;
  return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
}

}  // namespace iehip

namespace iehip {

bool decode_mfma_f32_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim,
                               int chunk_tokens) {
  return kv_dtype == IE_KV_F32 && head_dim == 64 && n_kv_heads * head_dim == kKvd &&
         n_heads <= 16 && n_heads % n_kv_heads == 0 && chunk_tokens % IE_HIP_PAGE_SIZE == 0 &&
         chunk_tokens >= IE_HIP_PAGE_SIZE && chunk_tokens <= 1024;
}

int decode_mfma_f32(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                    const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                    int num_chunks, int chunk_tokens, void* workspace, int n_heads,
                    int n_kv_heads, hipStream_t stream, const int32_t* plan) {
  const Workspace ws = carve_workspace(workspace, T, n_heads, 64, num_chunks);
  const int64_t slots = int64_t(T) * num_chunks;  // upper bound on the non-empty chunks
  if (slots * n_heads * 64 * 4 > 0x7fffffff)
    return fail(IE_HIP_EINVAL, "attention: split-K workspace above 2 GB (too many rows x chunks)");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k_pool) |
       reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return fail(IE_HIP_EINVAL, "attention: q, out and the pools must be 16-byte aligned");
  hipLaunchKernelGGL(decode_partial_mfma_f32, dim3(static_cast<unsigned>(slots)), dim3(64),
                     2 * kPageF32, stream, out, ws.part_o, ws.part_ml, q,
                     static_cast<const float*>(k_pool), static_cast<const float*>(v_pool), row_pos,
                     row_seq, kv.tables, T, kv.max_pages, kv.num_pages, n_heads,
                     n_heads / n_kv_heads, num_chunks, chunk_tokens, plan);
  if (int rc = check_launch("attention_mfma_f32")) return rc;
  return decode_merge(out, ws, row_pos, T, n_heads, num_chunks, chunk_tokens, stream);
}

}  // namespace iehip
