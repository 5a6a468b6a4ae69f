// Chunked-prefill attention into pages on the matrix cores (gfx950), for KV
// caches of every type with head_dim 64: 16-bit caches on the 16-bit
// instructions (prefill_mfma_kernel), f32 caches on the f32 ones
// (prefill_mfma_f32_kernel, further down).
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
// Precision: K and V enter exactly. With an f16 cache, q (pre-scaled by
// log2(e)/8) and P (weights <= 2^kLazyMax) enter as single f16 values rounded
// to nearest -- the operand rounding of the reference's tensor-core kernel
// (src/cuda/kernels.cu:673-674,741), here with the row sums taken from the same
// rounded P on the matrix cores, so the output is a weighted mean with weights
// off by <= 2^-11 relative (errors ~6e-4 at 4,000 keys against the 2e-3
// absolute bound). bf16 keeps 8 mantissa bits, too few for that bound:
// with a bf16 cache q and P are split into hi + lo halves and each product is
// done twice (float32-level scores and weights, errors ~1e-6).
//
// Layout of the work:
//   One workgroup per (pair of 16-row blocks, KV head); one wave per query head
//   of the KV head (the 7 heads of a Qwen2.5 group share every K/V tile through
//   LDS). Two heads per wave (each K/V operand feeding both) was measured
//   slower: half the waves leave the dependency and barrier stalls exposed.
//   The pair is block b and block n-1-b: the causal triangle gives block b b+1
//   key tiles of work, so every pair carries about the same total and the
//   ceil(n/2) x n_kv_heads workgroups finish together (the heavier block goes
//   first). When that grid leaves compute units with at most one workgroup,
//   two teams of waves split each block's key tiles (even and odd) and merge
//   their (m, l, O) through LDS at the end.
//   K/V tiles of 64 keys (4 pages, 16 KB) go through an LDS ring by DMA
//   (global_load_lds_dwordx4, 16 x 1 KB per tile spread over 4 waves of a team):
//   4 tiles with one team, 3 steps of 2 tiles with two. The page ids of up to
//   512 tiles are staged in LDS at a block's start (scalar loads of the table
//   inside the loop would share lgkmcnt with the K reads and put the table's
//   round trip on every step). K rows are stored with their 16-byte pieces
//   swizzled (piece ^ (row/2 % 8)) so the A-operand reads (16 rows, one piece each) hit
//   distinct banks; V rows with piece ^ 2*(row/2 % 4) so the transposed reads
//   (ds_read_b64_tr_b16: 8 rows x 32 bytes per half-wave) do.
//   Keys past the block's last position and pages outside the pool are masked
//   (-inf scores, and their V rows zeroed in LDS before use, so stale or
//   non-finite memory cannot reach the output through 0 * x).
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "mfma.hpp"
#include "prefill.hpp"

namespace iehip {
namespace {

constexpr int kRows = 16;                  // query rows per block (one MFMA column tile)
constexpr int kKeys = 64;                  // keys per LDS tile
constexpr int kTileBytes = kKeys * 128;    // 64 keys x 64 dims x 2 B
constexpr int kBufBytes = 2 * kTileBytes;  // K tile + V tile
constexpr int kMaxGroup = 8;
constexpr int kHeadsPerWave = 1;           // query heads per wave (2 measured slower: fewer waves)
static_assert(kHeadsPerWave == 1, "the team exchange hands over one head per wave");
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLazyMax = 8.0f;           // log2 headroom of the lazily raised softmax max
constexpr float kSumMax = 16384.0f;        // largest tile row sum taken without a new max
constexpr int kSegTiles = 512;             // key tiles (32,768 keys) with page ids in LDS at once
constexpr int kRopeStride = 68;            // floats per staged RoPE row (64 + 4 of padding)

// kWaves = group / kHeadsPerWave waves per team (rounded up), wave w of a team
// taking query heads kHeadsPerWave * w .. of the KV head. kTeams teams of
// kWaves waves split each block's key tiles (team t takes tiles kTeams s + t)
// and merge their (m, l, O) through LDS at the end of the block.
template <int KV, int kWaves, int kTeams, bool kSplitF16>
__global__ void __launch_bounds__(64 * kWaves * kTeams)
prefill_mfma_kernel(float* __restrict__ out, const float* __restrict__ q,
                    const uint16_t* __restrict__ k_pool, const uint16_t* __restrict__ v_pool,
                    int T, const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                    const int32_t* __restrict__ tables, int max_pages, int num_pages, int n_heads,
                    int n_kv_heads, int n_blocks, const float* __restrict__ rope,
                    int rope_positions) {
  using M = Mfma<KV>;
  using op = typename M::op;
  using E = typename M::elem;
  // hi + lo operands: always for bf16; for f16 under IE_HIP_PREFILL_SPLIT.
  constexpr bool kSplit = kSplitF16 || !std::is_same_v<E, _Float16>;
  constexpr int kRingSteps = kTeams == 1 ? 4 : 3;  // steps of kTeams tiles in LDS
  static_assert(kSegTiles % kTeams == 0, "a step's tiles never straddle two segments");
  constexpr int kRingBytes = kRingSteps * kTeams * kBufBytes;
  op ones;  // all-ones A operand: row sums of P^T on the matrix cores
#pragma unroll
  for (int i = 0; i < 8; ++i) ones[i] = static_cast<E>(1.0f);
  // A tile's 16 loads of 1 KB, spread evenly over kDmaWaves waves of its team.
  constexpr int kDmaWaves = kWaves >= 4 ? 4 : kWaves >= 2 ? 2 : 1;
  constexpr int kPerWave = 16 / kDmaWaves;
  extern __shared__ __align__(16) unsigned char smem[];
  const int group = n_heads / n_kv_heads;
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int team = wave_id / kWaves, wave = wave_id - team * kWaves;
  const int g = lane >> 4, r = lane & 15;
  const int h0 = kvh * group + kHeadsPerWave * wave;       // this wave's first head
  const int nh = min(kHeadsPerWave, group - kHeadsPerWave * wave);  // 1 or 2 (uniform)
  const int kv_dim = n_kv_heads * 64;
  const int pos0 = __builtin_amdgcn_readfirstlane(row_pos[0]);
  const int seq = __builtin_amdgcn_readfirstlane(row_seq[0]);
  const int32_t* tab = tables + size_t(seq) * max_pages;

  // The page ids of a segment of key tiles, staged in LDS after the ring by all
  // threads at the segment's start: ids[4 (tile - seg0) + j] is page j of the
  // tile, or -1 for a page past the table row or outside the pool (loaded as
  // page 0 and masked). A step then reads its tiles' ids from LDS instead of
  // the table: no memory round trip inside the tile loop.
  int* const ids = reinterpret_cast<int*>(smem + kRingBytes);
  // Per step of the segment, staged after the ids: bits 4 tm .. 4 tm + 3 = the
  // in-pool bits of team tm's tile, bit 8 = some tile of the step needs V rows
  // zeroed (past max_pos or a page outside the pool). One LDS read per step.
  int* const step_flags = ids + 4 * (kSegTiles + kTeams);
  // With a RoPE table: the cos/sin rows of the block's 16 positions, staged once
  // per block after the step flags and read by every wave; rows kRopeStride
  // floats apart (64 + 4), so that the 16 rows one lane group reads at the same
  // offset fall into different banks.
  float* const rope_rows = reinterpret_cast<float*>(step_flags + kSegTiles);
  int seg0 = 0;  // first tile of the segment in progress
  auto tile_ids = [&](const int tile) {
    return *reinterpret_cast<const int4*>(ids + 4 * (tile - seg0));
  };
  // Buffer of the tile a team takes at step s.
  auto buffer = [&](const int ring_step, const int tm) { return ring_step * kTeams + tm; };

  // DMA of a tile into buffer `buf`: 8 K loads and 8 V loads of 1 KB (8 key rows
  // of 128 bytes each), the same kPerWave for every tile, so a wave can wait for
  // "all but the newest steps" by count. Load u (rows 8u .. 8u+7) lands lane l at
  // base + 16 l: key row 8u + l/8, LDS slot l % 8, holding the global piece the
  // row's swizzle maps to that slot (K: piece ^ (row/2 % 8); V: piece ^ 2*(row/2 % 4)).
  // Per-lane byte offsets (row & 15 = 8 (u & 1) + l / 8) depend only on u & 1.
  const int row_bytes = kv_dim * 2;
  const int lrow = lane >> 3, lslot = lane & 7;
  int koff[2], voff[2];
#pragma unroll
  for (int odd = 0; odd < 2; ++odd) {
    const int row15 = 8 * odd + lrow;
    koff[odd] = row15 * row_bytes + 16 * (lslot ^ (4 * odd + (lrow >> 1)));
    voff[odd] = row15 * row_bytes + 16 * (lslot ^ (2 * (lrow >> 1)));
  }
  const unsigned smem_lds = lds_address(smem);
  const char* kbase_g = reinterpret_cast<const char*>(k_pool) + kvh * 128;
  const char* vbase_g = reinterpret_cast<const char*>(v_pool) + kvh * 128;
  const size_t page_bytes = size_t(IE_HIP_PAGE_SIZE) * row_bytes;
  auto issue = [&](const int buf, const int tile) {
    if (wave >= kDmaWaves) return;
    const int4 v = tile_ids(tile);
    const int id[4] = {max(__builtin_amdgcn_readfirstlane(v.x), 0),
                       max(__builtin_amdgcn_readfirstlane(v.y), 0),
                       max(__builtin_amdgcn_readfirstlane(v.z), 0),
                       max(__builtin_amdgcn_readfirstlane(v.w), 0)};
    // Quarter qt of the loads: qt = 0, 1 the K rows 0-31, 32-63; qt = 2, 3 the V rows.
#pragma unroll
    for (int k = 0; k < 4 / kDmaWaves; ++k) {
      const int qt = wave + k * kDmaWaves;
      const bool is_v = qt >= 2;
      const int half = qt & 1;  // rows 32 half .. 32 half + 31: pages 2 half, 2 half + 1
      const int ida = half ? id[2] : id[0], idb = half ? id[3] : id[1];
      const char* base = is_v ? vbase_g : kbase_g;
      const char* pa = base + size_t(ida) * page_bytes;
      const char* pb = base + size_t(idb) * page_bytes;
      const unsigned dst = smem_lds + buf * kBufBytes + (is_v ? kTileBytes : 0) + half * 4096;
#pragma unroll
      for (int j = 0; j < 4; ++j) {  // u = 4 half + j: page u / 2 of the tile
        const int off = is_v ? voff[j & 1] : koff[j & 1];
        dma16(((j >> 1) ? pb : pa) + off, dst + j * 1024);
      }
    }
  };
  // Wait until this wave's loads of all but the newest `newer` steps have landed.
  auto wait_steps = [&](const int newer) {
    if (newer >= 2) wait_vmcnt<2 * kPerWave>();
    else if (newer == 1) wait_vmcnt<kPerWave>();
    else wait_vmcnt<0>();
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

    // Queries of row t0 + r for the wave's heads, times log2(e)/8 (split hi + lo
    // for bf16): the B operands of S^T (dims 32 ks + 8g .. +8). Their loads (and
    // the RoPE table rows') are issued here and turned into operands (make_q) only
    // after the block's first page-id staging is under way, so that the query's
    // round trip and the table's overlap instead of following each other.
    const int t = t0 + r;
    const bool row_ok = t < T;
    const int rp = pos0 + t;  // this lane's row position
    float4 qa[kHeadsPerWave][2][2];
#pragma unroll
    for (int hh = 0; hh < kHeadsPerWave; ++hh)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        qa[hh][ks][0] = qa[hh][ks][1] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (row_ok && hh < nh) {
          const float4* src = reinterpret_cast<const float4*>(
              q + (size_t(t) * n_heads + h0 + hh) * 64 + 32 * ks + 8 * g);
          qa[hh][ks][0] = src[0];
          qa[hh][ks][1] = src[1];
        }
      }
    // With a RoPE table (ie_hip_rope_cache_attention_prefill) q arrives unrotated,
    // and the rotation ie_hip_rope_and_cache would have applied in place happens
    // in make_q: lane (g, r) holds dims 8g + j and 32 + 8g + j, the rotation
    // pairs, and takes cos/sin of its row's position from the table; the same
    // fmaf in the same order, so the same float32 values. Rows whose position
    // lies outside the table are used unrotated, as there. The table is read for
    // every lane (row 0's entries where the row is not rotated), the rotation
    // applied by selection.
    const bool rot = rope && row_ok && rp >= 0 && rp < rope_positions;
    op qhi[kHeadsPerWave][2], qlo[kHeadsPerWave][2];
    auto make_q = [&]() {
      float4 tcs[4] = {};  // cos of dims 8g .. 8g+7, then sin (rows staged in LDS)
      if (rope) {
        const float* trow = rope_rows + r * kRopeStride + 8 * g;
        tcs[0] = *reinterpret_cast<const float4*>(trow);
        tcs[1] = *reinterpret_cast<const float4*>(trow + 4);
        tcs[2] = *reinterpret_cast<const float4*>(trow + 32);
        tcs[3] = *reinterpret_cast<const float4*>(trow + 36);
      }
#pragma unroll
      for (int hh = 0; hh < kHeadsPerWave; ++hh) {
        float x[2][8] = {{qa[hh][0][0].x, qa[hh][0][0].y, qa[hh][0][0].z, qa[hh][0][0].w,
                          qa[hh][0][1].x, qa[hh][0][1].y, qa[hh][0][1].z, qa[hh][0][1].w},
                         {qa[hh][1][0].x, qa[hh][1][0].y, qa[hh][1][0].z, qa[hh][1][0].w,
                          qa[hh][1][1].x, qa[hh][1][1].y, qa[hh][1][1].z, qa[hh][1][1].w}};
        if (rope) {
          const float cs[8] = {tcs[0].x, tcs[0].y, tcs[0].z, tcs[0].w,
                               tcs[1].x, tcs[1].y, tcs[1].z, tcs[1].w};
          const float sn[8] = {tcs[2].x, tcs[2].y, tcs[2].z, tcs[2].w,
                               tcs[3].x, tcs[3].y, tcs[3].z, tcs[3].w};
          const bool on = rot && hh < nh;
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const float x0 = x[0][j], x1 = x[1][j];
            const float r0 = __builtin_fmaf(x0, cs[j], -(x1 * sn[j]));  // x0*c - x1*s
            const float r1 = __builtin_fmaf(x1, cs[j], x0 * sn[j]);     // x1*c + x0*s
            x[0][j] = on ? r0 : x0;
            x[1][j] = on ? r1 : x1;
          }
        }
        const float qs = 0.125f * kLog2e;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            E hv, lv = static_cast<E>(0.0f);
            if constexpr (kSplit) {
              split16(x[ks][j] * qs, hv, lv);
            } else {
              // The float32 product, then its f16 rounding: kept opaque so that no
              // instantiation folds the two into one mixed-precision fma (a single
              // rounding of the exact product), whether q was rotated here or not.
              float xq = x[ks][j] * qs;
              asm("" : "+v"(xq));
              hv = static_cast<E>(xq);
            }
            qhi[hh][ks][j] = hv;
            qlo[hh][ks][j] = lv;
          }
        }
      }
    };

    // nref: every entry -(the reference max, 0 while m = -inf), the value the S
    // accumulators start from; kept across steps and changed only when m is raised.
    float m[kHeadsPerWave];
    float lsum[kHeadsPerWave];  // the row's sum of weights
    f32x4 nref[kHeadsPerWave];
    f32x4 o[kHeadsPerWave][4];
#pragma unroll
    for (int hh = 0; hh < kHeadsPerWave; ++hh) {
      m[hh] = -INFINITY;
      lsum[hh] = 0.0f;
      nref[hh] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < 4; ++mt) o[hh][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    // The block's key tiles in segments of kSegTiles, each with its page ids
    // staged in LDS. Within a segment, a ring of kRingSteps steps of kTeams tile
    // buffers: steps 0 .. kRingSteps-2 are issued up front; at step s, step
    // s + kRingSteps - 1 goes into the buffers step s - 1 used. A step past the
    // last tile still loads (page 0 or in-pool pages, never read), keeping every
    // step's load count the same for the counted waits. Segments hold an even
    // number of tiles, so a step never straddles two.
    // Staging of the segment starting at seg0: its page ids and step flags into
    // LDS, and the ring's first steps issued.
    int n_steps = 0;
    auto stage = [&]() {
      n_steps = (min(kSegTiles, n_tiles - seg0) + kTeams - 1) / kTeams;
      // The ring is idle here and every wave is past its last read of the previous
      // segment's ids (the last step, or the team exchange, ended in a barrier).
      for (int i = tid; i < 4 * kTeams * n_steps; i += 64 * kWaves * kTeams) {
        const int pi = 4 * seg0 + i;
        const int id = pi < max_pages ? tab[pi] : -1;
        ids[i] = id >= 0 && id < num_pages ? id : -1;
      }
      // The block's RoPE rows (first segment only; rows outside the table or past
      // the block's rows are not used and stay as they are).
      if (rope && seg0 == 0 && tid < kRows * 16) {
        const int ri = tid >> 4, p = pos0 + t0 + ri;
        if (t0 + ri < T && p >= 0 && p < rope_positions)
          reinterpret_cast<float4*>(rope_rows + ri * kRopeStride)[tid & 15] =
              reinterpret_cast<const float4*>(rope + size_t(p) * 64)[tid & 15];
      }
      __syncthreads();
      for (int i = tid; i < n_steps; i += 64 * kWaves * kTeams) {
        int f = 0;
#pragma unroll
        for (int tm = 0; tm < kTeams; ++tm) {
          const int tile = seg0 + kTeams * i + tm;
          const int4 v = tile_ids(tile);
          const int ok = int(v.x >= 0) | (int(v.y >= 0) << 1) | (int(v.z >= 0) << 2) |
                         (int(v.w >= 0) << 3);
          f |= ok << (4 * tm);
          if (tile < n_tiles && (tile * kKeys + kKeys - 1 > max_pos || ok != 15)) f |= 1 << 8;
        }
        step_flags[i] = f;
      }  // read after the barrier below
      for (int pre = 0; pre < kRingSteps - 1 && pre < n_steps; ++pre)
        issue(buffer(pre, team), seg0 + kTeams * pre + team);
    };
    seg0 = 0;
    stage();
    make_q();  // the query's loads landed with the staging's
    for (;;) {
      wait_steps(min(kRingSteps - 2, n_steps - 1));  // step 0 has landed
      __syncthreads();

      int rs = 0;               // ring slot of step s
      int is = kRingSteps - 1;  // ring slot of step s + kRingSteps - 1
      for (int st = 0; st < n_steps; ++st) {
        const int fl = __builtin_amdgcn_readfirstlane(step_flags[st]);  // read with the ids below
        const int ahead = st + kRingSteps - 1;
        if (ahead < n_steps)  // its buffers held step s - 1: free since the last barrier
          issue(buffer(is, team), seg0 + kTeams * ahead + team);
        is = is + 1 == kRingSteps ? 0 : is + 1;
        const int kb = seg0 + kTeams * st + team;  // this team's tile
        const int buf = buffer(rs, team);
        rs = rs + 1 == kRingSteps ? 0 : rs + 1;
        const int kbase = kb * kKeys;
        const unsigned char* kt = smem + buf * kBufBytes;
        unsigned char* vt = smem + buf * kBufBytes + kTileBytes;
        // Keys past max_pos (the last tile) or in pages outside the pool: zero
        // their V rows before the team reads the tile. The decision covers every
        // tile of the step, so every wave takes the same branch and barrier.
        const bool zero_step = (fl >> 8) & 1;
        const int okb = (fl >> (4 * team)) & 15;
        if (zero_step) {
          if (kb < n_tiles) {
            for (int i = tid - 64 * kWaves * team; i < kKeys * 8; i += 64 * kWaves) {
              const int key = i >> 3;
              if (kbase + key > max_pos || !((okb >> (key >> 4)) & 1))
                *reinterpret_cast<uint4*>(vt + key * 128 + (i & 7) * 16) = make_uint4(0, 0, 0, 0);
            }
          }
          __syncthreads();
        }

        if (kb < n_tiles) {  // uniform per team (the odd last step of team 1 skips)
          // S^T for the tile's 4 key groups of 16: A = K rows 16 kt4 + r, dims 32 ks + 8g.
          op ka[4][2];
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4) {
            const int row = 16 * kt4 + r;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks)
              ka[kt4][ks] = *reinterpret_cast<const op*>(kt + row * 128 +
                                                         16 * ((4 * ks + g) ^ ((row >> 1) & 7)));
          }
          // The accumulators start at -mref (the row's reference max, 0 before any
          // visible key), so the products come out as s - mref directly.
          f32x4 s[kHeadsPerWave][4];
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
            for (int hh = 0; hh < kHeadsPerWave; ++hh) {
              f32x4 acc = nref[hh];
#pragma unroll
              for (int ks = 0; ks < 2; ++ks) {
                acc = M::mma(ka[kt4][ks], qhi[hh][ks], acc);
                if constexpr (kSplit) acc = M::mma(ka[kt4][ks], qlo[hh][ks], acc);
              }
              s[hh][kt4] = acc;
            }
          // Causal mask (and masked pages) where the tile is not entirely visible.
          if (kbase + kKeys - 1 > min_pos || okb != 15) {
#pragma unroll
            for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int kp = kbase + 16 * kt4 + 4 * g + e;
                const bool vis = kp <= rp && ((okb >> kt4) & 1);
#pragma unroll
                for (int hh = 0; hh < kHeadsPerWave; ++hh)
                  s[hh][kt4][e] = vis ? s[hh][kt4][e] : -INFINITY;
              }
          }
          // Online softmax per head on s - mref; P^T operands per 32-key group kg:
          // slots 0-3 = keys 32kg + 4g + e (group 2kg), slots 4-7 = keys 32kg + 16 +
          // 4g + e. The reference max mref is raised lazily: weights are 2^(s - mref)
          // with mref the row's max when it was last raised, and O and l are rescaled
          // only when the reference has to move.
          //   Until every row of the wave has a reference (its first visible tile),
          //   each tile's max is taken and the reference raised when a row's max
          //   passes mref + kLazyMax (weights then <= 2^kLazyMax).
          //   After that (single-rounded f16 operands; split hi + lo operands take
          //   the max on every tile) a tile's weights are formed against the standing reference
          //   without a max, and the tile's row sums (from the matrix cores, from the
          //   same rounded operands as O) tell whether it may: while every row's sum
          //   is <= kSumMax, so is every weight -- in range for f16, whose largest
          //   value is 65504, and at a magnitude where rounding is relative, as it
          //   is at any normal magnitude. A larger sum (or an f16 weight rounded to
          //   inf) sends the tile through the max and the raise above, and its
          //   weights are formed again. The row sums l come from the matrix cores.
          op phi[kHeadsPerWave][2], plo[kHeadsPerWave][2];
#pragma unroll
          for (int hh = 0; hh < kHeadsPerWave; ++hh) {
            auto raise = [&]() {
              const f32x4(&sh)[4] = s[hh];
              float mx = max_nn(max3_nn(max3_nn(sh[0][0], sh[0][1], sh[0][2]),
                                        max3_nn(sh[0][3], sh[1][0], sh[1][1]),
                                        max3_nn(sh[1][2], sh[1][3], sh[2][0])),
                                max3_nn(max3_nn(sh[2][1], sh[2][2], sh[2][3]),
                                        max3_nn(sh[3][0], sh[3][1], sh[3][2]), sh[3][3]));
              mx = group_max4(mx);  // the tile's row max, relative to mref
              // m = -inf (nothing visible yet) always counts as growth when mx is finite.
              const bool grow = mx > (m[hh] == -INFINITY ? -INFINITY : kLazyMax);
              if (__builtin_amdgcn_ballot_w64(grow) != 0) {
                const float mref = -nref[hh][0];
                const float m_new = fmaxf(m[hh], mref + mx);
                // m = -inf (nothing seen yet): the old terms are all zero
                const float corr = m_new == -INFINITY ? 1.0f : exp2_weight(m[hh] - m_new);
                lsum[hh] *= corr;
#pragma unroll
                for (int mt = 0; mt < 4; ++mt) o[hh][mt] *= corr;
                m[hh] = m_new;
                // Re-reference this tile's scores to the new max.
                const float ref = m_new == -INFINITY ? 0.0f : m_new;
                const float shift = ref - mref;
#pragma unroll
                for (int kt4 = 0; kt4 < 4; ++kt4) s[hh][kt4] -= shift;
                nref[hh] = f32x4{-ref, -ref, -ref, -ref};
              }
            };
            auto weights = [&]() {
#pragma unroll
              for (int kg = 0; kg < 2; ++kg)
#pragma unroll
                for (int e = 0; e < 4; e += 2) {
                  const float pa0 = exp2_weight(s[hh][2 * kg][e]);
                  const float pa1 = exp2_weight(s[hh][2 * kg][e + 1]);
                  const float pb0 = exp2_weight(s[hh][2 * kg + 1][e]);
                  const float pb1 = exp2_weight(s[hh][2 * kg + 1][e + 1]);
                  E h0, h1, l0, l1;
                  if constexpr (kSplit) {
                    split16x2(pa0, pa1, h0, h1, l0, l1);
                    plo[hh][kg][e] = l0;
                    plo[hh][kg][e + 1] = l1;
                  } else {
                    round16x2(pa0, pa1, h0, h1);
                  }
                  phi[hh][kg][e] = h0;
                  phi[hh][kg][e + 1] = h1;
                  if constexpr (kSplit) {
                    split16x2(pb0, pb1, h0, h1, l0, l1);
                    plo[hh][kg][4 + e] = l0;
                    plo[hh][kg][5 + e] = l1;
                  } else {
                    round16x2(pb0, pb1, h0, h1);
                  }
                  phi[hh][kg][4 + e] = h0;
                  phi[hh][kg][5 + e] = h1;
                }
            };
            // The tile's row sums: an all-ones A operand against P^T puts sum_k P[r][k]
            // of the tile's keys in every entry of lane r's accumulator.
            auto row_sum = [&]() {
              f32x4 tl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kg = 0; kg < 2; ++kg) {
                tl = M::mma(ones, phi[hh][kg], tl);
                if constexpr (kSplit) tl = M::mma(ones, plo[hh][kg], tl);
              }
              return tl[0];
            };
            if constexpr (kSplit) {
              // hi + lo operands: twice the weight registers, no room for a second
              // formation; every tile takes the max.
              raise();
              weights();
              lsum[hh] += row_sum();
            } else {
              const bool fresh = __builtin_amdgcn_ballot_w64(m[hh] == -INFINITY) != 0;
              if (fresh) raise();
              weights();
              float tl = row_sum();
              if (!fresh && __builtin_amdgcn_ballot_w64(!(tl <= kSumMax)) != 0) {
                raise();
                weights();
                tl = row_sum();
              }
              lsum[hh] += tl;
            }
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
#pragma unroll
              for (int hh = 0; hh < kHeadsPerWave; ++hh) {
                o[hh][mt] = M::mma(a, phi[hh][kg], o[hh][mt]);
                if constexpr (kSplit) o[hh][mt] = M::mma(a, plo[hh][kg], o[hh][mt]);
              }
            }
          }
        }
        // This wave's loads of step s + 1 have landed (later steps may still be in
        // flight); after the barrier every wave's have, and every wave is done
        // with step s's buffers.
        wait_steps(max(0, min(kRingSteps - 2, n_steps - st - 2)));
        __syncthreads();
      }
      seg0 += kSegTiles;
      if (seg0 >= n_tiles) break;
      stage();
    }

    // Teams 1.. hand their (m, l, O) to team 0 through LDS (the ring is idle:
    // every load has landed and every tile was consumed before the last barrier).
    // Lane L of a head's waves holds the same rows and dims in every team.
    float* xo = reinterpret_cast<float*>(smem);                       // [kWaves][4][64] f32x4
    float* xml = reinterpret_cast<float*>(smem + kWaves * 4096);      // [kWaves][64] float2
    if constexpr (kTeams > 1) {
#pragma unroll
      for (int tm = 1; tm < kTeams; ++tm) {
        if (team == tm) {
#pragma unroll
          for (int mt = 0; mt < 4; ++mt)
            *reinterpret_cast<f32x4*>(xo + ((wave * 4 + mt) * 64 + lane) * 4) = o[0][mt];
          *reinterpret_cast<float2*>(xml + (wave * 64 + lane) * 2) = make_float2(m[0], lsum[0]);
        }
        __syncthreads();
        if (team == 0) {
          const float2 ml = *reinterpret_cast<const float2*>(xml + (wave * 64 + lane) * 2);
          const float m_new = fmaxf(m[0], ml.x);
          const float c0 = m[0] == -INFINITY ? 0.0f : exp2_weight(m[0] - m_new);
          const float c1 = ml.x == -INFINITY ? 0.0f : exp2_weight(ml.x - m_new);
          lsum[0] = lsum[0] * c0 + ml.y * c1;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) {
            const f32x4 o1 = *reinterpret_cast<const f32x4*>(xo + ((wave * 4 + mt) * 64 + lane) * 4);
            o[0][mt] = o[0][mt] * c0 + o1 * c1;
          }
          m[0] = m_new;
        }
        __syncthreads();  // the exchange area is free again (next team or next pass)
      }
    }

    if (team == 0 && row_ok) {
#pragma unroll
      for (int hh = 0; hh < kHeadsPerWave; ++hh) {
        if (hh >= nh) break;
        const float il = 1.0f / lsum[hh];
        float* dst = out + (size_t(t) * n_heads + h0 + hh) * 64 + 4 * g;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) *reinterpret_cast<f32x4*>(dst + 16 * mt) = o[hh][mt] * il;
      }
    }
  }
}

// LDS of the kernel: the ring of steps (which also holds the team exchange
// area), then the page ids of one segment of key tiles.
template <int kTeams>
constexpr int prefill_lds_bytes() {
  return (kTeams == 1 ? 4 : 3) * kTeams * kBufBytes + 16 * (kSegTiles + kTeams) +
         4 * kSegTiles + kRows * kRopeStride * 4;
}

template <int KV, int W, int kTeams, bool kSplitF16>
int launch_prefill_split(const dim3 grid, float* out, const float* q, const uint16_t* kp,
                         const uint16_t* vp, int T, const int32_t* row_pos,
                         const int32_t* row_seq, const ie_kv_layout& kv, int n_heads,
                         int n_kv_heads, int n_blocks, const PrefillRope& rope,
                         hipStream_t stream) {
  constexpr int lds = prefill_lds_bytes<kTeams>();
  static_assert(lds - 16 * (kSegTiles + kTeams) - 4 * kSegTiles - kRows * kRopeStride * 4 >=
                    W * 4096 + W * 512,
                "team exchange area must fit in the ring");
  if (lds > 65536) {  // above the default dynamic-LDS cap, within gfx950's 160 KB
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(prefill_mfma_kernel<KV, W, kTeams, kSplitF16>),
        hipFuncAttributeMaxDynamicSharedMemorySize, lds);
    if (int rc = check_hip(attr, "hipFuncSetAttribute(attention_prefill_mfma)")) return rc;
  }
  hipLaunchKernelGGL((prefill_mfma_kernel<KV, W, kTeams, kSplitF16>), grid,
                     dim3(64 * W * kTeams), lds, stream, out, q, kp, vp, T, row_pos, row_seq,
                     kv.tables, kv.max_pages, kv.num_pages, n_heads, n_kv_heads, n_blocks,
                     rope.table, rope.positions);
  return check_launch("attention_prefill_mfma");
}

// f16 caches take q and P as single f16 values unless the process asked for the
// split operands (ie_hip_set_prefill_rounding); bf16 caches always split.
template <int KV, int W, int kTeams>
int launch_prefill_variant(const dim3 grid, float* out, const float* q, const uint16_t* kp,
                           const uint16_t* vp, int T, const int32_t* row_pos,
                           const int32_t* row_seq, const ie_kv_layout& kv, int n_heads,
                           int n_kv_heads, int n_blocks, const PrefillRope& rope,
                           hipStream_t stream) {
  if (KV == IE_KV_F16 && prefill_rounding() == IE_HIP_PREFILL_SPLIT)
    return launch_prefill_split<KV, W, kTeams, true>(grid, out, q, kp, vp, T, row_pos, row_seq,
                                                     kv, n_heads, n_kv_heads, n_blocks, rope,
                                                     stream);
  return launch_prefill_split<KV, W, kTeams, false>(grid, out, q, kp, vp, T, row_pos, row_seq,
                                                    kv, n_heads, n_kv_heads, n_blocks, rope,
                                                    stream);
}

template <int KV>
int launch_prefill_mfma(float* out, const float* q, const uint16_t* kp, const uint16_t* vp, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, const PrefillRope& rope, hipStream_t stream) {
  const int group = n_heads / n_kv_heads;
  const int waves = (group + kHeadsPerWave - 1) / kHeadsPerWave;
  const int n_blocks = (T + kRows - 1) / kRows;
  const dim3 grid((n_blocks + 1) / 2, n_kv_heads);
  // Two teams splitting the key tiles when the grid alone leaves compute units
  // without a workgroup or with one: twice the waves per CU, half the serial
  // tile chain per wave. Larger grids already hold two workgroups per CU.
  const bool teams2 = int64_t(grid.x) * grid.y <= device_compute_units();
#define IE_PF_CASE(W)                                                                             \
  case W:                                                                                         \
    return teams2 ? launch_prefill_variant<KV, W, 2>(grid, out, q, kp, vp, T, row_pos, row_seq,   \
                                                      kv, n_heads, n_kv_heads, n_blocks, rope,    \
                                                      stream)                                     \
                  : launch_prefill_variant<KV, W, 1>(grid, out, q, kp, vp, T, row_pos, row_seq,   \
                                                      kv, n_heads, n_kv_heads, n_blocks, rope,    \
                                                      stream);
  switch (waves) {
    IE_PF_CASE(1)
    IE_PF_CASE(2)
    IE_PF_CASE(3)
    IE_PF_CASE(4)
    IE_PF_CASE(5)
    IE_PF_CASE(6)
    IE_PF_CASE(7)
    IE_PF_CASE(8)
    default:
      return fail(IE_HIP_EINVAL, "attention_prefill: at most 8 query heads per KV head");
  }
#undef IE_PF_CASE
}


// ---------------------------------------------------------------------------
// float32 KV caches: the same block structure on v_mfma_f32_16x16x4_f32 (full
// fp32 operands: no hi + lo split, 16x the matrix-core time per product of the
// 16-bit kernel, still far above the VALU path).
//   S^T[16 keys x 16 rows] per key group of 16: 16 steps of 4 dims; step s
//     takes dims 16g + s for lane group g, so lane (g, r) reads key r's dims
//     16g .. 16g+15 (64 bytes, 4 LDS reads) and holds, as B, row r's query at
//     the same dims.
//   O^T[64 dims x 16 rows] += V^T . P^T: 16 steps of 4 keys; step (kt4, s)
//     takes keys 16 kt4 + 4g + s, so lane (g, r)'s B operand is its own score
//     of that key; row i of tile mt is dim 4i + mt, so its A operand is the
//     16-byte piece r of that key's V row (one LDS read, the 4 tiles' values).
//     Lane (g, r) ends up holding row r's dims 16g + 4t + mt (o[mt][t]).
// K/V tiles of 64 keys (16 KB each, f32) go through a ring of 3 tiles in LDS
// by DMA. K rows are stored with their 16-byte pieces swizzled (piece ^ (key
// & 15)), so the 16 lanes of a group reading the same dims of 16 keys hit
// distinct banks; V rows are read a whole row per 16 lanes and stay as they are.
constexpr int kTileF32 = kKeys * 64 * 4;     // 16 KB: one f32 K or V tile of one KV head
constexpr int kBufF32 = 2 * kTileF32;        // K tile + V tile
constexpr int kRingF32 = 3;

template <int kWaves>
__global__ void __launch_bounds__(64 * kWaves)
prefill_mfma_f32_kernel(float* __restrict__ out, const float* __restrict__ q,
                        const float* __restrict__ k_pool, const float* __restrict__ v_pool, int T,
                        const int32_t* __restrict__ row_pos, const int32_t* __restrict__ row_seq,
                        const int32_t* __restrict__ tables, int max_pages, int num_pages,
                        int n_heads, int n_kv_heads, int n_blocks) {
  // A tile's 32 loads of 1 KB (16 K, 16 V), spread evenly over kDmaWaves waves.
  constexpr int kDmaWaves = kWaves >= 4 ? 4 : kWaves >= 2 ? 2 : 1;
  constexpr int kPerWave = 32 / kDmaWaves;
  extern __shared__ __align__(16) unsigned char smem[];
  const int group = n_heads / n_kv_heads;
  const int kvh = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int h0 = kvh * group + wave;  // this wave's head
  const int kv_dim = n_kv_heads * 64;
  const int pos0 = __builtin_amdgcn_readfirstlane(row_pos[0]);
  const int seq = __builtin_amdgcn_readfirstlane(row_seq[0]);
  const int32_t* tab = tables + size_t(seq) * max_pages;
  // Page ids of a segment of key tiles staged in LDS after the ring, as in the
  // 16-bit kernel: ids[4 (tile - seg0) + j], -1 past the table row or outside
  // the pool.
  int* const ids = reinterpret_cast<int*>(smem + kRingF32 * kBufF32);
  int seg0 = 0;
  auto tile_ids = [&](const int tile) {
    return *reinterpret_cast<const int4*>(ids + 4 * (tile - seg0));
  };
  auto tile_ok = [&](const int tile) -> int {
    const int4 v = tile_ids(tile);
    return __builtin_amdgcn_readfirstlane(int(v.x >= 0) | (int(v.y >= 0) << 1) |
                                          (int(v.z >= 0) << 2) | (int(v.w >= 0) << 3));
  };

  // DMA of a tile into buffer `buf`: load u (0..15 K, 16..31 V) moves keys
  // 4 (u & 15) .. +3 (page (u & 15) / 4 of the tile); lane l lands at base + 16 l:
  // key 4 (u & 15) + l / 16, LDS slot l % 16, holding global piece slot ^ (key & 15)
  // for K and piece slot for V.
  const size_t row_bytes = size_t(kv_dim) * 4;
  const int lkey = lane >> 4, lslot = lane & 15;
  const unsigned smem_lds = lds_address(smem);
  const char* kbase_g = reinterpret_cast<const char*>(k_pool) + kvh * 256;
  const char* vbase_g = reinterpret_cast<const char*>(v_pool) + kvh * 256;
  auto issue = [&](const int buf, const int tile) {
    if (wave >= kDmaWaves) return;
    const int4 v = tile_ids(tile);
    const int id0 = max(__builtin_amdgcn_readfirstlane(v.x), 0);
    const int id1 = max(__builtin_amdgcn_readfirstlane(v.y), 0);
    const int id2 = max(__builtin_amdgcn_readfirstlane(v.z), 0);
    const int id3 = max(__builtin_amdgcn_readfirstlane(v.w), 0);
#pragma unroll
    for (int k = 0; k < kPerWave; ++k) {
      const int u = wave * kPerWave + k;        // 0..31
      const bool is_v = u >= 16;
      const int uu = u & 15;
      const int pg = uu >> 2;                   // page of the tile
      const int id = pg == 0 ? id0 : pg == 1 ? id1 : pg == 2 ? id2 : id3;
      const int key = 4 * uu + lkey;            // key within the tile
      const int piece = is_v ? lslot : (lslot ^ (key & 15));
      const char* src = (is_v ? vbase_g : kbase_g) +
                        (size_t(id) * IE_HIP_PAGE_SIZE + (key & 15)) * row_bytes +
                        16 * piece;
      dma16(src, smem_lds + buf * kBufF32 + (is_v ? kTileF32 : 0) + uu * 1024);
    }
  };
  auto wait_tiles = [&](const int newer) {
    if (newer >= 1) wait_vmcnt<kPerWave>();
    else wait_vmcnt<0>();
  };

  for (int pass = 0; pass < 2; ++pass) {
    const int hi_block = n_blocks - 1 - int(blockIdx.x);
    const int rb = pass == 0 ? hi_block : int(blockIdx.x);
    if (pass == 1 && rb == hi_block) break;  // the middle block of an odd count
    const int t0 = rb * kRows;
    const int t_last = min(t0 + kRows, T) - 1;
    const int max_pos = pos0 + t_last;
    const int min_pos = pos0 + t0;
    const int n_tiles = max_pos / kKeys + 1;
    const int t = t0 + r;
    const bool row_ok = t < T;
    const int rp = pos0 + t;

    // Row r's query, times log2(e)/8, at dims 16g .. 16g+15 (B of the score steps).
    float qb[16];
    {
      const float4* src = reinterpret_cast<const float4*>(
          q + (size_t(row_ok ? t : t0) * n_heads + h0) * 64 + 16 * g);
      const float qs = row_ok ? 0.125f * kLog2e : 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float4 x = src[i];
        qb[4 * i + 0] = x.x * qs;
        qb[4 * i + 1] = x.y * qs;
        qb[4 * i + 2] = x.z * qs;
        qb[4 * i + 3] = x.w * qs;
      }
    }
    float m = -INFINITY, l = 0.0f;  // running max (base 2), this lane's part of the sum
    f32x4 o[4];                      // o[mt][t]: row r, dim 16g + 4t + mt
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) o[mt] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Segments of kSegTiles key tiles, each with its page ids staged in LDS;
    // within a segment, a ring of kRingF32 tiles.
    for (seg0 = 0; seg0 < n_tiles; seg0 += kSegTiles) {
      const int seg_end = min(n_tiles, seg0 + kSegTiles);
      // The ring is idle and every wave is past its last read of the old ids.
      for (int i = tid; i < 4 * (seg_end - seg0); i += 64 * kWaves) {
        const int pi = 4 * seg0 + i;
        const int id = pi < max_pages ? tab[pi] : -1;
        ids[i] = id >= 0 && id < num_pages ? id : -1;
      }
      __syncthreads();
      for (int pre = 0; pre < kRingF32 - 1 && seg0 + pre < seg_end; ++pre) issue(pre, seg0 + pre);
      wait_tiles(min(kRingF32 - 2, seg_end - seg0 - 1));  // the segment's first tile has landed
      __syncthreads();

      int buf = 0, ibuf = kRingF32 - 1;
      for (int kb = seg0; kb < seg_end; ++kb) {
        const int ahead = kb + kRingF32 - 1;
        if (ahead < seg_end)  // its buffer held tile kb - 1: free since the last barrier
          issue(ibuf, ahead);
        ibuf = ibuf + 1 == kRingF32 ? 0 : ibuf + 1;
        const int kbase = kb * kKeys;
        const unsigned char* kt = smem + buf * kBufF32;
        unsigned char* vt = smem + buf * kBufF32 + kTileF32;
        buf = buf + 1 == kRingF32 ? 0 : buf + 1;
        const int okb = tile_ok(kb);
        // Keys past max_pos or in pages outside the pool: zero their V rows first.
        if (kbase + kKeys - 1 > max_pos || okb != 15) {
          for (int i = tid; i < kKeys * 16; i += 64 * kWaves) {
            const int key = i >> 4;
            if (kbase + key > max_pos || !((okb >> (key >> 4)) & 1))
              *reinterpret_cast<uint4*>(vt + key * 256 + (i & 15) * 16) = make_uint4(0, 0, 0, 0);
          }
          __syncthreads();
        }
        const float mref = m == -INFINITY ? 0.0f : m;
        // S^T per key group kt4: A = key 16 kt4 + r, dims 16g + s.
        f32x4 s[4];
#pragma unroll
        for (int kt4 = 0; kt4 < 4; ++kt4) {
          const int key = 16 * kt4 + r;
          float ka[16];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float4 x = *reinterpret_cast<const float4*>(kt + key * 256 +
                                                              16 * ((4 * g + i) ^ (key & 15)));
            ka[4 * i + 0] = x.x;
            ka[4 * i + 1] = x.y;
            ka[4 * i + 2] = x.z;
            ka[4 * i + 3] = x.w;
          }
          f32x4 acc = {-mref, -mref, -mref, -mref};
#pragma unroll
          for (int st = 0; st < 16; ++st)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[st], qb[st], acc, 0, 0, 0);
          s[kt4] = acc;
        }
        if (kbase + kKeys - 1 > min_pos || okb != 15) {
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int kp = kbase + 16 * kt4 + 4 * g + e;
              s[kt4][e] = (kp <= rp && ((okb >> kt4) & 1)) ? s[kt4][e] : -INFINITY;
            }
        }
        // Online softmax on s - mref, the reference max raised lazily (as in the
        // 16-bit kernel: O and l rescaled only when a row's max grows past
        // m + kLazyMax somewhere in the wave).
        float mx = -INFINITY;
#pragma unroll
        for (int kt4 = 0; kt4 < 4; ++kt4)
          mx = fmaxf(mx, fmaxf(fmaxf(s[kt4][0], s[kt4][1]), fmaxf(s[kt4][2], s[kt4][3])));
        mx = group_max4(mx);
        const bool grow = m == -INFINITY ? mx != -INFINITY : mx > kLazyMax;
        if (__builtin_amdgcn_ballot_w64(grow) != 0) {
          const float m_new = fmaxf(m, mref + mx);
          const float corr = m_new == -INFINITY ? 1.0f : exp2_weight(m - m_new);  // m = -inf: 0
          l *= corr;
#pragma unroll
          for (int mt = 0; mt < 4; ++mt) o[mt] *= corr;
          m = m_new;
          const float shift = (m_new == -INFINITY ? 0.0f : m_new) - mref;
#pragma unroll
          for (int kt4 = 0; kt4 < 4; ++kt4) s[kt4] -= shift;
        }
        float sum = 0.0f;
#pragma unroll
        for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            s[kt4][e] = exp2_weight(s[kt4][e]);
            sum += s[kt4][e];
          }
        l += sum;
        // O^T += V^T P^T: step (kt4, e) takes key 16 kt4 + 4g + e; lane (g, r)
        // reads that key's V piece r (dims 4r .. 4r+3, the 4 tiles' A values).
#pragma unroll
        for (int kt4 = 0; kt4 < 4; ++kt4)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float4 v =
                *reinterpret_cast<const float4*>(vt + (16 * kt4 + 4 * g + e) * 256 + 16 * r);
            const float pw = s[kt4][e];
            o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(v.x, pw, o[0], 0, 0, 0);
            o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(v.y, pw, o[1], 0, 0, 0);
            o[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(v.z, pw, o[2], 0, 0, 0);
            o[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(v.w, pw, o[3], 0, 0, 0);
          }
        wait_tiles(max(0, min(kRingF32 - 2, seg_end - kb - 2)));
        __syncthreads();
      }
    }

    l = group_sum4(l);
    if (row_ok) {
      const float il = 1.0f / l;
      float* dst = out + (size_t(t) * n_heads + h0) * 64 + 16 * g;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const f32x4 v = {o[0][e], o[1][e], o[2][e], o[3][e]};
        *reinterpret_cast<f32x4*>(dst + 4 * e) = v * il;
      }
    }
  }
}

template <int W>
int launch_prefill_f32(const dim3 grid, float* out, const float* q, const float* kp,
                       const float* vp, int T, const int32_t* row_pos, const int32_t* row_seq,
                       const ie_kv_layout& kv, int n_heads, int n_kv_heads, int n_blocks,
                       hipStream_t stream) {
  constexpr int lds = kRingF32 * kBufF32 + 16 * kSegTiles;  // 96 KB ring + the segment's page ids
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(prefill_mfma_f32_kernel<W>),
      hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  if (int rc = check_hip(attr, "hipFuncSetAttribute(attention_prefill_mfma_f32)")) return rc;
  hipLaunchKernelGGL((prefill_mfma_f32_kernel<W>), grid, dim3(64 * W), lds, stream, out, q, kp,
                     vp, T, row_pos, row_seq, kv.tables, kv.max_pages, kv.num_pages, n_heads,
                     n_kv_heads, n_blocks);
  return check_launch("attention_prefill_mfma_f32");
}

}  // namespace

bool prefill_mfma_supported(int kv_dtype, int n_heads, int n_kv_heads, int head_dim) {
  return (kv_dtype == IE_KV_F16 || kv_dtype == IE_KV_BF16 || kv_dtype == IE_KV_F32) &&
         head_dim == 64 && n_kv_heads > 0 && n_heads % n_kv_heads == 0 &&
         n_heads / n_kv_heads <= kMaxGroup;
}

int prefill_mfma_launch(float* out, const float* q, const void* k_pool, const void* v_pool, int T,
                        const int32_t* row_pos, const int32_t* row_seq, const ie_kv_layout& kv,
                        int n_heads, int n_kv_heads, const PrefillRope& rope,
                        hipStream_t stream) {
  if (rope.table && (reinterpret_cast<uintptr_t>(rope.table) & 15))
    return fail(IE_HIP_EINVAL, "attention_prefill: the RoPE table must be 16-byte aligned");
  if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) |
       reinterpret_cast<uintptr_t>(k_pool) | reinterpret_cast<uintptr_t>(v_pool)) & 15)
    return fail(IE_HIP_EINVAL, "attention_prefill: q, out and the pools must be 16-byte aligned");
  if (kv.kv_dtype == IE_KV_F32) {
    // The f32 kernel takes q already rotated (its lanes hold 16 consecutive dims,
    // not the rotation pairs; reading the partner dims and the table per lane
    // cost more than the append's q traffic saves).
    if (rope.table)
      return fail(IE_HIP_EINVAL, "attention_prefill: f32 caches take q rotated by rope_and_cache");
    const int group = n_heads / n_kv_heads;
    const int n_blocks = (T + kRows - 1) / kRows;
    const dim3 grid((n_blocks + 1) / 2, n_kv_heads);
    const float* kf = static_cast<const float*>(k_pool);
    const float* vf = static_cast<const float*>(v_pool);
    switch (group) {
#define IE_PF32_CASE(W)                                                                      \
  case W:                                                                                    \
    return launch_prefill_f32<W>(grid, out, q, kf, vf, T, row_pos, row_seq, kv, n_heads,     \
                                 n_kv_heads, n_blocks, stream);
      IE_PF32_CASE(1)
      IE_PF32_CASE(2)
      IE_PF32_CASE(3)
      IE_PF32_CASE(4)
      IE_PF32_CASE(5)
      IE_PF32_CASE(6)
      IE_PF32_CASE(7)
      IE_PF32_CASE(8)
#undef IE_PF32_CASE
    }
    return fail(IE_HIP_EINVAL, "attention_prefill: at most 8 query heads per KV head");
  }
  const uint16_t* kp = static_cast<const uint16_t*>(k_pool);
  const uint16_t* vp = static_cast<const uint16_t*>(v_pool);
  if (kv.kv_dtype == IE_KV_F16)
    return launch_prefill_mfma<IE_KV_F16>(out, q, kp, vp, T, row_pos, row_seq, kv, n_heads,
                                          n_kv_heads, rope, stream);
  return launch_prefill_mfma<IE_KV_BF16>(out, q, kp, vp, T, row_pos, row_seq, kv, n_heads,
                                         n_kv_heads, rope, stream);
}

}  // namespace iehip
