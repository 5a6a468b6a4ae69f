// The dense ops of the decode step around the paged-KV path (gfx950): the
// embedding lookup, rmsnorm, the projections (q/k/v, o_proj, down) and the
// fused gate/up + SiLU. Reference: src/cuda/kernels.cuh:40-66 and
// src/cuda/kernels.cu:191-241,1236-1285; CPU semantics src/ops.cpp:23-32,68,
// src/matrix.cpp:131-146,247-289, src/model.cpp:53-90.
//
// Weights are BF16 bits or INT8 with one f32 scale per row (the reference's
// DeviceMatrix). Activations are f32.
//
// matmul_mfma_kernel: y[t][o] (+)= (sum_k W[o][k] x[t][k]) * s[o] + bias[o] on
// v_mfma_f32_16x16x32_bf16, in 16-row x 16-token output tiles:
//   D[16 rows x 16 tokens] = W[16 x K] . x^T[K x 16]
// The weights enter the MFMA exactly (BF16 as stored; INT8 values widened to
// bf16, exact for |q| <= 127). Each activation is split into three bf16
// parts, x = hi + mid + lo exactly (each remainder is exact in f32 and holds
// at most 16, then 8, significant bits), and each block is multiplied three
// times, so every product is the f32-exact w * x. Only the summation order
// differs from the CPU's: the results agree to float32 rounding of the sum.
// The 8 waves of a workgroup take interleaved 32-wide K blocks and their
// partial tiles are added through LDS in a fixed order, so results do not
// depend on scheduling. Larger launches take several tiles per workgroup
// (see launch_matmul).
// Lane (g, r) of a tile: A = W[row r][k + 8g .. +8], B = x[token r][k + 8g ..
// +8]; the result lane holds rows 4g .. 4g+3 of token r.
#include <algorithm>

#include "common.hpp"
#include "mfma.hpp"

namespace iehip {
namespace {

constexpr int kMmWaves = 8;  // waves of a workgroup, splitting K

using bf16 = __bf16;

template <bool I8>
__device__ __forceinline__ bf16x8 load_weights(const void* w, size_t idx) {
  bf16x8 a;
  if constexpr (!I8) {
    a = *reinterpret_cast<const bf16x8*>(static_cast<const uint16_t*>(w) + idx);
  } else {
    const uint2 raw = *reinterpret_cast<const uint2*>(static_cast<const int8_t*>(w) + idx);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t word = j < 4 ? raw.x : raw.y;
      const int8_t q = static_cast<int8_t>((word >> (8 * (j & 3))) & 0xFF);
      a[j] = static_cast<bf16>(static_cast<float>(q));
    }
  }
  return a;
}

// 8 activations as three bf16 operands whose sum is exact.
__device__ __forceinline__ void split3(const float4 p, const float4 q, bf16x8& hi, bf16x8& mid,
                                       bf16x8& lo) {
  const float v[8] = {p.x, p.y, p.z, p.w, q.x, q.y, q.z, q.w};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const bf16 h = static_cast<bf16>(v[j]);
    const float r1 = v[j] - static_cast<float>(h);
    const bf16 m = static_cast<bf16>(r1);
    const float r2 = r1 - static_cast<float>(m);
    hi[j] = h;
    mid[j] = m;
    lo[j] = static_cast<bf16>(r2);
  }
}

__device__ __forceinline__ f32x4 mma3(bf16x8 a, bf16x8 bh, bf16x8 bm, bf16x8 bl, f32x4 c) {
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, c, 0, 0, 0);
  c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bm, c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, c, 0, 0, 0);
}

__device__ __forceinline__ float silu(float v) { return v / (1.0f + expf(-v)); }

// GATE: out = silu(x . Wg^T * sg) * (x . Wu^T * su) (gate_up_silu); otherwise
// y (+)= x . W^T * s + bias. A workgroup owns RT x TT tiles of 16 rows x 16
// tokens: each weight fragment is loaded once per K block and used for all TT
// token tiles (so the weights are read once per launch when T <= 16 TT), each
// activation fragment split once and used for all RT row tiles. cols % 8 == 0;
// the K tail past cols is zero.
// Outputs: rows [0, split0) go to y ([T, split0]), rows [split0, split1) to y1
// ([T, split1 - split0]) and the rest to y2 ([T, rows - split1]); a plain
// matmul has split0 = split1 = rows.
struct RowSplit {
  float* y1;
  float* y2;
  int split0, split1;
};

// NORM: the rmsnorm before the matmul, folded into it (the decode step's
// xn = rmsnorm(x); y = xn . W^T pairs). y = (x * w_norm) . W^T * inv_rms(x):
// the activations are scaled by the norm weight as they are split, each lane
// sums the squares of the raw x it loads, the waves add those sums through LDS
// in the same fixed tree as their tiles, and the epilogue takes the row's
// 1 / sqrt(mean(x^2) + eps). The orders depend on the matrix shape alone.
struct RowNorm {
  const float* weight;  // [cols]
  float eps;
};

// STAGED (the 8-wave, one-token-tile launches; cols % 32 == 0): the K blocks'
// weight and activation tiles reach each wave's own LDS stages by DMA
// (global_load_lds_dwordx4) in whole 64-byte row pieces, one block ahead, and
// the MFMA operands are read back from there. A lane's direct loads of its
// operands (row r, columns 8g..8g+7) put 16 rows into each quarter-wave, one
// L1 access per lane; the L1 access rate then bounded these launches (probe,
// down 896 x 4,864 at 64 tokens: 15.3 us direct, 8.5 us staged). The MFMA
// operands and their order are the same, so the results are the same bits.
template <bool GATE, int RT, int TT, int W, bool I8, bool NORM = false, bool STAGED = false>
__global__ void __launch_bounds__(64 * W)
matmul_mfma_kernel(float* __restrict__ y, const float* __restrict__ x, const void* __restrict__ w,
                   const float* __restrict__ scale, const void* __restrict__ w2,
                   const float* __restrict__ scale2, const float* __restrict__ bias,
                   int T, int rows, int cols, int accumulate, RowSplit out, RowNorm norm) {
  constexpr int NA = GATE ? 2 : 1, NT = NA * RT * TT;
  static_assert(NT <= 16, "at most 16 accumulator tiles (64 KB of LDS for the reduction)");
  __shared__ f32x4 red[W / 2][NT][64];
  __shared__ float red_ss[NORM ? W / 2 : 1][TT][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int row0 = blockIdx.x * 16 * RT, tok0 = blockIdx.y * 16 * TT;
  size_t wrow[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) wrow[i] = size_t(min(row0 + 16 * i + r, rows - 1)) * cols;
  const float* xrow[TT];
#pragma unroll
  for (int j = 0; j < TT; ++j) xrow[j] = x + size_t(min(tok0 + 16 * j + r, T - 1)) * cols;
  f32x4 acc[NA][RT][TT];
#pragma unroll
  for (int n = 0; n < NA; ++n)
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int j = 0; j < TT; ++j) acc[n][i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float ss[TT];  // NORM: this lane's sum of x^2 of its token (row r of token tile j)
#pragma unroll
  for (int j = 0; j < TT; ++j) ss[j] = 0.0f;
  if constexpr (STAGED) {
    static_assert(TT == 1 && W == 8, "staged: 8-wave, one-token-tile launches");
    constexpr int kWTile = I8 ? 512 : 1024;               // 16 rows x 32 columns
    constexpr int kStage = NA * RT * kWTile + 2048;        // + 16 tokens x 32 floats
    constexpr int kPerStage = NA * RT + 2;                 // DMA instructions per stage
    extern __shared__ __align__(16) unsigned char dyn[];
    // [0, nbytes): the norm weight (NORM); then each wave's two stages.
    const int nbytes = NORM ? cols * 4 : 0;
    unsigned char* const stages = dyn + nbytes + wave * 2 * kStage;
    const unsigned stages_lds = lds_address(stages);
    // DMA sources. Weight tile: bf16, lane l takes row l/4, 16-byte piece
    // (l%4) ^ (row/2 % 4); int8, lanes 0-31, row l/2, piece (l%2) ^ (row/4 % 2).
    // Activation tile: lane l of DMA u takes token 8u + l/8, piece (l%8) ^ (l/8).
    // LDS slot = lane, so each row's pieces land swizzled and the operand reads
    // below spread over the banks.
    const int wr = I8 ? (lane >> 1) : (lane >> 2);
    const int wp = I8 ? ((lane & 1) ^ ((wr >> 2) & 1)) : ((lane & 3) ^ ((wr >> 1) & 3));
    const char* wsrc[NA][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      const size_t off = (size_t(min(row0 + 16 * i + (wr & 15), rows - 1)) * cols + 8 * (I8 ? 2 : 1) * wp) *
                         (I8 ? 1 : 2);
      wsrc[0][i] = static_cast<const char*>(w) + off;
      if constexpr (GATE) wsrc[NA - 1][i] = static_cast<const char*>(w2) + off;
    }
    const int xq = (lane & 7) ^ ((lane >> 3) & 7);
    const float* xsrc0 = x + size_t(min(tok0 + (lane >> 3), T - 1)) * cols + 4 * xq;
    const float* xsrc1 = x + size_t(min(tok0 + 8 + (lane >> 3), T - 1)) * cols + 4 * xq;
    const int nblk = cols > 32 * wave ? (cols - 32 * wave + 32 * W - 1) / (32 * W) : 0;
    auto issue = [&](const int slot, const int j) {
      const int kb = min(32 * (wave + W * j), cols - 32);  // j < nblk: always in bounds
      const unsigned dst = stages_lds + slot * kStage;
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          const char* src = wsrc[n][i] + size_t(kb) * (I8 ? 1 : 2);
          if constexpr (I8) {
            if (lane < 32) dma16(src, dst + (n * RT + i) * kWTile);
          } else {
            dma16(src, dst + (n * RT + i) * kWTile);
          }
        }
      dma16(xsrc0 + kb, dst + NA * RT * kWTile);
      dma16(xsrc1 + kb, dst + NA * RT * kWTile + 1024);
    };
    // Operand offsets in a stage (the inverse of the swizzles above).
    const int aoff = I8 ? 16 * (2 * r + ((g >> 1) ^ ((r >> 2) & 1))) + 8 * (g & 1)
                        : 16 * (4 * r + (g ^ ((r >> 1) & 3)));
    const int boff0 = NA * RT * kWTile + 16 * (8 * r + ((2 * g) ^ (r & 7)));
    const int boff1 = NA * RT * kWTile + 16 * (8 * r + ((2 * g + 1) ^ (r & 7)));
    // Blocks 0 and 1 go out first. NORM: then the norm weight, also by DMA (so
    // that every wait here is on this wave's own count of DMAs), and the whole
    // workgroup waits for it: its round trip overlaps the blocks' instead of
    // preceding them.
    if (nblk > 0) issue(0, 0);
    if (nblk > 1) issue(1, 1);
    if constexpr (NORM) {
      const int n4 = cols / 4;  // 16-byte pieces; lane l of a DMA lands at base + 16 l
      const unsigned norm_lds = lds_address(dyn);
      for (int i0 = 64 * wave; i0 < n4; i0 += 64 * W)
        if (i0 + lane < n4) dma16(norm.weight + 4 * (i0 + lane), norm_lds + 16 * i0);
      wait_vmcnt<0>();
      __syncthreads();
    }
    for (int j = 0; j < nblk; ++j) {
      // Block j's tiles have landed (block j + 1's, when there is one, may not).
      if (j + 1 < nblk)
        wait_vmcnt<kPerStage>();
      else
        wait_vmcnt<0>();
      const unsigned char* st = stages + (j & 1) * kStage;
      float4 x0 = *reinterpret_cast<const float4*>(st + boff0);
      float4 x1 = *reinterpret_cast<const float4*>(st + boff1);
      if constexpr (NORM) {
        const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) ss[0] = __builtin_fmaf(v[e], v[e], ss[0]);
        const float* wn = reinterpret_cast<const float*>(dyn) + 32 * (wave + W * j) + 8 * g;
        const float4 wn0 = *reinterpret_cast<const float4*>(wn);
        const float4 wn1 = *reinterpret_cast<const float4*>(wn + 4);
        x0 = make_float4(x0.x * wn0.x, x0.y * wn0.y, x0.z * wn0.z, x0.w * wn0.w);
        x1 = make_float4(x1.x * wn1.x, x1.y * wn1.y, x1.z * wn1.z, x1.w * wn1.w);
      }
      bf16x8 bh, bm, bl;
      split3(x0, x1, bh, bm, bl);
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          bf16x8 a;
          if constexpr (I8) {
            const uint2 raw = *reinterpret_cast<const uint2*>(st + (n * RT + i) * kWTile + aoff);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const uint32_t word = e < 4 ? raw.x : raw.y;
              a[e] = static_cast<bf16>(static_cast<float>(static_cast<int8_t>((word >> (8 * (e & 3))) & 0xFF)));
            }
          } else {
            a = *reinterpret_cast<const bf16x8*>(st + (n * RT + i) * kWTile + aoff);
          }
          acc[n][i][0] = mma3(a, bh, bm, bl, acc[n][i][0]);
        }
      // Block j + 2 into the stage just read, once those LDS reads are done
      // (s_waitcnt lgkmcnt(0), the other counters at their no-wait maxima).
      if (j + 2 < nblk) {
        __builtin_amdgcn_s_waitcnt(0xC07F);
        issue(j & 1, j + 2);
      }
    }
  } else
  for (int kb = 32 * wave; kb < cols; kb += 32 * W) {
    const int k = kb + 8 * g;
    const bool kin = k < cols;
    float4 wn0 = make_float4(1.f, 1.f, 1.f, 1.f), wn1 = wn0;
    if constexpr (NORM) {
      if (kin) {
        wn0 = *reinterpret_cast<const float4*>(norm.weight + k);
        wn1 = *reinterpret_cast<const float4*>(norm.weight + k + 4);
      }
    }
    bf16x8 a[NA][RT];
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      a[0][i] = kin ? load_weights<I8>(w, wrow[i] + k) : bf16x8{};
      if constexpr (GATE) a[NA - 1][i] = kin ? load_weights<I8>(w2, wrow[i] + k) : bf16x8{};
    }
#pragma unroll
    for (int j = 0; j < TT; ++j) {
      bf16x8 bh = {}, bm = {}, bl = {};
      if (kin) {
        const float4* xp = reinterpret_cast<const float4*>(xrow[j] + k);
        float4 x0 = xp[0], x1 = xp[1];
        if constexpr (NORM) {
          const float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) ss[j] = __builtin_fmaf(v[e], v[e], ss[j]);
          x0 = make_float4(x0.x * wn0.x, x0.y * wn0.y, x0.z * wn0.z, x0.w * wn0.w);
          x1 = make_float4(x1.x * wn1.x, x1.y * wn1.y, x1.z * wn1.z, x1.w * wn1.w);
        }
        split3(x0, x1, bh, bm, bl);
      }
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int i = 0; i < RT; ++i) acc[n][i][j] = mma3(a[n][i], bh, bm, bl, acc[n][i][j]);
    }
  }
  // NORM: the token's sum over the 4 lane groups of its K slices (lanes r,
  // r + 16, r + 32, r + 48), then with the tiles through the waves' tree.
  if constexpr (NORM) {
#pragma unroll
    for (int j = 0; j < TT; ++j) ss[j] = group_sum4(ss[j]);
  }
  // The waves' partial tiles summed through LDS in a fixed tree (waves 4-7
  // into 0-3, 2-3 into 0-1, 1 into 0), so results do not depend on timing.
#pragma unroll
  for (int half = W / 2; half >= 1; half /= 2) {
    if (wave >= half && wave < 2 * half) {
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int j = 0; j < TT; ++j) red[wave - half][(n * RT + i) * TT + j][lane] = acc[n][i][j];
      if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < TT; ++j) red_ss[wave - half][j][lane] = ss[j];
      }
    }
    __syncthreads();
    if (wave < half) {
#pragma unroll
      for (int n = 0; n < NA; ++n)
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int j = 0; j < TT; ++j) acc[n][i][j] += red[wave][(n * RT + i) * TT + j][lane];
      if constexpr (NORM) {
#pragma unroll
        for (int j = 0; j < TT; ++j) ss[j] += red_ss[wave][j][lane];
      }
    }
    __syncthreads();
  }
  if (wave > 0) return;
#pragma unroll
  for (int j = 0; j < TT; ++j) {
    const int tok = tok0 + 16 * j + r;
    if (tok >= T) break;
    // NORM: the token's 1 / rms (1 otherwise)
    const float inv = NORM ? 1.0f / sqrtf(ss[j] / float(cols) + norm.eps) : 1.0f;
#pragma unroll
    for (int i = 0; i < RT; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int row = row0 + 16 * i + 4 * g + e;
        if (row >= rows) break;
        float v = acc[0][i][j][e] * (I8 ? scale[row] : 1.0f);
        if constexpr (NORM) v *= inv;
        float* dst;
        if (row < out.split0)
          dst = y + size_t(tok) * out.split0 + row;
        else if (row < out.split1)
          dst = out.y1 + size_t(tok) * (out.split1 - out.split0) + (row - out.split0);
        else
          dst = out.y2 + size_t(tok) * (rows - out.split1) + (row - out.split1);
        if constexpr (GATE) {
          float u = acc[NA - 1][i][j][e] * (I8 ? scale2[row] : 1.0f);
          if constexpr (NORM) u *= inv;
          v = silu(v) * u;
        } else {
          if (bias) v += bias[row];
          if (accumulate) v += *dst;
        }
        *dst = v;
      }
    }
  }
}

// y[t] = x[t] * (1 / sqrt(mean(x[t]^2) + eps)) * weight; one workgroup per row.
// Each element is read and written by the same thread, so y may equal x.
__global__ void __launch_bounds__(256)
rmsnorm_kernel(float* y, const float* x, const float* __restrict__ weight, int dim, float eps) {
  __shared__ float part[4];
  const float* xt = x + size_t(blockIdx.x) * dim;
  float* yt = y + size_t(blockIdx.x) * dim;
  // Rows up to 8 elements a thread (2,048 floats) stay in registers between
  // the sum and the scaling, so the row is read once.
  constexpr int kHeld = 8;
  const bool held = dim <= kHeld * int(blockDim.x);
  float xv[kHeld];
  float ss = 0.0f;
  if (held) {
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      const int i = int(threadIdx.x) + j * int(blockDim.x);
      xv[j] = i < dim ? xt[i] : 0.0f;
      ss += xv[j] * xv[j];
    }
  } else {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) ss += xt[i] * xt[i];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  const float total = (part[0] + part[1]) + (part[2] + part[3]);
  const float inv_rms = 1.0f / sqrtf(total / float(dim) + eps);
  if (held) {
#pragma unroll
    for (int j = 0; j < kHeld; ++j) {
      const int i = int(threadIdx.x) + j * int(blockDim.x);
      if (i < dim) yt[i] = xv[j] * inv_rms * weight[i];
    }
  } else {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) yt[i] = xt[i] * inv_rms * weight[i];
  }
}

// x[t] = E[ids[t]] widened to f32 (times the row's scale for INT8).
__global__ void __launch_bounds__(256)
embedding_kernel(float* __restrict__ x, const int32_t* __restrict__ ids, const void* __restrict__ e,
                 const float* __restrict__ scale, int int8, int dim) {
  const int id = ids[blockIdx.x];
  float* xt = x + size_t(blockIdx.x) * dim;
  if (int8) {
    const int8_t* row = static_cast<const int8_t*>(e) + size_t(id) * dim;
    const float s = scale[id];
    for (int i = threadIdx.x; i < dim; i += blockDim.x) xt[i] = s * static_cast<float>(row[i]);
  } else {
    const uint16_t* row = static_cast<const uint16_t*>(e) + size_t(id) * dim;
    for (int i = threadIdx.x; i < dim; i += blockDim.x)
      xt[i] = __uint_as_float(static_cast<uint32_t>(row[i]) << 16);
  }
}

int check_matrix(const ie_matrix& m, const char* who) {
  if (!m.data || m.rows <= 0 || m.cols <= 0)
    return fail(IE_HIP_EINVAL, std::string(who) + ": empty weight matrix");
  if (m.int8 && !m.scale) return fail(IE_HIP_EINVAL, std::string(who) + ": INT8 needs row scales");
  return IE_HIP_OK;
}

// The staged kernel's launch: dynamic LDS = the norm weight (NORM) + two stages
// for each of the 8 waves. Returns false (nothing launched) when that exceeds
// kStagedMaxLds; *rc is the launch status otherwise.
constexpr int kStagedMaxLds = 128 * 1024;

template <bool G, int R, bool I8, bool N>
bool launch_staged_variant(const dim3 grid, hipStream_t stream, float* y, const float* x,
                           const ie_matrix& w, const void* w2d, const float* s2, const float* bias,
                           int T, int accumulate, RowSplit split, RowNorm norm, int* rc) {
  constexpr int kStage = (G ? 2 : 1) * R * (I8 ? 512 : 1024) + 2048;
  const size_t lds = (N ? size_t(w.cols) * 4 : 0) + size_t(2 * kMmWaves) * kStage;
  if (lds > size_t(kStagedMaxLds)) return false;
  const void* kernel = reinterpret_cast<const void*>(matmul_mfma_kernel<G, R, 1, kMmWaves, I8, N, true>);
  if (lds > 64 * 1024) {  // above the default dynamic-LDS cap, within gfx950's 160 KB
    static const hipError_t attr =
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kStagedMaxLds);
    if ((*rc = check_hip(attr, "hipFuncSetAttribute(matmul)"))) return true;
  }
  hipLaunchKernelGGL((matmul_mfma_kernel<G, R, 1, kMmWaves, I8, N, true>), grid, dim3(64 * kMmWaves),
                     lds, stream, y, x, w.data, w.scale, w2d, s2, bias, T, w.rows, w.cols, accumulate,
                     split, norm);
  *rc = IE_HIP_OK;
  return true;
}

template <bool G, int R>
bool launch_staged_rt(bool i8, bool n, const dim3 grid, hipStream_t stream, float* y,
                      const float* x, const ie_matrix& w, const void* w2d, const float* s2,
                      const float* bias, int T, int accumulate, RowSplit split, RowNorm norm,
                      int* rc) {
#define IE_MM_STAGED(I, N_)                                                                    return launch_staged_variant<G, R, I, N_>(grid, stream, y, x, w, w2d, s2, bias, T, accumulate,                                             split, norm, rc)
  if (i8) {
    if (n) IE_MM_STAGED(true, true);
    IE_MM_STAGED(true, false);
  }
  if (n) IE_MM_STAGED(false, true);
  IE_MM_STAGED(false, false);
#undef IE_MM_STAGED
}

int launch_matmul(bool gate, float* y, const float* x, const ie_matrix& w, const ie_matrix* w2,
                  const float* bias, int T, int accumulate, hipStream_t stream, const char* who,
                  RowSplit split = RowSplit{nullptr, nullptr, 0, 0},
                  RowNorm norm = RowNorm{nullptr, 0.0f}) {
  if (split.split0 == 0 && split.split1 == 0) split.split0 = split.split1 = w.rows;
  if (int rc = check_matrix(w, who)) return rc;
  if (w2) {
    if (int rc = check_matrix(*w2, who)) return rc;
    if (w2->rows != w.rows || w2->cols != w.cols || w2->int8 != w.int8)
      return fail(IE_HIP_EINVAL, std::string(who) + ": gate and up shapes differ");
  }
  if (T < 0) return fail(IE_HIP_EINVAL, std::string(who) + ": T < 0");
  if (T == 0) return IE_HIP_OK;
  if (!y || !x) return fail(IE_HIP_EINVAL, std::string(who) + ": null pointer");
  if (w.cols % 8)
    return fail(IE_HIP_EINVAL, std::string(who) + ": cols must be a multiple of 8");
  const uintptr_t align = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w.data) |
                          (w2 ? reinterpret_cast<uintptr_t>(w2->data) : 0);
  if (align & (w.int8 ? 7 : 15))
    return fail(IE_HIP_EINVAL, std::string(who) + ": x and the weights must be 16-byte aligned");
  // The waves of a workgroup split K, so their count fixes every output's
  // summation order. It depends on the matrix alone, never on T: a token's
  // result is then the same bit for bit whatever batch it is computed in (the
  // reference's "batch of N == N single tokens" contract,
  // src/cuda/cuda_runner.cu:798-829). Wide matrices (row tiles alone reach 16
  // per compute unit: the 151,936-row LM head) take 4-wave workgroups of 4 x 4
  // tiles: at ~140 registers a lane three fit on a compute unit where one of 8
  // would (LM head at 64 tokens: 176 -> 149 us on MI355X), each weight is read
  // once and each activation fragment a quarter as often (366 -> 172 us).
  // Otherwise 8 waves, and the tiles per workgroup (which do not change the
  // arithmetic) follow the count of 16 x 16 output tiles, measured at 64
  // tokens: below 4 per compute unit (q/k/v/o and down at 896 rows) one tile
  // per workgroup keeps every unit busy; from 4 per unit two row tiles share
  // each activation fragment, except for gate/up in the staged kernel (one row
  // tile, below).
  const int cus = device_compute_units();
  const bool wide = (w.rows + 15) / 16 >= 16 * cus;
  const int waves = wide ? 4 : kMmWaves;
  const int64_t tiles = int64_t((w.rows + 15) / 16) * ((T + 15) / 16);
  int RT = wide ? 4 : tiles >= 4 * int64_t(cus) ? 2 : 1;
  // The staged kernel (below) for every 8-wave launch whose K is whole 32-column
  // blocks and whose weights are 16-byte aligned (for the DMA).
  const bool staged = !wide && w.cols % 32 == 0 &&
                      ((reinterpret_cast<uintptr_t>(w.data) |
                        reinterpret_cast<uintptr_t>(w2 ? w2->data : nullptr)) & 15) == 0;
  // Two weight matrices: at most 2 row tiles; staged, one (its LDS then fits two
  // workgroups on a compute unit: config 6's gate/up, 1.657 -> 1.608 ms a step).
  if (gate) RT = std::min(RT, staged ? 1 : 2);
  const int tok_tiles = (T + 15) / 16;  // kernels exist for 1, 2 and 4 token tiles
  const int TT = !wide ? 1 : tok_tiles > 2 ? 4 : tok_tiles;
  const dim3 grid((w.rows + 16 * RT - 1) / (16 * RT), (T + 16 * TT - 1) / (16 * TT));
  const dim3 block(64 * waves);
  if (grid.y > 65535) return fail(IE_HIP_EINVAL, std::string(who) + ": too many tokens");
  const void* w2d = gate ? w2->data : nullptr;
  const float* s2 = gate ? w2->scale : nullptr;
  // The staged kernel: the same operands in the same order, so the same results
  // as the direct loads below.
  if (staged) {
    int rc = IE_HIP_OK;
    const bool n = norm.weight != nullptr;
    bool launched;
    if (gate)
      launched = RT == 2 ? launch_staged_rt<true, 2>(w.int8, n, grid, stream, y, x, w, w2d, s2, bias,
                                                     T, accumulate, split, norm, &rc)
                         : launch_staged_rt<true, 1>(w.int8, n, grid, stream, y, x, w, w2d, s2, bias,
                                                     T, accumulate, split, norm, &rc);
    else
      launched = RT == 2 ? launch_staged_rt<false, 2>(w.int8, n, grid, stream, y, x, w, w2d, s2, bias,
                                                      T, accumulate, split, norm, &rc)
                         : launch_staged_rt<false, 1>(w.int8, n, grid, stream, y, x, w, w2d, s2, bias,
                                                      T, accumulate, split, norm, &rc);
    if (launched) return rc != IE_HIP_OK ? rc : check_launch(who);
  }
  if (norm.weight) {
    // The folded rmsnorm exists for the 8-wave, one-token-tile launches (every
    // matrix below 16 row tiles per compute unit).
    if (wide) return fail(IE_HIP_EINVAL, std::string(who) + ": too many rows for the folded rmsnorm");
#define IE_MM_NORM(G, R)                                                                          \
  do {                                                                                            \
    if (w.int8)                                                                                   \
      hipLaunchKernelGGL((matmul_mfma_kernel<G, R, 1, kMmWaves, true, true>), grid, block, 0,     \
                         stream, y, x, w.data, w.scale, w2d, s2, bias, T, w.rows, w.cols,         \
                         accumulate, split, norm);                                                \
    else                                                                                          \
      hipLaunchKernelGGL((matmul_mfma_kernel<G, R, 1, kMmWaves, false, true>), grid, block, 0,    \
                         stream, y, x, w.data, w.scale, w2d, s2, bias, T, w.rows, w.cols,         \
                         accumulate, split, norm);                                                \
  } while (0)
    if (gate) {
      if (RT == 2)
        IE_MM_NORM(true, 2);
      else
        IE_MM_NORM(true, 1);
    } else {
      if (RT == 2)
        IE_MM_NORM(false, 2);
      else
        IE_MM_NORM(false, 1);
    }
#undef IE_MM_NORM
    return check_launch(who);
  }
#define IE_MM_LAUNCH_W(G, R, C, W)                                                               \
  do {                                                                                           \
    if (w.int8)                                                                                  \
      hipLaunchKernelGGL((matmul_mfma_kernel<G, R, C, W, true>), grid, block, 0, stream, y, x,   \
                         w.data, w.scale, w2d, s2, bias, T, w.rows, w.cols, accumulate, split,   \
                         norm);                                                                  \
    else                                                                                         \
      hipLaunchKernelGGL((matmul_mfma_kernel<G, R, C, W, false>), grid, block, 0, stream, y, x,  \
                         w.data, w.scale, w2d, s2, bias, T, w.rows, w.cols, accumulate, split,   \
                         norm);                                                                  \
  } while (0)
#define IE_MM_LAUNCH(G, R, C)            \
  do {                                   \
    if (wide)                            \
      IE_MM_LAUNCH_W(G, R, C, 4);        \
    else                                 \
      IE_MM_LAUNCH_W(G, R, C, kMmWaves); \
  } while (0)
#define IE_MM_TT(G, R)            \
  if (TT == 4)                    \
    IE_MM_LAUNCH(G, R, 4);        \
  else if (TT == 2)               \
    IE_MM_LAUNCH(G, R, 2);        \
  else                            \
    IE_MM_LAUNCH(G, R, 1);
  if (gate) {
    if (RT == 2) {
      IE_MM_TT(true, 2)
    } else {
      IE_MM_TT(true, 1)
    }
  } else if (RT == 4) {
    IE_MM_TT(false, 4)
  } else if (RT == 2) {
    IE_MM_TT(false, 2)
  } else {
    IE_MM_TT(false, 1)
  }
#undef IE_MM_TT
#undef IE_MM_LAUNCH
#undef IE_MM_LAUNCH_W
  return check_launch(who);
}

}  // namespace
}  // namespace iehip

using namespace iehip;

extern "C" int ie_hip_embedding(float* x, const int32_t* ids, ie_matrix e, int T,
                                hipStream_t stream) {
  clear_error();
  if (int rc = check_matrix(e, "embedding")) return rc;
  if (T < 0) return fail(IE_HIP_EINVAL, "embedding: T < 0");
  if (T == 0) return IE_HIP_OK;
  if (!x || !ids) return fail(IE_HIP_EINVAL, "embedding: null pointer");
  hipLaunchKernelGGL(embedding_kernel, dim3(T), dim3(256), 0, stream, x, ids, e.data, e.scale,
                     e.int8, e.cols);
  return check_launch("embedding");
}

extern "C" int ie_hip_rmsnorm(float* y, const float* x, const float* weight, int T, int dim,
                              float eps, hipStream_t stream) {
  clear_error();
  if (T < 0 || dim <= 0) return fail(IE_HIP_EINVAL, "rmsnorm: bad sizes");
  if (T == 0) return IE_HIP_OK;
  if (!y || !x || !weight) return fail(IE_HIP_EINVAL, "rmsnorm: null pointer");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(T), dim3(256), 0, stream, y, x, weight, dim, eps);
  return check_launch("rmsnorm");
}

extern "C" int ie_hip_matmul(float* y, const float* x, ie_matrix w, const float* bias, int T,
                             int accumulate, hipStream_t stream) {
  clear_error();
  return launch_matmul(false, y, x, w, nullptr, bias, T, accumulate, stream, "matmul");
}

extern "C" int ie_hip_qkv_proj(float* q, float* k, float* v, const float* x, ie_matrix w_qkv,
                               const float* b_qkv, int T, int q_dim, int kv_dim,
                               hipStream_t stream) {
  clear_error();
  if (q_dim <= 0 || kv_dim <= 0 || w_qkv.rows != q_dim + 2 * kv_dim)
    return fail(IE_HIP_EINVAL, "qkv_proj: weight rows must be q_dim + 2 kv_dim");
  if (T > 0 && (!q || !k || !v)) return fail(IE_HIP_EINVAL, "qkv_proj: null pointer");
  return launch_matmul(false, q, x, w_qkv, nullptr, b_qkv, T, 0, stream, "qkv_proj",
                       RowSplit{k, v, q_dim, q_dim + kv_dim});
}

extern "C" int ie_hip_gate_up_silu(float* out, const float* x, ie_matrix w_gate, ie_matrix w_up,
                                   int T, hipStream_t stream) {
  clear_error();
  return launch_matmul(true, out, x, w_gate, &w_up, nullptr, T, 0, stream, "gate_up_silu");
}

extern "C" int ie_hip_rmsnorm_qkv_proj(float* q, float* k, float* v, const float* x,
                                       const float* norm_weight, float eps, ie_matrix w_qkv,
                                       const float* b_qkv, int T, int q_dim, int kv_dim,
                                       hipStream_t stream) {
  clear_error();
  if (q_dim <= 0 || kv_dim <= 0 || w_qkv.rows != q_dim + 2 * kv_dim)
    return fail(IE_HIP_EINVAL, "rmsnorm_qkv_proj: weight rows must be q_dim + 2 kv_dim");
  if (T > 0 && (!q || !k || !v || !norm_weight))
    return fail(IE_HIP_EINVAL, "rmsnorm_qkv_proj: null pointer");
  if (reinterpret_cast<uintptr_t>(norm_weight) & 15)
    return fail(IE_HIP_EINVAL, "rmsnorm_qkv_proj: the norm weight must be 16-byte aligned");
  return launch_matmul(false, q, x, w_qkv, nullptr, b_qkv, T, 0, stream, "rmsnorm_qkv_proj",
                       RowSplit{k, v, q_dim, q_dim + kv_dim}, RowNorm{norm_weight, eps});
}

extern "C" int ie_hip_rmsnorm_gate_up_silu(float* out, const float* x, const float* norm_weight,
                                           float eps, ie_matrix w_gate, ie_matrix w_up, int T,
                                           hipStream_t stream) {
  clear_error();
  if (T > 0 && !norm_weight) return fail(IE_HIP_EINVAL, "rmsnorm_gate_up_silu: null pointer");
  if (reinterpret_cast<uintptr_t>(norm_weight) & 15)
    return fail(IE_HIP_EINVAL, "rmsnorm_gate_up_silu: the norm weight must be 16-byte aligned");
  return launch_matmul(true, out, x, w_gate, &w_up, nullptr, T, 0, stream, "rmsnorm_gate_up_silu",
                       RowSplit{nullptr, nullptr, 0, 0}, RowNorm{norm_weight, eps});
}
