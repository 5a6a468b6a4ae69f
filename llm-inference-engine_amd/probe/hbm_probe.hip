// HBM probes for bench.py (measurement only; not part of libie_hip.so): the
// read rate a kernel with no arithmetic reaches on this device, so that the
// decode kernel's rate can be set against a measured ceiling next to the
// nominal 8 TB/s. The reference measures its ceiling the same way, with a
// device-to-device copy kernel (src/cuda/device_check.cu:78-112).
//
// ie_probe_read: a contiguous stream. Every thread reads 16-byte pieces in a
// grid stride, four in flight, and folds them into one word; the word is
// stored only when it equals a value the data never produces, so the loads
// stay and the stores do not count.
//
// Each comes in four load forms: 16-byte loads into registers, plain or with
// the non-temporal hint, and LDS DMA (global_load_lds_dwordx4: 1 KB per wave
// instruction straight into LDS, the form the decode kernels read V pages
// with), plain or non-temporal; the bench takes the fastest.
//
// ie_probe_pages: the decode kernel's access pattern without its arithmetic.
// One workgroup per (row, chunk of chunk_tokens positions) of a batch in block
// tables, exactly as the flash-decoding grid: it reads the chunk's page ids,
// then every K and V page of the chunk (16 rows of 256 bytes at f16), and
// folds them the same way. Its rate is the floor the decode kernel's data
// movement cannot beat.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ uint32_t fold(uint4 a) { return a.x ^ (a.y * 3u) ^ (a.z * 5u) ^ (a.w * 7u); }

// One wave instruction moving 1 KB from src (lane l: bytes 16 l ..) to LDS
// address lds (lane l lands at lds + 16 l).
template <bool NT>
__device__ __forceinline__ void dma_1k(const void* src, unsigned lds) {
  if constexpr (NT)
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
  else
    asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
                 :
                 : "v"(src), "s"(lds)
                 : "memory", "m0");
}

__device__ __forceinline__ unsigned lds_base(const void* p) {
  return __builtin_amdgcn_readfirstlane(static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p))));
}

template <bool NT>
__device__ __forceinline__ uint4 load16(const void* p) {
  if constexpr (NT) {
    typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
    const u32x4 v = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
    return uint4{v.x, v.y, v.z, v.w};
  } else {
    return *static_cast<const uint4*>(p);
  }
}

template <bool NT>
__global__ void __launch_bounds__(kThreads)
probe_read_kernel(const uint4* __restrict__ src, size_t n16, uint32_t* __restrict__ sink) {
  const size_t stride = size_t(gridDim.x) * kThreads;
  size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = load16<NT>(src + i), b = load16<NT>(src + i + stride),
                c = load16<NT>(src + i + 2 * stride), d = load16<NT>(src + i + 3 * stride);
    acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
  }
  for (; i < n16; i += stride) acc ^= fold(load16<NT>(src + i));
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// The contiguous stream by LDS DMA: each wave moves 4 KB blocks (4 x 1 KB)
// into its own LDS area, grid-stride over the blocks, one block in flight, and
// folds one word of each so that the loads stay.
template <bool NT>
__global__ void __launch_bounds__(kThreads)
probe_read_dma_kernel(const unsigned char* __restrict__ src, size_t blocks,
                      uint32_t* __restrict__ sink) {
  __shared__ __align__(16) unsigned char buf[kThreads / 64][4096];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const unsigned base = lds_base(&buf[wave][0]);
  uint32_t acc = 0;
  for (size_t b = size_t(blockIdx.x) * (kThreads / 64) + wave; b < blocks;
       b += size_t(gridDim.x) * (kThreads / 64)) {
    const unsigned char* p = src + b * 4096 + lane * 16;
#pragma unroll
    for (int u = 0; u < 4; ++u) dma_1k<NT>(p + u * 1024, base + u * 1024);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    acc ^= fold(*reinterpret_cast<const uint4*>(&buf[wave][lane * 16]));
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// Workgroup = (row, chunk), numbered row by row over each row's own chunk
// count (computed by the host). A page of one pool is 16 rows x row_bytes;
// 256 threads x 16 bytes cover 4 KB per load round.
template <bool NT>
__global__ void __launch_bounds__(kThreads)
probe_pages_kernel(const unsigned char* __restrict__ k_pool, const unsigned char* __restrict__ v_pool,
                   const int32_t* __restrict__ tables, const int32_t* __restrict__ work_row,
                   const int32_t* __restrict__ work_chunk, const int32_t* __restrict__ row_len,
                   int max_pages, int chunk_tokens, int page_bytes, uint32_t* __restrict__ sink) {
  const int w = blockIdx.x;
  const int row = work_row[w], c = work_chunk[w];
  const int len = row_len[row];
  const int p0 = c * chunk_tokens / 16;
  const int p1 = min((c + 1) * chunk_tokens, len);
  const int np = (p1 - c * chunk_tokens + 15) / 16;
  const int32_t* tab = tables + size_t(row) * max_pages + p0;
  const int per_page = page_bytes / 16;
  uint32_t acc = 0;
  for (int j = threadIdx.x; j < np * per_page; j += 4 * kThreads) {
    uint4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int jj = j + u * kThreads;
      const int pg = jj < np * per_page ? tab[jj / per_page] : 0;
      const size_t off = size_t(pg) * page_bytes + size_t(jj % per_page) * 16;
      const bool in = jj < np * per_page;
      a[u] = in ? load16<NT>(k_pool + off) : uint4{0, 0, 0, 0};
      b[u] = in ? load16<NT>(v_pool + off) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= fold(a[u]) ^ fold(b[u]);
  }
  if (acc == 0x9E3779B9u) sink[w] = acc;
}

// The same walk by LDS DMA: wave w of the workgroup moves pages w, w + 4, ...
// of the chunk, K then V (page_bytes / 1 KB instructions each), one page in
// flight per wave.
template <bool NT>
__global__ void __launch_bounds__(kThreads)
probe_pages_dma_kernel(const unsigned char* __restrict__ k_pool,
                       const unsigned char* __restrict__ v_pool, const int32_t* __restrict__ tables,
                       const int32_t* __restrict__ work_row, const int32_t* __restrict__ work_chunk,
                       const int32_t* __restrict__ row_len, int max_pages, int chunk_tokens,
                       int page_bytes, uint32_t* __restrict__ sink) {
  extern __shared__ __align__(16) unsigned char dbuf[];  // [4 waves][2 pools][page_bytes]
  const int w = blockIdx.x, wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row = work_row[w], c = work_chunk[w];
  const int len = row_len[row];
  const int p0 = c * chunk_tokens / 16;
  const int np = (min((c + 1) * chunk_tokens, len) - c * chunk_tokens + 15) / 16;
  const int32_t* tab = tables + size_t(row) * max_pages + p0;
  unsigned char* mine = dbuf + size_t(wave) * 2 * page_bytes;
  const unsigned base = lds_base(mine);
  const int per = page_bytes / 1024;
  uint32_t acc = 0;
  for (int pg = wave; pg < np; pg += kThreads / 64) {
    const size_t off = size_t(tab[pg]) * page_bytes + lane * 16;
    for (int u = 0; u < per; ++u) dma_1k<NT>(k_pool + off + u * 1024, base + u * 1024);
    for (int u = 0; u < per; ++u) dma_1k<NT>(v_pool + off + u * 1024, base + page_bytes + u * 1024);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    acc ^= fold(*reinterpret_cast<const uint4*>(mine + lane * 16)) ^
           fold(*reinterpret_cast<const uint4*>(mine + page_bytes + lane * 16));
  }
  if (acc == 0x9E3779B9u) sink[w] = acc;
}

// A walk of random 4 KB pages that owes nothing to the decode kernel's shape:
// persistent one-wave workgroups over a flat list of page ids (each entry = the
// K page and the V page of that id, 8 KB), every wave a contiguous, balanced
// range of the list, with R pages in flight per wave in an LDS ring of R
// stages (non-temporal LDS DMA, 8 instructions of 1 KB per page). The wave
// waits for the oldest page only (vmcnt counts the 8 x (R-1) instructions
// issued after it), folds a word of it and refills its stage. A wave's range
// is at most 64 pages (its ids are loaded once, one per lane).
template <int R>
__global__ void __launch_bounds__(64)
probe_ring_kernel(const unsigned char* __restrict__ k_pool, const unsigned char* __restrict__ v_pool,
                  const int32_t* __restrict__ pages, int n, uint32_t* __restrict__ sink) {
  extern __shared__ __align__(16) unsigned char ring[];  // [R][2 pools][4096]
  const int lane = threadIdx.x;
  const int64_t waves = gridDim.x;
  const int begin = int(int64_t(n) * blockIdx.x / waves);
  const int cnt = int(int64_t(n) * (blockIdx.x + 1) / waves) - begin;
  const int id_lane = lane < cnt ? pages[begin + lane] : 0;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  const unsigned base = lds_base(ring);
  auto issue = [&](const int u) {
    const size_t off = size_t(__builtin_amdgcn_readlane(id_lane, u)) * 4096 + lane * 16;
    const unsigned st = base + (u % R) * 8192;
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_1k<true>(k_pool + off + i * 1024, st + i * 1024);
#pragma unroll
    for (int i = 0; i < 4; ++i) dma_1k<true>(v_pool + off + i * 1024, st + 4096 + i * 1024);
  };
  for (int u = 0; u < R && u < cnt; ++u) issue(u);
  uint32_t acc = 0;
  for (int u = 0; u < cnt; ++u) {
    if (u + R - 1 < cnt) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(8 * (R - 1)) : "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
    const unsigned char* st = ring + (u % R) * 8192;
    acc ^= fold(*reinterpret_cast<const uint4*>(st + lane * 16)) ^
           fold(*reinterpret_cast<const uint4*>(st + 4096 + lane * 16));
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the stage is read before it is refilled
    if (u + R < cnt) issue(u + R);
  }
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

template <bool NT>
int probe_pages(const void* k_pool, const void* v_pool, const int32_t* tables,
                       const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                       int items, int max_pages, int chunk_tokens, int page_bytes, uint32_t* sink,
                       hipStream_t stream) {
  if (!k_pool || !v_pool || !tables || items <= 0 || chunk_tokens % 16 || page_bytes % 16)
    return 1;
  hipLaunchKernelGGL(probe_pages_kernel<NT>, dim3(items), dim3(kThreads), 0, stream,
                     static_cast<const unsigned char*>(k_pool),
                     static_cast<const unsigned char*>(v_pool), tables, work_row, work_chunk,
                     row_len, max_pages, chunk_tokens, page_bytes, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from src with `workgroups` workgroups of 256
// threads; sink holds one word per workgroup.
int ie_probe_read(const void* src, size_t bytes, int workgroups, uint32_t* sink,
                  hipStream_t stream) {
  if (!src || !sink || bytes % 16 || workgroups <= 0) return 1;
  hipLaunchKernelGGL(probe_read_kernel<false>, dim3(workgroups), dim3(kThreads), 0, stream,
                     static_cast<const uint4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Forms: 0 plain loads, 1 non-temporal loads, 2 LDS DMA, 3 non-temporal LDS
// DMA. The DMA forms read bytes / 4096 whole 4 KB blocks.
int ie_probe_read_form(const void* src, size_t bytes, int workgroups, int form, uint32_t* sink,
                       hipStream_t stream) {
  if (!src || !sink || bytes % 16 || workgroups <= 0 || form < 0 || form > 3) return 1;
  const dim3 g(workgroups), b(kThreads);
  if (form == 0)
    hipLaunchKernelGGL(probe_read_kernel<false>, g, b, 0, stream, static_cast<const uint4*>(src),
                       bytes / 16, sink);
  else if (form == 1)
    hipLaunchKernelGGL(probe_read_kernel<true>, g, b, 0, stream, static_cast<const uint4*>(src),
                       bytes / 16, sink);
  else if (form == 2)
    hipLaunchKernelGGL(probe_read_dma_kernel<false>, g, b, 0, stream,
                       static_cast<const unsigned char*>(src), bytes / 4096, sink);
  else
    hipLaunchKernelGGL(probe_read_dma_kernel<true>, g, b, 0, stream,
                       static_cast<const unsigned char*>(src), bytes / 4096, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The page walk of a flash-decoding launch of `items` (row, chunk) workgroups.
int ie_probe_pages(const void* k_pool, const void* v_pool, const int32_t* tables,
                   const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                   int items, int max_pages, int chunk_tokens, int page_bytes, uint32_t* sink,
                   hipStream_t stream) {
  return probe_pages<false>(k_pool, v_pool, tables, work_row, work_chunk, row_len, items,
                            max_pages, chunk_tokens, page_bytes, sink, stream);
}
// Forms as for ie_probe_read_form; the DMA forms need page_bytes % 1024 == 0
// (8 KB of LDS per page and wave, at most 8 KB pages).
int ie_probe_pages_form(const void* k_pool, const void* v_pool, const int32_t* tables,
                        const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                        int items, int max_pages, int chunk_tokens, int page_bytes, int form,
                        uint32_t* sink, hipStream_t stream) {
  if (form == 0 || form == 1)
    return form ? probe_pages<true>(k_pool, v_pool, tables, work_row, work_chunk, row_len, items,
                                    max_pages, chunk_tokens, page_bytes, sink, stream)
                : probe_pages<false>(k_pool, v_pool, tables, work_row, work_chunk, row_len, items,
                                     max_pages, chunk_tokens, page_bytes, sink, stream);
  if (form != 2 && form != 3) return 1;
  if (!k_pool || !v_pool || !tables || items <= 0 || chunk_tokens % 16 || page_bytes % 1024 ||
      page_bytes > 8192)
    return 1;
  const size_t lds = size_t(kThreads / 64) * 2 * page_bytes;
  const auto kern = form == 3 ? probe_pages_dma_kernel<true> : probe_pages_dma_kernel<false>;
  hipLaunchKernelGGL(kern, dim3(items), dim3(kThreads), lds, stream,
                     static_cast<const unsigned char*>(k_pool),
                     static_cast<const unsigned char*>(v_pool), tables, work_row, work_chunk,
                     row_len, max_pages, chunk_tokens, page_bytes, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The persistent ring walk: `waves` one-wave workgroups over the flat list of
// n page ids (each the K page and the V page of that id, 4 KB each), `ring`
// pages in flight per wave (1, 2, 4 or 8; ring x 8 KB of LDS per wave). Every
// wave's range must fit 64 pages: n <= 64 x waves.
int ie_probe_pages_ring(const void* k_pool, const void* v_pool, const int32_t* pages, int n,
                        int waves, int ring, uint32_t* sink, hipStream_t stream) {
  if (!k_pool || !v_pool || !pages || !sink || n <= 0 || waves <= 0 ||
      int64_t(n) > 64 * int64_t(waves))
    return 1;
  const dim3 g(waves), b(64);
  const size_t lds = size_t(ring) * 8192;
  switch (ring) {
    case 1:
      hipLaunchKernelGGL(probe_ring_kernel<1>, g, b, lds, stream,
                         static_cast<const unsigned char*>(k_pool),
                         static_cast<const unsigned char*>(v_pool), pages, n, sink);
      break;
    case 2:
      hipLaunchKernelGGL(probe_ring_kernel<2>, g, b, lds, stream,
                         static_cast<const unsigned char*>(k_pool),
                         static_cast<const unsigned char*>(v_pool), pages, n, sink);
      break;
    case 4:
      hipLaunchKernelGGL(probe_ring_kernel<4>, g, b, lds, stream,
                         static_cast<const unsigned char*>(k_pool),
                         static_cast<const unsigned char*>(v_pool), pages, n, sink);
      break;
    case 8: {
      static const hipError_t attr = hipFuncSetAttribute(
          reinterpret_cast<const void*>(probe_ring_kernel<8>),
          hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
      if (attr != hipSuccess) return 2;
      hipLaunchKernelGGL(probe_ring_kernel<8>, g, b, lds, stream,
                         static_cast<const unsigned char*>(k_pool),
                         static_cast<const unsigned char*>(v_pool), pages, n, sink);
      break;
    }
    default:
      return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
