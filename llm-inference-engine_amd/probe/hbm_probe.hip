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
// Each comes in two load forms: plain, and with the non-temporal hint (the
// form the decode kernels use for their pages); the bench takes the faster.
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

// The same with non-temporal loads.
int ie_probe_read_nt(const void* src, size_t bytes, int workgroups, uint32_t* sink,
                     hipStream_t stream) {
  if (!src || !sink || bytes % 16 || workgroups <= 0) return 1;
  hipLaunchKernelGGL(probe_read_kernel<true>, dim3(workgroups), dim3(kThreads), 0, stream,
                     static_cast<const uint4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The page walk of a flash-decoding launch of `items` (row, chunk) workgroups;
// ie_probe_pages_nt with non-temporal loads.
int ie_probe_pages(const void* k_pool, const void* v_pool, const int32_t* tables,
                   const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                   int items, int max_pages, int chunk_tokens, int page_bytes, uint32_t* sink,
                   hipStream_t stream) {
  return probe_pages<false>(k_pool, v_pool, tables, work_row, work_chunk, row_len, items,
                            max_pages, chunk_tokens, page_bytes, sink, stream);
}
int ie_probe_pages_nt(const void* k_pool, const void* v_pool, const int32_t* tables,
                      const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                      int items, int max_pages, int chunk_tokens, int page_bytes, uint32_t* sink,
                      hipStream_t stream) {
  return probe_pages<true>(k_pool, v_pool, tables, work_row, work_chunk, row_len, items,
                           max_pages, chunk_tokens, page_bytes, sink, stream);
}

}  // extern "C"
