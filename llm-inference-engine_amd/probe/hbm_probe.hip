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

__global__ void __launch_bounds__(kThreads)
probe_read_kernel(const uint4* __restrict__ src, size_t n16, uint32_t* __restrict__ sink) {
  const size_t stride = size_t(gridDim.x) * kThreads;
  size_t i = size_t(blockIdx.x) * kThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + 3 * stride < n16; i += 4 * stride) {
    const uint4 a = src[i], b = src[i + stride], c = src[i + 2 * stride], d = src[i + 3 * stride];
    acc ^= fold(a) ^ fold(b) ^ fold(c) ^ fold(d);
  }
  for (; i < n16; i += stride) acc ^= fold(src[i]);
  if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

// Workgroup = (row, chunk), numbered row by row over each row's own chunk
// count (computed by the host). A page of one pool is 16 rows x row_bytes;
// 256 threads x 16 bytes cover 4 KB per load round.
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
      a[u] = in ? *reinterpret_cast<const uint4*>(k_pool + off) : uint4{0, 0, 0, 0};
      b[u] = in ? *reinterpret_cast<const uint4*>(v_pool + off) : uint4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) acc ^= fold(a[u]) ^ fold(b[u]);
  }
  if (acc == 0x9E3779B9u) sink[w] = acc;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) from src with `workgroups` workgroups of 256
// threads; sink holds one word per workgroup.
int ie_probe_read(const void* src, size_t bytes, int workgroups, uint32_t* sink,
                  hipStream_t stream) {
  if (!src || !sink || bytes % 16 || workgroups <= 0) return 1;
  hipLaunchKernelGGL(probe_read_kernel, dim3(workgroups), dim3(kThreads), 0, stream,
                     static_cast<const uint4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// The page walk of a flash-decoding launch of `items` (row, chunk) workgroups.
int ie_probe_pages(const void* k_pool, const void* v_pool, const int32_t* tables,
                   const int32_t* work_row, const int32_t* work_chunk, const int32_t* row_len,
                   int items, int max_pages, int chunk_tokens, int page_bytes, uint32_t* sink,
                   hipStream_t stream) {
  if (!k_pool || !v_pool || !tables || items <= 0 || chunk_tokens % 16 || page_bytes % 16)
    return 1;
  hipLaunchKernelGGL(probe_pages_kernel, dim3(items), dim3(kThreads), 0, stream,
                     static_cast<const unsigned char*>(k_pool),
                     static_cast<const unsigned char*>(v_pool), tables, work_row, work_chunk,
                     row_len, max_pages, chunk_tokens, page_bytes, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
