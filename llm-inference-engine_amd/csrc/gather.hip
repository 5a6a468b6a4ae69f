// Row gather and block-table gather (gfx950).
#include "common.hpp"

namespace iehip {
namespace {

// dst[r, :] = src[rows[r], :]  (reference: src/cuda/kernels.cu:778-783).
// One workgroup per output row; 16-byte copies when the row allows them.
__global__ void __launch_bounds__(256)
gather_rows_kernel(float* __restrict__ dst, const float* __restrict__ src,
                   const int32_t* __restrict__ rows, int dim, int vec4) {
  const float* in = src + size_t(rows[blockIdx.x]) * dim;
  float* out = dst + size_t(blockIdx.x) * dim;
  if (vec4) {
    const float4* in4 = reinterpret_cast<const float4*>(in);
    float4* out4 = reinterpret_cast<float4*>(out);
    for (int i = threadIdx.x; i < dim / 4; i += blockDim.x) out4[i] = in4[i];
  } else {
    for (int i = threadIdx.x; i < dim; i += blockDim.x) out[i] = in[i];
  }
}

// dst[p, :] = widen(pool row of (seq, p)), p < len: the paged -> contiguous copy
// (reference self-test: src/cuda/cuda_runner.cu:959-964). One thread per 8
// elements; positions whose page id lies outside the pool are written as 0.
template <int KV>
__global__ void __launch_bounds__(256)
gather_kv_kernel(float* __restrict__ dst, const typename Kv<KV>::elem* __restrict__ pool,
                 const int32_t* __restrict__ tables, int max_pages, int num_pages, int seq,
                 int len, int kv_dim) {
  const int per_row = kv_dim / 8;
  const int64_t gid = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  const int p = int(gid / per_row);
  if (p >= len) return;
  const int i = int(gid - int64_t(p) * per_row) * 8;
  const int page_index = p / IE_HIP_PAGE_SIZE;
  const int page = page_index < max_pages ? tables[size_t(seq) * max_pages + page_index] : -1;
  float x[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (page >= 0 && page < num_pages)
    Kv<KV>::load8(pool + (size_t(page) * IE_HIP_PAGE_SIZE + p % IE_HIP_PAGE_SIZE) * kv_dim + i, x);
  float4* o = reinterpret_cast<float4*>(dst + size_t(p) * kv_dim + i);
  o[0] = make_float4(x[0], x[1], x[2], x[3]);
  o[1] = make_float4(x[4], x[5], x[6], x[7]);
}

}  // namespace
}  // namespace iehip

using namespace iehip;

extern "C" int ie_hip_gather_rows(float* dst, const float* src, const int32_t* rows, int R, int dim,
                                  hipStream_t stream) {
  clear_error();
  if (R < 0 || dim <= 0) return fail(IE_HIP_EINVAL, "gather_rows: bad sizes");
  if (R == 0) return IE_HIP_OK;
  if (!dst || !src || !rows) return fail(IE_HIP_EINVAL, "gather_rows: null pointer");
  const int vec4 = (dim % 4 == 0 && (reinterpret_cast<uintptr_t>(dst) % 16) == 0 &&
                    (reinterpret_cast<uintptr_t>(src) % 16) == 0);
  hipLaunchKernelGGL(gather_rows_kernel, dim3(R), dim3(256), 0, stream, dst, src, rows, dim, vec4);
  return check_launch("gather_rows");
}

extern "C" int ie_hip_gather_kv(float* dst, const void* pool, ie_kv_layout kv, int seq, int len,
                                int kv_dim, hipStream_t stream) {
  clear_error();
  if (int rc = check_layout(kv, "gather_kv")) return rc;
  if (seq < 0 || len < 0 || kv_dim <= 0 || kv_dim % 8)
    return fail(IE_HIP_EINVAL, "gather_kv: bad sizes (kv_dim must be a multiple of 8)");
  if (len == 0) return IE_HIP_OK;
  if (!dst || !pool) return fail(IE_HIP_EINVAL, "gather_kv: null pointer");
  const int64_t threads = int64_t(len) * (kv_dim / 8);
  const unsigned blocks = unsigned((threads + 255) / 256);
#define IE_GATHER_CASE(KVT)                                                                        \
  if (kv.kv_dtype == KVT) {                                                                        \
    hipLaunchKernelGGL((gather_kv_kernel<KVT>), dim3(blocks), dim3(256), 0, stream, dst,           \
                       static_cast<const typename Kv<KVT>::elem*>(pool), kv.tables, kv.max_pages,  \
                       kv.num_pages, seq, len, kv_dim);                                            \
    return check_launch("gather_kv");                                                              \
  }
  IE_GATHER_CASE(IE_KV_F32)
  IE_GATHER_CASE(IE_KV_F16)
  IE_GATHER_CASE(IE_KV_BF16)
#undef IE_GATHER_CASE
  return fail(IE_HIP_EINVAL, "gather_kv: unsupported kv_dtype");
}
