// Greedy token choice on the device: the index of each logit row's maximum,
// so a greedy decode step copies back R token ids instead of R x vocab floats
// (BatchRunner::prefill_greedy / decode_greedy, src/runner.h:64-68).
//
// Semantics are the reference's CPU argmax (src/sampler.cpp:26-31): a scan from
// element 0 that moves only on a strictly greater value. So ties go to the
// lowest index, NaNs are never chosen, a NaN in element 0 gives 0 (nothing
// compares greater than it), and a row of -inf gives 0. (The reference's GPU
// kernel, src/cuda/kernels.cu:785-812, returns 0x7fffffff for a row with no
// value above -inf; this one follows the CPU.)
//
// One workgroup of 1,024 threads per row. A thread scans a strided set of
// 16-byte pieces, four loads in flight, keeping the first strict maximum it
// sees (its indices only increase); the workgroup then keeps the larger value,
// the lower index on ties: wave64 butterflies, then the 16 waves through LDS.
#include "common.hpp"

namespace iehip {
namespace {

constexpr int kArgThreads = 1024;

struct Best {
  float v;
  int i;
};

__device__ __forceinline__ Best better(Best a, Best b) {
  // b wins with a larger value, or an equal one at a lower index. An unset
  // slot (i = INT_MAX, v = -inf) loses to every set one.
  return (b.v > a.v || (b.v == a.v && b.i < a.i)) ? b : a;
}

__device__ __forceinline__ void consider(Best& b, float v, int i) {
  if (v > b.v) {
    b.v = v;
    b.i = i;
  }
}

__global__ void __launch_bounds__(kArgThreads)
argmax_rows_kernel(int32_t* __restrict__ out, const float* __restrict__ x, int n, int vec4) {
  __shared__ Best red[kArgThreads / 64];
  const float* row = x + size_t(blockIdx.x) * n;
  const int tid = threadIdx.x;
  Best b{-INFINITY, 0x7fffffff};
  if (vec4) {
    const float4* r4 = reinterpret_cast<const float4*>(row);
    const int n4 = n / 4;
    int i = tid;
    for (; i + 3 * kArgThreads < n4; i += 4 * kArgThreads) {
      float4 a[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) a[u] = r4[i + u * kArgThreads];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = 4 * (i + u * kArgThreads);
        consider(b, a[u].x, e);
        consider(b, a[u].y, e + 1);
        consider(b, a[u].z, e + 2);
        consider(b, a[u].w, e + 3);
      }
    }
    for (; i < n4; i += kArgThreads) {
      const float4 a = r4[i];
      consider(b, a.x, 4 * i);
      consider(b, a.y, 4 * i + 1);
      consider(b, a.z, 4 * i + 2);
      consider(b, a.w, 4 * i + 3);
    }
    for (int e = 4 * n4 + tid; e < n; e += kArgThreads) consider(b, row[e], e);
  } else {
    for (int e = tid; e < n; e += kArgThreads) consider(b, row[e], e);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    Best o;
    o.v = __shfl_xor(b.v, off, 64);
    o.i = __shfl_xor(b.i, off, 64);
    b = better(b, o);
  }
  if ((tid & 63) == 0) red[tid >> 6] = b;
  __syncthreads();
  if (tid != 0) return;
  Best r = red[0];
  for (int w = 1; w < kArgThreads / 64; ++w) r = better(r, red[w]);
  // Element 0 NaN, or nothing above -inf: the CPU scan stays at 0.
  const float x0 = row[0];
  out[blockIdx.x] = (x0 != x0 || r.i == 0x7fffffff) ? 0 : r.i;
}

}  // namespace
}  // namespace iehip

using namespace iehip;

extern "C" int ie_hip_argmax_rows(int32_t* out, const float* logits, int R, int n,
                                  hipStream_t stream) {
  clear_error();
  if (R < 0 || n <= 0) return fail(IE_HIP_EINVAL, "argmax_rows: bad sizes");
  if (R == 0) return IE_HIP_OK;
  if (!out || !logits) return fail(IE_HIP_EINVAL, "argmax_rows: null pointer");
  const int vec4 = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 && n % 4 == 0;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(R), dim3(kArgThreads), 0, stream, out, logits, n,
                     vec4);
  return check_launch("argmax_rows");
}
