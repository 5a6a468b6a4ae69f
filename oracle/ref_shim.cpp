// C-ABI shim over the reference's own CPU path, so Python tests and bench.py
// can call it. TEST INFRASTRUCTURE ONLY. It is compiled together with the
// reference's unmodified src/ops.cpp, src/matrix.cpp and src/threadpool.cpp
// (read in place from the reference checkout, never copied) by oracle/Makefile
// into oracle/_ref/libieref.so. Nothing here restates the reference: each
// function forwards to the reference function it names.
#include <cstdint>
#include <vector>

#include "matrix.h"      // reference: src/matrix.h
#include "ops.h"         // reference: src/ops.h
#include "threadpool.h"  // reference: src/threadpool.h

extern "C" {

// ie::rope, src/ops.cpp:34-55
void ref_rope(float* x, int T, int n_heads, int head_dim, int pos0, float theta) {
  ie::rope(x, T, n_heads, head_dim, pos0, theta);
}

// ie::softmax, src/ops.cpp:57-66
void ref_softmax(float* x, int n) { ie::softmax(x, n); }

// ie::attention, src/ops.cpp:70-108 (runs on the reference's thread pool)
void ref_attention(float* out, const float* q, const float* k, const float* v, int T, int pos0,
                   int n_heads, int n_kv_heads, int head_dim) {
  ie::attention(out, q, k, v, T, pos0, n_heads, n_kv_heads, head_dim);
}

// ie::set_num_threads / thread_pool / physical_cores, src/threadpool.cpp:92-147
void ref_set_num_threads(int n) { ie::set_num_threads(n); }
int ref_num_threads() { return ie::thread_pool().num_threads(); }
int ref_physical_cores() { return ie::physical_cores(); }

// ie::rmsnorm, src/ops.cpp:23-32
void ref_rmsnorm(float* y, const float* x, const float* weight, int T, int dim, float eps) {
  ie::rmsnorm(y, x, weight, T, dim, eps);
}

// ie::silu, src/ops.cpp:68
float ref_silu(float x) { return ie::silu(x); }

// ie::make_matrix_bf16 + ie::matmul (src/matrix.cpp:101-118,284-289) with the
// kernel set by ie::set_kernel (0 scalar, 1 AVX2): weights given as bf16 bits
// and stored as `dtype` (0 F32, 1 BF16, 2 I8, converted by the reference).
// Also returns the stored matrix's per-row scales (I8) in `scale_out` when
// not null.
void ref_matmul_bf16(float* y, const float* x, const uint16_t* w_bits, int dtype,
                     const float* bias, int T, int rows, int cols, int kernel,
                     float* scale_out, int8_t* i8_out) {
  const ie::DType d = dtype == 0 ? ie::DType::F32 : dtype == 1 ? ie::DType::BF16 : ie::DType::I8;
  ie::Matrix m = ie::make_matrix_bf16(
      std::vector<uint16_t>(w_bits, w_bits + size_t(rows) * cols), rows, cols, d);
  ie::set_kernel(kernel ? ie::Kernel::Avx2 : ie::Kernel::Scalar);
  ie::matmul(y, x, m, bias, T);
  if (scale_out && d == ie::DType::I8)
    for (int r = 0; r < rows; ++r) scale_out[r] = m.scale[r];
  if (i8_out && d == ie::DType::I8)
    for (size_t i = 0; i < m.i8.size(); ++i) i8_out[i] = m.i8[i];
}

// A matrix built once by ie::make_matrix_bf16 and then multiplied by
// ie::matmul (AVX2 kernel, the reference's default) as often as a timing loop
// needs: the CPU baseline of the decode step's projections.
void* ref_matrix_create(const uint16_t* w_bits, int dtype, int rows, int cols) {
  const ie::DType d = dtype == 0 ? ie::DType::F32 : dtype == 1 ? ie::DType::BF16 : ie::DType::I8;
  return new ie::Matrix(ie::make_matrix_bf16(
      std::vector<uint16_t>(w_bits, w_bits + size_t(rows) * cols), rows, cols, d));
}
void ref_matrix_destroy(void* m) { delete static_cast<ie::Matrix*>(m); }
void ref_matrix_matmul(float* y, const float* x, const void* m, const float* bias, int T) {
  ie::set_kernel(ie::Kernel::Avx2);
  ie::matmul(y, x, *static_cast<const ie::Matrix*>(m), bias, T);
}

// ie::Matrix::row_to_f32 (src/matrix.cpp:60-67) of a bf16-bits matrix stored as `dtype`.
void ref_row_to_f32(float* out, const uint16_t* w_bits, int dtype, int rows, int cols, int r) {
  const ie::DType d = dtype == 0 ? ie::DType::F32 : dtype == 1 ? ie::DType::BF16 : ie::DType::I8;
  ie::Matrix m = ie::make_matrix_bf16(
      std::vector<uint16_t>(w_bits, w_bits + size_t(rows) * cols), rows, cols, d);
  m.row_to_f32(r, out);
}

}  // extern "C"
