// CPU oracle for the paged KV-cache path. TEST INFRASTRUCTURE ONLY.
//
// A restatement, in plain C++17 with a C ABI, of the reference engine's CPU
// path for RoPE, the KV append, softmax and attention, plus the paged-cache
// addressing and the 16-bit rounding rules. It is the checker that tests/,
// __graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
// library against. Nothing in the product library links or calls it.
//
// Every function cites the reference file:line it follows (paths relative to
// the reference repository root). Floating-point order is pinned: the file is
// compiled with -ffp-contract=off and the fused multiply-adds that GCC
// -O3 -mavx2 -mfma emits for the reference's expressions are written out as
// explicit fmaf calls, in the same places.
//
// Pinning (what checks each function, all in tests/test_oracle.py):
//   orc_inv_freq, orc_rope_table, orc_rope   bit-exact vs the reference's own
//       ie::rope compiled from its sources (oracle/_ref), position 0 identity,
//       rotation norm preservation.
//   orc_softmax, orc_attention                bit-exact vs the reference's
//       ie::softmax / ie::attention (oracle/_ref); closed forms (one position
//       gives v0, constant keys give the mean of V); fp64 brute force.
//   orc_f32_to_f16 / orc_f16_to_f32           numpy float16 (IEEE RNE) on
//       every float32 exponent band, subnormals, ties and overflow.
//   orc_f32_to_bf16 / orc_bf16_to_f32         torch bfloat16 (RNE) on finite
//       values; known-answer ties; inf/NaN truncation.
//   orc_kv_offset, orc_gather_kv              closed form and page-permutation
//       invariance.
//   orc_rope_append_paged, orc_paged_attention   composition of the above;
//       golden fixtures under tests/golden/ made from oracle/_ref.
//   orc_compare                                numpy restatement of the metric.
//   orc_matmul, orc_quantize_i8, orc_row_to_f32   bit-exact vs the reference's
//       own ie::matmul (scalar kernel) and ie::make_matrix / row_to_f32
//       (oracle/_ref); identity and one-hot matrices; fp64 dot products.
//   orc_rmsnorm, orc_silu_mul                   bit-exact vs ie::rmsnorm /
//       ie::silu (oracle/_ref); closed forms (constant rows, silu(0) = 0).
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// KV element types of a page pool (same codes as include/ie_hip.h).
enum { ORC_KV_F32 = 0, ORC_KV_F16 = 1, ORC_KV_BF16 = 2 };

// inv_freq[i] = 1 / powf(theta, float(2i) / float(head_dim)), i < head_dim/2.
// Reference: src/ops.cpp:37-40.
void orc_inv_freq(float* inv_freq, int head_dim, float theta);

// cos/sin table: table[p * head_dim + i] = cosf(float(p) * inv_freq[i]) and
// table[p * head_dim + half + i] = sinf(...), for p < n_pos, i < half.
// Reference: the angle and the cos/sin calls of src/ops.cpp:42-48.
void orc_rope_table(float* table, int n_pos, int head_dim, float theta);

// In-place RoPE of x [T, n_heads * head_dim], token t at position pos0 + t.
// Reference: src/ops.cpp:34-55 (rotation as GCC contracts it:
// x0' = fma(x0, c, -(x1*s)), x1' = fma(x1, c, x0*s)).
void orc_rope(float* x, int T, int n_heads, int head_dim, int pos0, float theta);

// In-place numerically stable softmax. Reference: src/ops.cpp:57-66.
void orc_softmax(float* x, int n);

// Causal GQA attention over a contiguous cache. Reference: src/ops.cpp:70-108.
// k, v: [pos0 + T, n_kv_heads * head_dim]; q, out: [T, n_heads * head_dim].
// threads <= 1 runs on the calling thread; otherwise heads are split evenly
// over `threads` threads the way src/threadpool.cpp:72-90 splits them.
void orc_attention(float* out, const float* q, const float* k, const float* v, int T, int pos0,
                   int n_heads, int n_kv_heads, int head_dim, int threads);

// Physical cores, counted as distinct (physical id, core id) pairs of
// /proc/cpuinfo. Reference: src/threadpool.cpp:92-130.
int orc_physical_cores(void);

// 16-bit conversions.
//   f16: IEEE binary16, round to nearest even, subnormals kept, overflow to inf
//        (the semantics of __float2half_rn used at src/cuda/kernels.cu:173 and
//        src/cuda/cuda_runner.cu:673-687).
//   bf16: src/matrix.cpp:46-52 (RNE by integer add; inf/NaN truncated).
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
uint16_t orc_f32_to_bf16(float f);
float orc_bf16_to_f32(uint16_t h);
void orc_round_to_kv(void* dst, const float* src, size_t n, int kv_dtype);  // dst in kv_dtype
void orc_widen_kv(float* dst, const void* src, size_t n, int kv_dtype);     // kv_dtype -> fp32

// Element offset of (seq, pos) in a page pool [num_pages * page_size, kv_dim].
// Reference: src/cuda/kernels.cu:183-186, src/cuda/cuda_runner.cu:708-710.
size_t orc_kv_offset(const int32_t* tables, int max_pages, int page_size, int seq, int pos,
                     int kv_dim);

// RoPE + append of T rows into a paged cache. q is rotated in place; row t's
// rotated key and its value are written at (row_seq[t], row_pos[t]) in
// kv_dtype. Reference: rope src/ops.cpp:34-55 applied per row at the row's
// position, the append src/model.cpp:70-75, the paged destination
// src/cuda/kernels.cu:284-306.
void orc_rope_append_paged(float* q, const float* k, const float* v, void* k_pool, void* v_pool,
                           int kv_dtype, int T, const int32_t* row_pos, const int32_t* row_seq,
                           const int32_t* tables, int max_pages, int page_size, int n_heads,
                           int n_kv_heads, int head_dim, float theta);

// Contiguous fp32 copy of positions [0, len) of `seq` from a paged pool
// (16-bit values widened). Reference: src/cuda/cuda_runner.cu:959-964.
void orc_gather_kv(float* dst, const void* pool, int kv_dtype, const int32_t* tables,
                   int max_pages, int page_size, int seq, int len, int kv_dim);

// Paged attention, one row at a time: each row's sequence is gathered into a
// contiguous fp32 copy, then orc_attention(T=1, pos0=row_pos). This is how the
// reference checks its paged kernels: src/cuda/cuda_runner.cu:955-965.
void orc_paged_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                         int kv_dtype, int T, const int32_t* row_pos, const int32_t* row_seq,
                         const int32_t* tables, int max_pages, int page_size, int n_heads,
                         int n_kv_heads, int head_dim, int threads);

// dst[r, :] = src[rows[r], :]. Reference: src/cuda/kernels.cu:778-783.
void orc_gather_rows(float* dst, const float* src, const int32_t* rows, int R, int dim);

// ------------------------------------------------ the decode step's layer ---
// Weight formats of the reference's Matrix (src/matrix.h:4-12): F32, BF16 bits,
// or I8 with one f32 scale per row. Same codes as include/ie_hip.h.
enum { ORC_W_F32 = 0, ORC_W_BF16 = 1, ORC_W_I8 = 2 };

// y[t][o] = (sum_k w[o][k] * x[t][k]) * s[o] + bias[o] (s = scale[o] for I8,
// else 1; bias may be null), the reference's scalar kernel and row loop
// (src/matrix.cpp:131-146,247-265): per token, the products summed in k order
// from 0 (one fma each for BF16 and I8 weights, as GCC compiles those
// instantiations; a multiply and an add for F32), the scale and then the bias
// applied after the sum. x: [T, cols], y: [T, rows]. Rows are split over
// `threads`.
void orc_matmul(float* y, const float* x, const void* w, int w_dtype, const float* scale,
                const float* bias, int T, int rows, int cols, int threads);

// Symmetric per-row int8 quantization, as ie::make_matrix builds an I8 matrix
// (src/matrix.cpp:84-97): s = max|w| / 127 (1 for an all-zero row), q =
// clamp(nearbyint(w / s), -127, 127).
void orc_quantize_i8(int8_t* q, float* scale, const float* w, int rows, int cols);

// One row of a weight matrix widened to f32 (ie::Matrix::row_to_f32,
// src/matrix.cpp:60-67): the embedding lookup of src/model.cpp:53-56.
void orc_row_to_f32(float* out, const void* w, int w_dtype, const float* scale, int cols, int r);

// ie::rmsnorm (src/ops.cpp:23-32): sum of squares in order (a multiply and an
// add each, as compiled there), then y = x * (1 / sqrt(sum / dim + eps)) * weight.
void orc_rmsnorm(float* y, const float* x, const float* weight, int T, int dim, float eps);

// gate[i] = silu(gate[i]) * up[i], silu(x) = x / (1 + exp(-x)) (src/ops.cpp:68,
// src/model.cpp:86).
void orc_silu_mul(float* gate, const float* up, size_t n);

// max|got - want| / max|want| (NaN counts as the worst error).
// Reference: src/npy.cpp:98-110.
double orc_compare(const float* got, const float* want, size_t n, double* max_abs_err,
                   size_t* worst_index);

#ifdef __cplusplus
}
#endif
