// Matrix-core (MFMA) building blocks shared by the gfx950 attention kernels:
// 16-bit operand types, the 16x16x32 products in the KV cache's own 16-bit
// type, and an s_waitcnt on the vector-memory counter alone.
#pragma once

#include <hip/hip_runtime.h>

#include "ie_hip.h"

namespace iehip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// D = A[16x32] . B[32x16] + C, float32 accumulation. Operand lane layout:
// lane (g, r) = (lane / 16, lane % 16) holds A[r][8g .. 8g+7] and B[8g .. 8g+7][r];
// the result lane (g, r) holds D[4g .. 4g+3][r].
template <int KV>
struct Mfma;

template <>
struct Mfma<IE_KV_F16> {
  using op = f16x8;
  using elem = _Float16;
  __device__ __forceinline__ static f32x4 mma(op a, op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<IE_KV_BF16> {
  using op = bf16x8;
  using elem = __bf16;
  __device__ __forceinline__ static f32x4 mma(op a, op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

// s_waitcnt with only the vector-memory counter set (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt and lgkmcnt left at their "no wait" maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// LDS byte address of a pointer into an LDS object.
__device__ __forceinline__ unsigned lds_address(const void* p) {
  return static_cast<unsigned>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)(p)));
}

// Global -> LDS DMA of 16 bytes per lane (global_load_lds_dwordx4): lane l's
// 16 bytes at `src` land at LDS byte address `lds` + 16 l (lds uniform, in M0;
// one wait state between the M0 write and the load). Written as inline
// assembly so that the compiler sees no LDS store here: after the builtin form
// it puts a vmcnt(0) before every later LDS read it cannot prove disjoint from
// the DMA (the transposing reads among them), which stalls on every load still
// in flight, prefetches included. Callers wait for completion themselves:
// wait_vmcnt on the issuing wave, then a barrier where other waves read the data.
__device__ __forceinline__ void dma16(const void* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}

// Loads of data read once per launch (the decode kernels' K/V pages), with the
// non-temporal hint. A page walk of config 3's pattern (72 MB of 4 KB pages,
// probe): plain 16-byte loads 16.8 us, non-temporal 15.6; LDS DMA 16.1,
// non-temporal DMA 14.2. The prefill, whose K/V tiles several workgroups
// read, keeps the plain forms.
__device__ __forceinline__ void dma16_nt(const void* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt"
               :
               : "v"(src), "s"(lds)
               : "memory", "m0");
}
template <typename T>
__device__ __forceinline__ T load_nt16(const void* p) {
  static_assert(sizeof(T) == 16, "16-byte loads");
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  return __builtin_bit_cast(T, __builtin_nontemporal_load(static_cast<const u32x4*>(p)));
}

// Max and sum over the 4 lane groups of a 16-column tile (lanes r, r+16, r+32,
// r+48), on gfx950's VALU lane swaps instead of LDS-routed shuffles. With the
// same value in both registers, v_permlane32_swap leaves each lane holding its
// own value and lane^32's (one in each register); v_permlane16_swap likewise
// for lane^16. Written as inline assembly: this toolchain's builtins for these
// two-result instructions return the first register's value for both results.
// One wait state between a VALU write of the operands and the swap (s_nop 1,
// as the compiler itself places before these instructions).
__device__ __forceinline__ void lane_pair32(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void lane_pair16(float x, float& a, float& b) {
  a = x;
  b = x;
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
// Maxima of values that are never NaN (scores from the matrix cores, or -inf
// where masked): v_max_f32 / v_max3_f32 as written. fmaxf first quiets a
// possible signalling NaN in each operand (a v_max_f32 x, x, x apiece), which
// in the softmax loops costs as many instructions as the maxima themselves.
// For non-NaN operands both give the same value.
__device__ __forceinline__ float max_nn(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_nn(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float group_max4(float x) {
  float a, b;
  lane_pair32(x, a, b);
  lane_pair16(max_nn(a, b), a, b);
  return max_nn(a, b);
}
__device__ __forceinline__ float group_sum4(float x) {
  float a, b;
  lane_pair32(x, a, b);
  lane_pair16(a + b, a, b);
  return a + b;
}

// Transposing LDS read (ds_read_b64_tr_b16): in each 16-lane group, lane 4a+b
// receives element b of the 8-byte reads of lanes a, a+4, a+8, a+12.
__device__ __forceinline__ s16x4 lds_read_tr16(const unsigned char* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// Two transposing reads joined into one 8-element operand. Joined as whole
// vectors: element-wise extraction of these results miscompiles (it
// broadcasts element 0) with this toolchain.
template <typename Op>
__device__ __forceinline__ Op join_tr(s16x4 lo, s16x4 hi) {
  return __builtin_bit_cast(Op, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// x = hi + lo in the 16-bit type E, |x - hi - lo| ~ 2^-22 |x|. x - hi is exact in
// float32; written as an fma of the widened hi so that for f16 it becomes one
// mixed-precision v_fma_mix (f32 and f16 sources, f16 result). x is made opaque
// first: otherwise, when x is a product, the compiler may fold the multiply into
// the conversion (v_fma_mixlo_f16 a, b, 0), rounding the exact product once to
// f16 instead of the float32 product to f16 -- one ulp apart in rare cases, and
// chosen differently in different kernels, so two paths over the same data
// would not give the same bits.
template <typename E>
__device__ __forceinline__ void split16(float x, E& hi, E& lo) {
  asm("" : "+v"(x));
  hi = static_cast<E>(x);
  lo = static_cast<E>(__builtin_fmaf(-1.0f, static_cast<float>(hi), x));
}

// Two values split into hi + lo halves at once, for operand slots 2i, 2i+1: the hi
// pair is one packed conversion rounding toward zero (f16: v_cvt_pkrtz), so
// |x - hi| < 1 ulp and |x - hi - lo| ~ 2^-21 |x|; lo = x - hi, rounded to nearest.
template <typename E>
__device__ __forceinline__ void split16x2(float x0, float x1, E& h0, E& h1, E& l0, E& l1);

// f16: lo = x - hi in one mixed-precision fma per value (f16 hi operand, f32 x,
// f16 result into the low or high half), written as inline assembly because
// the compiler converts hi back to f32, subtracts and repacks instead (3 VALU
// per value against 1.5).
template <>
__device__ __forceinline__ void split16x2<_Float16>(float x0, float x1, _Float16& h0,
                                                    _Float16& h1, _Float16& l0, _Float16& l1) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(x0, x1);
  const unsigned hb = __builtin_bit_cast(unsigned, h);
  unsigned lb;
  asm("v_fma_mixlo_f16 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=&v"(lb) : "v"(hb), "v"(x0));
  asm("v_fma_mixhi_f16 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "+v"(lb)
      : "v"(hb), "v"(x1));
  h0 = __builtin_bit_cast(_Float16, static_cast<unsigned short>(hb));
  h1 = __builtin_bit_cast(_Float16, static_cast<unsigned short>(hb >> 16));
  l0 = __builtin_bit_cast(_Float16, static_cast<unsigned short>(lb));
  l1 = __builtin_bit_cast(_Float16, static_cast<unsigned short>(lb >> 16));
}

template <>
__device__ __forceinline__ void split16x2<__bf16>(float x0, float x1, __bf16& h0, __bf16& h1,
                                                  __bf16& l0, __bf16& l1) {
  split16(x0, h0, l0);
  split16(x1, h1, l1);
}

// Two f32 values as one packed f16 pair rounded to nearest even
// (v_cvt_pk_f16_f32 on gfx950): |x - h| <= 2^-11 |x| for normal results, the
// rounding of __floats2half2_rn that the reference's tensor-core prefill
// applies to its weights (src/cuda/kernels.cu:741).
__device__ __forceinline__ void round16x2(float x0, float x1, _Float16& h0, _Float16& h1) {
  typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
  const half2_t h = {static_cast<_Float16>(x0), static_cast<_Float16>(x1)};
  h0 = h.x;
  h1 = h.y;
}

// 2^x for the softmax weights: the bare v_exp_f32 (x is a score minus the row's
// reference max, at most a few units above 0 where the max is raised lazily;
// results below 2^-126, where it may flush to zero, are far below the weights'
// tolerance).
__device__ __forceinline__ float exp2_weight(float x) { return __builtin_amdgcn_exp2f(x); }

}  // namespace iehip
