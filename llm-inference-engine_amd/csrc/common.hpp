// Shared pieces of the gfx950 paged KV-cache library: error reporting for the
// C ABI, KV element conversions, vector loads/stores of KV rows.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "ie_hip.h"

namespace iehip {

// ---------------------------------------------------------------- errors ---
// Each C entry point returns a status and leaves a message for
// ie_hip_last_error(); messages are per thread.
void set_error(const std::string& msg);
void clear_error();
int fail(int code, const std::string& msg);
// Turns a failed HIP call or launch into IE_HIP_ELAUNCH with a message.
int check_hip(hipError_t err, const char* what);
// Compute units of the current device (256 on MI355X; the fallback when the query fails).
int device_compute_units();
int check_launch(const char* kernel);
// Process-wide operand rounding of the f16 prefill (ie_hip_set_prefill_rounding).
int prefill_rounding();

// -------------------------------------------------------- KV conversions ---
// f16: the hardware conversion (v_cvt_f16_f32: round to nearest even,
// binary16 subnormals kept in the default denormal mode).
// bf16: round to nearest even by integer add, inf/NaN truncated, exactly the
// host rule of the reference (src/matrix.cpp:46-52).
// f is made opaque before the f16 conversion so that the compiler cannot fold
// the fma or multiply that produced it into one mixed-precision v_fma_mix with
// an f16 result: that rounds once where the float32 value rounds twice, and the
// page must hold the float32 value rounded to f16, as the host writes it.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  asm("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, static_cast<_Float16>(f));
}
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t b = __float_as_uint(f);
  if ((b & 0x7F800000u) == 0x7F800000u) return uint16_t(b >> 16);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return uint16_t(b >> 16);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Element type and row I/O per KV dtype. Rows are loaded 8 elements at a time
// (one 16-byte load for 16-bit types, two for f32) and stored 4 at a time.
template <int KV>
struct Kv;

template <>
struct Kv<IE_KV_F32> {
  using elem = float;
  __device__ __forceinline__ static void load8(const elem* p, float* o) {
    const float4 a = reinterpret_cast<const float4*>(p)[0];
    const float4 b = reinterpret_cast<const float4*>(p)[1];
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w;
    o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
  }
  __device__ __forceinline__ static void store4(elem* p, const float* x) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  }
  __device__ __forceinline__ static float load1(const elem* p) { return *p; }
};

template <int KV>
struct Kv16 {
  using elem = uint16_t;
  __device__ __forceinline__ static float widen(uint32_t bits16) {
    return KV == IE_KV_F16 ? f16_bits_to_f32(uint16_t(bits16)) : bf16_bits_to_f32(uint16_t(bits16));
  }
  __device__ __forceinline__ static uint32_t narrow(float f) {
    return KV == IE_KV_F16 ? f32_to_f16_bits(f) : f32_to_bf16_bits(f);
  }
  __device__ __forceinline__ static void load8(const elem* p, float* o) {
    const uint4 u = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[2 * i] = widen(w[i] & 0xFFFFu);
      o[2 * i + 1] = widen(w[i] >> 16);
    }
  }
  __device__ __forceinline__ static void store4(elem* p, const float* x) {
    uint2 u;
    u.x = narrow(x[0]) | (narrow(x[1]) << 16);
    u.y = narrow(x[2]) | (narrow(x[3]) << 16);
    *reinterpret_cast<uint2*>(p) = u;
  }
  __device__ __forceinline__ static float load1(const elem* p) { return widen(*p); }
};

template <>
struct Kv<IE_KV_F16> : Kv16<IE_KV_F16> {};
template <>
struct Kv<IE_KV_BF16> : Kv16<IE_KV_BF16> {};

inline size_t kv_elem_bytes(int kv_dtype) { return kv_dtype == IE_KV_F32 ? 4 : 2; }

// Validates the fields every paged kernel relies on.
int check_layout(const ie_kv_layout& kv, const char* who);

}  // namespace iehip
