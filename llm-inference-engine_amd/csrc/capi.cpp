// C-ABI plumbing shared by every entry point: per-thread error messages,
// version string, the process-wide kernel switches, ROCTX trace ranges, layout
// validation and the host RoPE table.
#include <rocprofiler-sdk-roctx/roctx.h>

#include <cmath>
#include <string>
#include <vector>

#include "common.hpp"
#include "decode.hpp"

namespace iehip {

namespace {
thread_local std::string g_last_error;
}

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const std::string& msg) {
  set_error(msg);
  return code;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return IE_HIP_OK;
  return fail(IE_HIP_ELAUNCH, std::string("HIP error in ") + what + ": " + hipGetErrorString(err));
}

int check_launch(const char* kernel) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return IE_HIP_OK;
  return fail(IE_HIP_ELAUNCH,
              std::string("HIP kernel ") + kernel + " failed to launch: " + hipGetErrorString(err));
}

namespace {
int g_attention_impl = IE_HIP_IMPL_AUTO;
int g_prefill_rounding = IE_HIP_PREFILL_SINGLE;
}

int attention_impl() { return g_attention_impl; }
int prefill_rounding() { return g_prefill_rounding; }

int check_layout(const ie_kv_layout& kv, const char* who) {
  if (kv.page_size != IE_HIP_PAGE_SIZE)
    return fail(IE_HIP_EINVAL, std::string(who) + ": KV page size must be 16");
  if (kv.kv_dtype != IE_KV_F32 && kv.kv_dtype != IE_KV_F16 && kv.kv_dtype != IE_KV_BF16)
    return fail(IE_HIP_EINVAL, std::string(who) + ": unknown kv_dtype " + std::to_string(kv.kv_dtype));
  if (!kv.tables || kv.max_pages <= 0 || kv.num_pages <= 0)
    return fail(IE_HIP_EINVAL, std::string(who) + ": empty page table or pool");
  return IE_HIP_OK;
}

}  // namespace iehip

using namespace iehip;

extern "C" {

const char* ie_hip_last_error(void) { return g_last_error.c_str(); }

const char* ie_hip_version(void) { return "ie_hip 0.1 (gfx950, wave64)"; }

int ie_hip_set_attention_impl(int impl) {
  const int prev = g_attention_impl;
  if (impl == IE_HIP_IMPL_AUTO || impl == IE_HIP_IMPL_VALU || impl == IE_HIP_IMPL_MFMA)
    g_attention_impl = impl;
  return prev;
}

int ie_hip_set_prefill_rounding(int mode) {
  const int prev = g_prefill_rounding;
  if (mode == IE_HIP_PREFILL_SINGLE || mode == IE_HIP_PREFILL_SPLIT) g_prefill_rounding = mode;
  return prev;
}

void ie_hip_range_push(const char* name) {
  if (name) roctxRangePushA(name);
}

void ie_hip_range_pop(void) { roctxRangePop(); }

// The angle and cos/sin of src/ops.cpp:37-48, evaluated with the host libm so
// the table equals what the reference CPU rope computes for every position.
int ie_hip_rope_table(float* table, int n_pos, int head_dim, float theta) {
  clear_error();
  if (!table || n_pos <= 0 || head_dim <= 0 || head_dim % 2)
    return fail(IE_HIP_EINVAL, "ie_hip_rope_table: bad arguments");
  const int half = head_dim / 2;
  std::vector<float> inv_freq(half);
  for (int i = 0; i < half; ++i)
    inv_freq[i] = 1.0f / powf(theta, float(2 * i) / float(head_dim));
  for (int p = 0; p < n_pos; ++p) {
    const float pos = float(p);
    float* row = table + size_t(p) * head_dim;
    for (int i = 0; i < half; ++i) {
      const float angle = pos * inv_freq[i];
      row[i] = cosf(angle);
      row[half + i] = sinf(angle);
    }
  }
  return IE_HIP_OK;
}

}  // extern "C"
