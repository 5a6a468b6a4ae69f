/* The MI355X engine behind the reference's Runner / BatchRunner interface.
 *
 * This header takes the place of src/cuda/cuda_runner.h for a build of the
 * reference engine that runs on gfx950: the same factories, in namespace
 * ie::hip, returning the reference's own interfaces (src/runner.h:19-80), which
 * this header includes from the reference's source tree ("runner.h" on the
 * include path; it is not copied here). The implementation is
 * llm-inference-engine_amd/runner/hip_runner.cpp over include/ie_hip_model.hpp
 * and include/ie_hip_engine.hpp, linked with libie_hip.so.
 *
 * The KV cache's element type is a KvDtype (f32, f16 or bf16); the overloads
 * taking the reference's `bool kv_f16` map it to F16 / F32. */
#ifndef IE_HIP_RUNNER_HPP_
#define IE_HIP_RUNNER_HPP_

#include <cstddef>
#include <memory>
#include <string>

#include "runner.h"

namespace ie::hip {

enum class KvDtype { F32 = 0, F16 = 1, BF16 = 2 };

/* True if a HIP device is present (cuda::device_available,
 * src/cuda/cuda_runner.h:12-13). */
bool device_available();
/* The device's name and architecture ("AMD Instinct MI355X (gfx950:...)"). */
std::string device_description();

/* One sequence of up to max_tokens tokens (cuda::make_runner,
 * src/cuda/cuda_runner.h:20-21). `w` holds BF16 or INT8 matrices and may be
 * freed afterwards. use_graphs: each decode step is recorded once per batch
 * size as a HIP graph and replayed. */
std::unique_ptr<Runner> make_runner(const Config& cfg, const Weights& w, int max_tokens,
                                    bool use_graphs, KvDtype kv);
std::unique_ptr<Runner> make_runner(const Config& cfg, const Weights& w, int max_tokens,
                                    bool use_graphs = true, bool kv_f16 = false);

/* Up to max_batch sequences of up to max_seq_len tokens sharing a page pool of
 * about kv_bytes bytes (cuda::make_batch_runner, src/cuda/cuda_runner.h:25-27). */
std::unique_ptr<BatchRunner> make_batch_runner(const Config& cfg, const Weights& w, int max_batch,
                                               int max_seq_len, size_t kv_bytes, bool use_graphs,
                                               KvDtype kv);
std::unique_ptr<BatchRunner> make_batch_runner(const Config& cfg, const Weights& w, int max_batch,
                                               int max_seq_len, size_t kv_bytes,
                                               bool use_graphs = true, bool kv_f16 = false);

/* The kernel switches the reference's command line sets (src/main.cpp:272-287).
 * Process-wide; set them before a runner steps.
 *
 * set_tensor_cores (cuda::set_tensor_cores, src/cuda/cuda_runner.h:29-30): on
 * (the default), attention runs on the matrix-core kernels; off, on the
 * float32 VALU kernels, for comparison. The dense products keep their matrix-
 * core kernels either way: their reduction order depends on the matrix shape
 * alone, so a batch gives each row the bits it gets alone and the switch's
 * purpose in the reference -- a bit-exact --check at 32 rows and more -- needs
 * no second kernel here. */
void set_tensor_cores(bool on);
/* set_tc_fp16 (cuda::set_tc_fp16, src/cuda/cuda_runner.h:31-32): on, the
 * prefill on f16 caches takes q and P as single f16 values (the reference's
 * FP16 tensor-core prompt kernel); off, it splits them into hi + lo halves
 * (float32-level). bf16 caches always split. The library's own default is on
 * (ie_hip_set_prefill_rounding); the reference's command line passes its
 * --tc-fp16 flag, off unless given. */
void set_tc_fp16(bool on);
/* set_cublas (cuda::set_cublas, src/cuda/cuda_runner.h:33-34): the reference's
 * comparison path through NVIDIA's cuBLAS has no counterpart on MI355X; every
 * dense product runs on this library's kernels. Off is accepted; on throws
 * std::runtime_error saying so. */
void set_cublas(bool on);

/* Every kernel family of libie_hip.so against the host program's CPU
 * operations (ie::rope, ie::attention, ie::rmsnorm, ie::matmul) on random
 * data, at the path's bars; prints a line per check and returns the number of
 * failures (cuda::run_selftest, src/cuda/cuda_runner.h:36-37). */
int run_selftest();
/* Device properties, a copy checked against the host, and device-to-device
 * bandwidth against the nominal 8 TB/s; 0 on success (cuda::run_device_check,
 * src/cuda/device_check.h:7). */
int run_device_check();

}  // namespace ie::hip

#endif  // IE_HIP_RUNNER_HPP_
