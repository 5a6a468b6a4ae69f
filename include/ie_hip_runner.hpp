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

}  // namespace ie::hip

#endif  // IE_HIP_RUNNER_HPP_
