// The reference's Runner and BatchRunner (src/runner.h:19-80) on MI355X:
// ie::hip::make_runner / make_batch_runner, the counterparts of
// cuda::make_runner / make_batch_runner (src/cuda/cuda_runner.h:20-27,
// src/cuda/cuda_runner.cu:606-622).
//
// HipEngine is a thin adapter: the paged KV cache, the page pool and the step
// machinery are KvEngine (include/ie_hip_engine.hpp), the weights and the
// per-layer dense work DecoderModel (include/ie_hip_model.hpp). What it adds is
// the interface's semantics:
//   - Runner: one sequence (slot 0, opened on first use); forward() appends
//     `ids` and returns the last row's logits, or every row's;
//   - BatchRunner: prefill one sequence, decode one token for each of several,
//     logits or (greedy) the device argmax of each row;
//   - prompts longer than a step holds run as consecutive steps of one
//     sequence (each attends to what the earlier ones appended);
//   - a one-row prefill and every decode step replay the batch size's graph.
// Built against the reference's headers in place (-I <reference>/src) and
// linked into its engine with libie_hip.so; it calls the reference's
// Weights::matrix_bytes() and num_params() (src/weights.cpp).
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>
#include <vector>

#include "ie_hip_model.hpp"
#include "ie_hip_runner.hpp"

namespace ie::hip {
namespace {

KvConfig kv_config(const Config& c) {
  KvConfig k;
  k.num_layers = c.num_layers;
  k.num_heads = c.num_heads;
  k.num_kv_heads = c.num_kv_heads;
  k.head_dim = c.head_dim;
  k.rope_theta = c.rope_theta;
  return k;
}

ModelShape model_shape(const Config& c) {
  ModelShape s;
  s.hidden = c.hidden_size;
  s.intermediate = c.intermediate_size;
  s.vocab = c.vocab_size;
  s.rms_eps = c.rms_norm_eps;
  return s;
}

MatrixView matrix_view(const Matrix& m) {
  MatrixView v;
  v.rows = m.rows;
  v.cols = m.cols;
  if (m.dtype == DType::BF16) {
    v.data = m.bf16.data();
  } else if (m.dtype == DType::I8) {
    v.data = m.i8.data();
    v.scale = m.scale.data();
    v.int8 = true;
  } else {
    throw std::runtime_error("the HIP backend runs bf16 or int8 weights (not f32)");
  }
  return v;
}

const float* optional(const std::vector<float>& v) { return v.empty() ? nullptr : v.data(); }

ModelView model_view(const Weights& w) {
  ModelView m;
  m.embed = matrix_view(w.embed);
  if (w.lm_head.rows) m.lm_head = matrix_view(w.lm_head);
  m.final_norm = w.final_norm.data();
  for (const LayerWeights& L : w.layers) {
    LayerView l;
    l.input_norm = L.input_norm.data();
    l.post_norm = L.post_attn_norm.data();
    l.wq = matrix_view(L.wq);
    l.wk = matrix_view(L.wk);
    l.wv = matrix_view(L.wv);
    l.wo = matrix_view(L.wo);
    l.bq = optional(L.bq);
    l.bk = optional(L.bk);
    l.bv = optional(L.bv);
    l.w_gate = matrix_view(L.w_gate);
    l.w_up = matrix_view(L.w_up);
    l.w_down = matrix_view(L.w_down);
    m.layers.push_back(l);
  }
  return m;
}

EngineLimits limits_for(int max_batch, int max_seq_len, int num_pages, int logit_rows) {
  EngineLimits lim;
  lim.max_batch = max_batch;
  lim.max_seq_len = max_seq_len;
  lim.num_pages = num_pages;
  lim.logit_rows = logit_rows;  // 0: the engine's default, max(max_batch, 16)
  return lim;
}

// Logit rows one step of a single-sequence Runner holds: every row of a
// forward(all_logits) of up to max_tokens tokens in one step where 128 MiB of
// logits (on the device, and again in pinned host memory) allow it -- 220 rows
// at Qwen2.5's 151,936-token vocabulary -- so a perplexity-style forward runs
// in steps of that many rows, not 16.
constexpr size_t kLogitBudget = size_t(128) << 20;
int runner_logit_rows(const Config& cfg, int max_tokens) {
  const size_t row_bytes = size_t(std::max(cfg.vocab_size, 1)) * sizeof(float);
  const int budget = int(std::max<size_t>(kLogitBudget / row_bytes, 16));
  return std::min(std::max(max_tokens, 1), budget);
}

const Config& checked(const Config& cfg, const Weights& w) {
  if (w.dtype != DType::BF16 && w.dtype != DType::I8)
    throw std::runtime_error("the HIP backend runs bf16 or int8 weights (not f32)");
  if (int(w.layers.size()) != cfg.num_layers)
    throw std::runtime_error("weights: layer count differs from the config");
  return cfg;
}

class HipEngine final : public Runner, public BatchRunner {
 public:
  HipEngine(const Config& cfg, const Weights& w, int max_batch, int max_seq_len, int num_pages,
            bool use_graphs, int kv_dtype, int logit_rows = 0)
      : cfg_(checked(cfg, w)), dtype_(w.dtype), weight_bytes_(w.matrix_bytes()),
        num_params_(w.num_params()),
        kv_(kv_config(cfg), limits_for(max_batch, max_seq_len, num_pages, logit_rows), kv_dtype,
            use_graphs),
        model_(kv_config(cfg), model_shape(cfg), model_view(w), kv_.limits().step_rows,
               kv_.limits().logit_rows) {
    kv_.set_body(model_.body(kv_));
    const size_t R = size_t(kv_.limits().logit_rows);
    host_logits_.allocate(R * cfg_.vocab_size * sizeof(float), "hipHostMalloc(logits)");
    host_tokens_.allocate(R * sizeof(int32_t), "hipHostMalloc(tokens)");
  }

  // ---------------------------------------------------------- Runner ----

  std::vector<float> forward(const std::vector<int32_t>& ids, bool all_logits,
                             const StageCallback& on_stage) override {
    if (!kv_.is_open(0) && kv_.open_sequence() != 0)
      throw std::runtime_error("forward: sequence slot 0 is taken");
    const int T = int(ids.size());
    if (T == 0) throw std::runtime_error("forward: no tokens");
    check_ids(ids);
    const int start = kv_.sequence_length(0), V = cfg_.vocab_size, H = cfg_.hidden_size;
    // Stages are gathered over the steps and reported once, [T, cols] each.
    std::vector<std::vector<float>> stages;
    if (on_stage) stages.assign(size_t(cfg_.num_layers) + 2, std::vector<float>(size_t(T) * H));
    std::vector<float> out;
    const int per_step = all_logits ? kv_.limits().logit_rows : kv_.limits().step_rows;
    for (int t0 = 0; t0 < T; t0 += per_step) {
      const int n = std::min(per_step, T - t0);
      const bool last = t0 + n == T;
      std::vector<int> seq(n, 0), pos(n), logit_rows;
      for (int i = 0; i < n; ++i) pos[i] = start + t0 + i;
      if (all_logits) {
        for (int i = 0; i < n; ++i) logit_rows.push_back(i);
      } else if (last) {
        logit_rows.push_back(n - 1);
      }
      const std::vector<int32_t> part(ids.begin() + t0, ids.begin() + t0 + n);
      std::function<void(int)> after_layer;
      if (on_stage) {
        after_layer = [&, t0, n](int layer) {  // layer -1: after the embedding
          pull(stages[size_t(layer + 1)].data() + size_t(t0) * H, model_.x(), size_t(n) * H);
        };
      }
      kv_.run(seq, pos, part, logit_rows, /*decode=*/T == 1 && !all_logits && !on_stage,
              after_layer);
      if (on_stage) {
        model_.final_norm_all(n, kv_.stream());
        pull(stages.back().data() + size_t(t0) * H, model_.xn(), size_t(n) * H);
      }
      if (!logit_rows.empty()) {
        const size_t m = logit_rows.size() * size_t(V);
        queue_logits(int(logit_rows.size()));
        kv_.sync();
        out.insert(out.end(), host_logits_.as<float>(), host_logits_.as<float>() + m);
      } else {
        kv_.sync();
      }
    }
    if (on_stage) {
      on_stage("embed", stages[0].data(), T, H);
      for (int l = 0; l < cfg_.num_layers; ++l) {
        char name[32];
        std::snprintf(name, sizeof(name), "layer_%02d", l);
        on_stage(name, stages[size_t(l) + 1].data(), T, H);
      }
      on_stage("final_norm", stages.back().data(), T, H);
      on_stage("logits", out.data(), int(out.size() / size_t(V)), V);
    }
    return out;
  }
  void reset() override {
    if (kv_.is_open(0)) kv_.close_sequence(0);
  }
  int position() const override { return kv_.sequence_length(0); }
  int max_tokens() const override { return kv_.max_seq_len(); }

  // ----------------------------------------------------- BatchRunner ----

  int open_sequence() override { return kv_.open_sequence(); }
  void close_sequence(int seq) override { kv_.close_sequence(seq); }
  int sequence_length(int seq) const override { return kv_.sequence_length(seq); }

  std::vector<float> prefill(int seq, const std::vector<int32_t>& ids) override {
    run_prefill(seq, ids);
    return logits_of(1);
  }
  int32_t prefill_greedy(int seq, const std::vector<int32_t>& ids) override {
    run_prefill(seq, ids);
    return tokens_of(1).at(0);
  }
  std::vector<float> decode(const std::vector<int>& seqs,
                            const std::vector<int32_t>& tokens) override {
    run_decode(seqs, tokens);
    return logits_of(int(seqs.size()));
  }
  std::vector<int32_t> decode_greedy(const std::vector<int>& seqs,
                                     const std::vector<int32_t>& tokens) override {
    run_decode(seqs, tokens);
    return tokens_of(int(seqs.size()));
  }

  int max_batch() const override { return kv_.max_batch(); }
  int max_seq_len() const override { return kv_.max_seq_len(); }
  int page_size() const override { return kv_.page_size(); }
  int total_pages() const override { return kv_.total_pages(); }
  int free_pages() const override { return kv_.free_pages(); }

  // ------------------------------------------------------------ both ----

  const Config& config() const override { return cfg_; }
  std::string device_name() const override { return kv_.device_name(); }
  DType weight_dtype() const override { return dtype_; }
  size_t weight_bytes() const override { return weight_bytes_; }
  size_t num_params() const override { return num_params_; }
  size_t kv_cache_bytes() const override { return kv_.kv_cache_bytes(); }

 private:
  void check_ids(const std::vector<int32_t>& ids) const {
    for (int32_t id : ids)
      if (id < 0 || id >= cfg_.vocab_size) throw std::runtime_error("token id out of range");
  }
  int open_length(int seq) const {
    if (seq < 0 || seq >= kv_.max_batch() || !kv_.is_open(seq))
      throw std::runtime_error("invalid or closed sequence id " + std::to_string(seq));
    return kv_.sequence_length(seq);
  }

  /* The prompt in steps of at most step_rows rows; logits of its last row. */
  void run_prefill(int seq, const std::vector<int32_t>& ids) {
    const int T = int(ids.size());
    if (T == 0) throw std::runtime_error("forward: no tokens");
    check_ids(ids);
    const int start = open_length(seq), per_step = kv_.limits().step_rows;
    for (int t0 = 0; t0 < T; t0 += per_step) {
      const int n = std::min(per_step, T - t0);
      std::vector<int> rs(n, seq), rp(n), logit_rows;
      for (int i = 0; i < n; ++i) rp[i] = start + t0 + i;
      if (t0 + n == T) logit_rows.push_back(n - 1);
      kv_.run(rs, rp, std::vector<int32_t>(ids.begin() + t0, ids.begin() + t0 + n), logit_rows,
              /*decode=*/T == 1);
      if (t0 + n < T) kv_.sync();
    }
  }

  void run_decode(const std::vector<int>& seqs, const std::vector<int32_t>& tokens) {
    const int n = int(seqs.size());
    if (n != int(tokens.size())) throw std::runtime_error("decode: one token per sequence");
    if (n > kv_.max_batch()) throw std::runtime_error("decode: more sequences than max_batch");
    check_ids(tokens);
    std::vector<int> rp(n), logit_rows(n);
    for (int i = 0; i < n; ++i) {
      rp[i] = open_length(seqs[i]);
      logit_rows[i] = i;
    }
    kv_.run(seqs, rp, tokens, logit_rows, /*decode=*/true);
  }

  void queue_logits(int R) {
    check(hipMemcpyAsync(host_logits_.as<float>(), model_.logits(),
                         size_t(R) * cfg_.vocab_size * sizeof(float), hipMemcpyDeviceToHost,
                         kv_.stream()),
          "logits");
  }
  std::vector<float> logits_of(int R) {
    queue_logits(R);
    kv_.sync();
    const float* p = host_logits_.as<float>();
    return std::vector<float>(p, p + size_t(R) * cfg_.vocab_size);
  }
  std::vector<int32_t> tokens_of(int R) {
    model_.argmax(R, kv_.stream());
    check(hipMemcpyAsync(host_tokens_.as<int32_t>(), model_.tokens(), size_t(R) * sizeof(int32_t),
                         hipMemcpyDeviceToHost, kv_.stream()),
          "argmax");
    kv_.sync();
    const int32_t* p = host_tokens_.as<int32_t>();
    return std::vector<int32_t>(p, p + R);
  }
  void pull(float* dst, const float* src, size_t n) {
    check(hipMemcpyAsync(dst, src, n * sizeof(float), hipMemcpyDeviceToHost, kv_.stream()),
          "stage copy");
    kv_.sync();
  }

  Config cfg_;
  DType dtype_;
  size_t weight_bytes_, num_params_;
  KvEngine kv_;
  DecoderModel model_;
  PinnedBlock host_logits_, host_tokens_;
};

}  // namespace

void set_tensor_cores(bool on) { ie_hip_set_attention_impl(on ? IE_HIP_IMPL_AUTO : IE_HIP_IMPL_VALU); }

void set_tc_fp16(bool on) {
  ie_hip_set_prefill_rounding(on ? IE_HIP_PREFILL_SINGLE : IE_HIP_PREFILL_SPLIT);
}

void set_cublas(bool on) {
  if (on)
    throw std::runtime_error(
        "--cublas: there is no cuBLAS comparison path on MI355X; the dense products run on this "
        "engine's own matrix-core kernels");
}

bool device_available() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return n > 0;
}

std::string device_description() {
  int dev = 0;
  hipDeviceProp_t prop{};
  if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess) {
    (void)hipGetLastError();
    return "no HIP device";
  }
  return std::string(prop.name[0] ? prop.name : "AMD GPU") + " (" + prop.gcnArchName + ")";
}

std::unique_ptr<Runner> make_runner(const Config& cfg, const Weights& w, int max_tokens,
                                    bool use_graphs, KvDtype kv) {
  if (max_tokens < 1) throw std::runtime_error("KV cache: max_tokens must be positive");
  return std::make_unique<HipEngine>(cfg, w, /*max_batch=*/1, max_tokens, ie_pages_for(max_tokens),
                                     use_graphs, int(kv), runner_logit_rows(cfg, max_tokens));
}

std::unique_ptr<Runner> make_runner(const Config& cfg, const Weights& w, int max_tokens,
                                    bool use_graphs, bool kv_f16) {
  return make_runner(cfg, w, max_tokens, use_graphs, kv_f16 ? KvDtype::F16 : KvDtype::F32);
}

std::unique_ptr<BatchRunner> make_batch_runner(const Config& cfg, const Weights& w, int max_batch,
                                               int max_seq_len, size_t kv_bytes, bool use_graphs,
                                               KvDtype kv) {
  if (max_batch < 1 || max_seq_len < 1)
    throw std::runtime_error("KV cache: max_batch and max_seq_len must be positive");
  const int pages =
      KvEngine::pages_for_budget(kv_config(cfg), max_batch, max_seq_len, kv_bytes, int(kv));
  return std::make_unique<HipEngine>(cfg, w, max_batch, max_seq_len, pages, use_graphs, int(kv));
}

std::unique_ptr<BatchRunner> make_batch_runner(const Config& cfg, const Weights& w, int max_batch,
                                               int max_seq_len, size_t kv_bytes, bool use_graphs,
                                               bool kv_f16) {
  return make_batch_runner(cfg, w, max_batch, max_seq_len, kv_bytes, use_graphs,
                           kv_f16 ? KvDtype::F16 : KvDtype::F32);
}

}  // namespace ie::hip
