/* The decode step around the paged-KV path: a Qwen2 decoder's weights on the
 * device and its work as a KvEngine LayerBody, in C++17 over the C ABI of
 * libie_hip.so. With KvEngine this is the reference's CudaEngine forward
 * (src/cuda/cuda_runner.cu:418-470):
 *   begin               x = E[ids]                               (embedding)
 *   per layer, around the engine's RoPE + paged append + attention:
 *     before_attention  q, k, v = rmsnorm(x) . W^T + b          (one launch)
 *     after_attention   x += attn . Wo^T;
 *                       mid = silu(xn . Wg^T) * (xn . Wu^T), xn = rmsnorm(x)
 *                                                                (one launch);
 *                       x += mid . Wd^T
 *   (each rmsnorm folded into the projection after it: ie_hip_rmsnorm_qkv_proj,
 *   ie_hip_rmsnorm_gate_up_silu)
 *   end                 for the rows that want logits: xg = rmsnorm(x[rows]);
 *                       logits = xg . E_out^T
 * The rows that want logits are gathered before the final norm, which is the
 * same per row as the reference's norm-then-gather (src/cuda/cuda_runner.cu:
 * 461-464) and skips the norm of the other rows of a prompt.
 *
 * Weights arrive as a view of host memory (ModelView): BF16 bits, or INT8 with
 * one f32 scale per row, in the reference's layout (nn.Linear [out, in]); norms
 * and biases f32. One device allocation holds them all; Wq, Wk and Wv are
 * stacked for the one-launch q/k/v projection. Header-only. */
#ifndef IE_HIP_MODEL_HPP_
#define IE_HIP_MODEL_HPP_

#include <cmath>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <vector>

#include "ie_hip_engine.hpp"

namespace ie::hip {

/* The rest of the model shape (the reference's Config, src/config.h:10-26). */
struct ModelShape {
  int hidden = 896;
  int intermediate = 4864;
  int vocab = 151936;
  float rms_eps = 1e-6f;
};

/* A host matrix [rows, cols]: BF16 bits, or INT8 values with a scale per row. */
struct MatrixView {
  const void* data = nullptr;
  const float* scale = nullptr;  // INT8 only
  bool int8 = false;
  int rows = 0, cols = 0;
};

/* One layer's host weights (the reference's LayerWeights, src/weights.h:22-30);
 * a null bias means the model has none. */
struct LayerView {
  const float* input_norm = nullptr;
  const float* post_norm = nullptr;
  MatrixView wq, wk, wv, wo;
  const float *bq = nullptr, *bk = nullptr, *bv = nullptr;
  MatrixView w_gate, w_up, w_down;
};

/* The model's host weights; lm_head.data == nullptr ties the LM head to the
 * embedding (Weights::lm_head_matrix, src/weights.h:38). */
struct ModelView {
  MatrixView embed, lm_head;
  const float* final_norm = nullptr;
  std::vector<LayerView> layers;
};

class DecoderModel {
 public:
  /* Uploads the weights. `rows` and `logit_rows` are the engine's step
   * capacities (EngineLimits after construction: KvEngine::limits()). */
  DecoderModel(const KvConfig& kv, const ModelShape& shape, const ModelView& w, int rows,
               int logit_rows)
      : kv_(kv), shape_(shape), rows_(rows), logit_rows_(logit_rows) {
    const int H = shape.hidden, I = shape.intermediate, QD = kv.q_dim(), KVD = kv.kv_dim();
    if (int(w.layers.size()) != kv.num_layers)
      throw std::runtime_error("DecoderModel: layer count differs from the engine's");
    expect(w.embed, shape.vocab, H, "embedding");
    if (w.lm_head.data) expect(w.lm_head, shape.vocab, H, "lm_head");
    if (!w.final_norm) throw std::runtime_error("DecoderModel: no final norm");
    int8_ = w.embed.int8;

    // Sizing pass, then one allocation, then the copies.
    struct Pending {
      size_t off;
      const void* src;
      size_t bytes;
    };
    std::vector<Pending> copies;
    auto put = [&](const void* src, size_t bytes) {
      const size_t off = arena_.add<unsigned char>(bytes);
      copies.push_back({off, src, bytes});
      return off;
    };
    struct MatOff {
      size_t data = 0, scale = 0;
      bool int8 = false;
      int rows = 0, cols = 0;
    };
    auto put_matrix = [&](const MatrixView& m) {
      MatOff o;
      o.int8 = m.int8;
      o.rows = m.rows;
      o.cols = m.cols;
      o.data = put(m.data, size_t(m.rows) * m.cols * (m.int8 ? 1 : 2));
      if (m.int8) o.scale = put(m.scale, size_t(m.rows) * sizeof(float));
      return o;
    };
    // Wq, Wk, Wv stacked into one region (and their scales, and their biases).
    std::vector<std::vector<float>> zero_bias;
    auto put_stacked = [&](const LayerView& L, MatOff& m, size_t& bias, bool& has_bias) {
      const size_t eb = L.wq.int8 ? 1 : 2;
      m.int8 = L.wq.int8;
      m.rows = QD + 2 * KVD;
      m.cols = H;
      m.data = arena_.add<unsigned char>(size_t(m.rows) * H * eb);
      copies.push_back({m.data, L.wq.data, size_t(QD) * H * eb});
      copies.push_back({m.data + size_t(QD) * H * eb, L.wk.data, size_t(KVD) * H * eb});
      copies.push_back({m.data + size_t(QD + KVD) * H * eb, L.wv.data, size_t(KVD) * H * eb});
      if (m.int8) {
        m.scale = arena_.add<float>(m.rows);
        copies.push_back({m.scale, L.wq.scale, size_t(QD) * 4});
        copies.push_back({m.scale + size_t(QD) * 4, L.wk.scale, size_t(KVD) * 4});
        copies.push_back({m.scale + size_t(QD + KVD) * 4, L.wv.scale, size_t(KVD) * 4});
      }
      has_bias = L.bq || L.bk || L.bv;
      if (has_bias) {
        bias = arena_.add<float>(m.rows);
        const float* parts[3] = {L.bq, L.bk, L.bv};
        const int lens[3] = {QD, KVD, KVD};
        size_t at = bias;
        for (int i = 0; i < 3; ++i) {
          if (!parts[i]) {  // a model with some biases: the missing ones are zero
            zero_bias.emplace_back(lens[i], 0.0f);
            parts[i] = zero_bias.back().data();
          }
          copies.push_back({at, parts[i], size_t(lens[i]) * 4});
          at += size_t(lens[i]) * 4;
        }
      }
    };

    const MatOff embed = put_matrix(w.embed);
    const MatOff head = w.lm_head.data ? put_matrix(w.lm_head) : embed;
    const size_t final_norm = put(w.final_norm, size_t(H) * 4);
    struct LayerOff {
      size_t input_norm, post_norm, bqkv = 0;
      bool has_bias = false;
      MatOff wqkv, wo, w_gate, w_up, w_down;
    };
    std::vector<LayerOff> lo(kv.num_layers);
    for (int l = 0; l < kv.num_layers; ++l) {
      const LayerView& L = w.layers[l];
      expect(L.wq, QD, H, "wq");
      expect(L.wk, KVD, H, "wk");
      expect(L.wv, KVD, H, "wv");
      expect(L.wo, H, QD, "wo");
      expect(L.w_gate, I, H, "w_gate");
      expect(L.w_up, I, H, "w_up");
      expect(L.w_down, H, I, "w_down");
      if (!L.input_norm || !L.post_norm) throw std::runtime_error("DecoderModel: missing norm");
      if (L.wk.int8 != L.wq.int8 || L.wv.int8 != L.wq.int8)
        throw std::runtime_error("DecoderModel: q/k/v weights in different formats");
      lo[l].input_norm = put(L.input_norm, size_t(H) * 4);
      lo[l].post_norm = put(L.post_norm, size_t(H) * 4);
      put_stacked(L, lo[l].wqkv, lo[l].bqkv, lo[l].has_bias);
      lo[l].wo = put_matrix(L.wo);
      lo[l].w_gate = put_matrix(L.w_gate);
      lo[l].w_up = put_matrix(L.w_up);
      lo[l].w_down = put_matrix(L.w_down);
    }
    // The step's activations.
    const size_t o_x = arena_.add<float>(size_t(rows) * H);
    const size_t o_xn = arena_.add<float>(size_t(rows) * H);
    const size_t o_mid = arena_.add<float>(size_t(rows) * I);
    const size_t o_xg = arena_.add<float>(size_t(logit_rows) * H);
    const size_t o_logits = arena_.add<float>(size_t(logit_rows) * shape.vocab);
    const size_t o_tokens = arena_.add<int32_t>(logit_rows);
    arena_.commit("hipMalloc(model weights)");
    for (const Pending& c : copies)
      check(hipMemcpy(arena_.at<unsigned char>(c.off), c.src, c.bytes, hipMemcpyHostToDevice),
            "hipMemcpy(weights)");

    auto mat = [&](const MatOff& o) {
      return ie_matrix{arena_.at<void>(o.data), o.int8 ? arena_.at<float>(o.scale) : nullptr,
                       o.int8 ? 1 : 0, o.rows, o.cols};
    };
    embed_ = mat(embed);
    head_ = mat(head);
    final_norm_ = arena_.at<float>(final_norm);
    for (const LayerOff& o : lo) {
      Layer d;
      d.input_norm = arena_.at<float>(o.input_norm);
      d.post_norm = arena_.at<float>(o.post_norm);
      d.bqkv = o.has_bias ? arena_.at<float>(o.bqkv) : nullptr;
      d.wqkv = mat(o.wqkv);
      d.wo = mat(o.wo);
      d.w_gate = mat(o.w_gate);
      d.w_up = mat(o.w_up);
      d.w_down = mat(o.w_down);
      layers_.push_back(d);
    }
    x_ = arena_.at<float>(o_x);
    xn_ = arena_.at<float>(o_xn);
    mid_ = arena_.at<float>(o_mid);
    xg_ = arena_.at<float>(o_xg);
    logits_ = arena_.at<float>(o_logits);
    tokens_ = arena_.at<int32_t>(o_tokens);
  }
  DecoderModel(const DecoderModel&) = delete;
  DecoderModel& operator=(const DecoderModel&) = delete;

  /* The model's work in the engine's steps (the engine must outlive it). */
  LayerBody body(KvEngine& engine) {
    LayerBody b;
    b.begin = [this, &engine](int rows, hipStream_t s) {
      check_rows(rows);
      embedding(x_, engine.ids(), embed_, rows, s);
    };
    b.before_attention = [this, &engine](int l, int rows, hipStream_t s) {
      const Layer& L = layers_[l];
      rmsnorm_qkv_proj(engine.q(), engine.k(), engine.v(), x_, L.input_norm, shape_.rms_eps,
                       L.wqkv, L.bqkv, rows, kv_.q_dim(), kv_.kv_dim(), s);
    };
    b.after_attention = [this, &engine](int l, int rows, hipStream_t s) {
      const Layer& L = layers_[l];
      matmul(x_, engine.attn(), L.wo, nullptr, rows, true, s);
      rmsnorm_gate_up_silu(mid_, x_, L.post_norm, shape_.rms_eps, L.w_gate, L.w_up, rows, s);
      matmul(x_, mid_, L.w_down, nullptr, rows, true, s);
    };
    b.end = [this, &engine](int rows, int n, hipStream_t s) {
      (void)rows;
      if (n == 0) return;
      gather_rows(xg_, x_, engine.logit_row_ids(), n, shape_.hidden, s);
      rmsnorm(xg_, xg_, final_norm_, n, shape_.hidden, shape_.rms_eps, s);
      matmul(logits_, xg_, head_, nullptr, n, false, s);
    };
    return b;
  }

  /* The greedy token of each of the last step's n logit rows, on `s`. */
  void argmax(int n, hipStream_t s) { argmax_rows(tokens_, logits_, n, shape_.vocab, s); }

  /* The final norm of all `rows` rows into xn() (for a stage report). */
  void final_norm_all(int rows, hipStream_t s) {
    rmsnorm(xn_, x_, final_norm_, rows, shape_.hidden, shape_.rms_eps, s);
  }

  float* x() { return x_; }            // [rows, hidden] residual stream
  float* xn() { return xn_; }          // [rows, hidden] normalised rows
  float* logits() { return logits_; }  // [logit rows, vocab]
  int32_t* tokens() { return tokens_; }  // [logit rows] greedy tokens
  const ModelShape& shape() const { return shape_; }
  bool int8() const { return int8_; }
  size_t device_bytes() const { return arena_.bytes(); }

 private:
  struct Layer {
    const float *input_norm, *post_norm, *bqkv;
    ie_matrix wqkv, wo, w_gate, w_up, w_down;
  };

  static void expect(const MatrixView& m, int rows, int cols, const char* what) {
    if (!m.data || m.rows != rows || m.cols != cols || (m.int8 && !m.scale))
      throw std::runtime_error(std::string("DecoderModel: ") + what + " missing or of the wrong shape");
  }
  void check_rows(int rows) const {
    if (rows < 0 || rows > rows_) throw std::runtime_error("DecoderModel: more rows than the step holds");
  }

  KvConfig kv_;
  ModelShape shape_;
  int rows_, logit_rows_;
  bool int8_ = false;
  DeviceArena arena_;
  ie_matrix embed_{}, head_{};
  const float* final_norm_ = nullptr;
  std::vector<Layer> layers_;
  float *x_ = nullptr, *xn_ = nullptr, *mid_ = nullptr, *xg_ = nullptr, *logits_ = nullptr;
  int32_t* tokens_ = nullptr;
};

}  // namespace ie::hip

#endif  // IE_HIP_MODEL_HPP_
