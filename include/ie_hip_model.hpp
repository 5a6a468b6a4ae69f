/* The decode step around the paged-KV path: a Qwen2 decoder's weights on the
 * device and its per-layer work as a KvEngine LayerBody, in C++17 over the C
 * ABI of libie_hip.so. Together with KvEngine this is the reference's
 * CudaEngine forward (src/cuda/cuda_runner.cu:418-470):
 *   embed(ids)              x = E[ids]                 (embedding)
 *   per layer, around the engine's RoPE + paged append + attention:
 *     before_attention      xn = rmsnorm(x); q, k, v = xn . W^T + b (one launch)
 *     after_attention       x += attn . Wo^T; xn = rmsnorm(x);
 *                           mid = silu(xn . Wg^T) * (xn . Wu^T); x += mid . Wd^T
 *   logits(rows)            xn = rmsnorm(x); logits = xn[rows] . E_out^T
 * Weights are BF16 bits in the reference's layout (nn.Linear [out, in]),
 * stored on the device as BF16 or quantized to INT8; the norms and biases f32. All work is enqueued on the engine's stream, so a
 * decode step's layers are recorded into the engine's graphs with its
 * attention. Header-only. */
#ifndef IE_HIP_MODEL_HPP_
#define IE_HIP_MODEL_HPP_

#include <algorithm>
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

/* One layer's weights on the host (src/weights.h LayerWeights). */
struct HostLayer {
  std::vector<float> input_norm, post_norm;       // [hidden]
  std::vector<uint16_t> wq, wk, wv, wo;           // [q_dim, hidden], [kv_dim, hidden] x2, [hidden, q_dim]
  std::vector<float> bq, bk, bv;                  // [q_dim], [kv_dim] x2
  std::vector<uint16_t> w_gate, w_up, w_down;     // [inter, hidden] x2, [hidden, inter]
};

/* The model's weights on the host; the LM head is the embedding (tied, as
 * Qwen2.5-0.5B's, src/weights.cpp lm_head_matrix). */
struct HostModel {
  std::vector<uint16_t> embed;    // [vocab, hidden]
  std::vector<float> final_norm;  // [hidden]
  std::vector<HostLayer> layers;
};

class DecoderModel {
 public:
  /* Uploads the weights; `max_rows` bounds a step's rows (as the engine's
   * max batch bounds a decode step, and the largest prompt chunk a prefill).
   * int8: every matrix, the embedding included, stored as INT8 with one scale
   * per row, quantized as the reference's --dtype int8 does
   * (src/weights.cpp:95-114, src/matrix.cpp:84-97). */
  DecoderModel(const KvConfig& kv, const ModelShape& shape, const HostModel& host, int max_rows,
               bool int8 = false)
      : kv_(kv), shape_(shape), max_rows_(max_rows), int8_(int8) {
    const int H = shape.hidden, I = shape.intermediate, QD = kv.q_dim(), KVD = kv.kv_dim();
    if (int(host.layers.size()) != kv.num_layers)
      throw std::runtime_error("DecoderModel: layer count differs from the engine's");
    if (host.embed.size() != size_t(shape.vocab) * H || host.final_norm.size() != size_t(H))
      throw std::runtime_error("DecoderModel: embedding or final norm of the wrong size");
    embed_ = upload_matrix(host.embed, shape.vocab, H);
    final_norm_ = upload(host.final_norm, H);
    for (const HostLayer& h : host.layers) {
      Layer l;
      l.input_norm = upload(h.input_norm, H);
      l.post_norm = upload(h.post_norm, H);
      if (h.wq.size() != size_t(QD) * H || h.wk.size() != size_t(KVD) * H ||
          h.wv.size() != size_t(KVD) * H || h.bq.size() != size_t(QD) ||
          h.bk.size() != size_t(KVD) || h.bv.size() != size_t(KVD))
        throw std::runtime_error("DecoderModel: q/k/v weight of the wrong size");
      // Wq, Wk, Wv stacked (and their biases), for one q/k/v launch.
      std::vector<uint16_t> wqkv(h.wq);
      wqkv.insert(wqkv.end(), h.wk.begin(), h.wk.end());
      wqkv.insert(wqkv.end(), h.wv.begin(), h.wv.end());
      std::vector<float> bqkv(h.bq);
      bqkv.insert(bqkv.end(), h.bk.begin(), h.bk.end());
      bqkv.insert(bqkv.end(), h.bv.begin(), h.bv.end());
      l.wqkv = upload_matrix(wqkv, QD + 2 * KVD, H);
      l.bqkv = upload(bqkv, bqkv.size());
      l.wo = upload_matrix(h.wo, H, QD);
      l.w_gate = upload_matrix(h.w_gate, I, H);
      l.w_up = upload_matrix(h.w_up, I, H);
      l.w_down = upload_matrix(h.w_down, H, I);
      layers_.push_back(l);
    }
    x_ = mem_.alloc<float>(size_t(max_rows) * H);
    xn_ = mem_.alloc<float>(size_t(max_rows) * H);
    mid_ = mem_.alloc<float>(size_t(max_rows) * I);
    ids_ = mem_.alloc<int32_t>(max_rows);
    ids_host_.resize(max_rows);
  }
  DecoderModel(const DecoderModel&) = delete;
  DecoderModel& operator=(const DecoderModel&) = delete;

  /* The per-layer work around the engine's attention (cuda_runner.cu:433-452),
   * for KvEngine::set_body. The engine must outlive the returned body. */
  LayerBody body(KvEngine& engine) {
    LayerBody b;
    b.before_attention = [this, &engine](int l, int rows, hipStream_t s) {
      check_rows(rows);
      const Layer& L = layers_.at(l);
      rmsnorm(xn_, x_, L.input_norm, rows, shape_.hidden, shape_.rms_eps, s);
      qkv_proj(engine.q(), engine.k(), engine.v(), xn_, L.wqkv, L.bqkv, rows, kv_.q_dim(),
               kv_.kv_dim(), s);
    };
    b.after_attention = [this, &engine](int l, int rows, hipStream_t s) {
      const Layer& L = layers_.at(l);
      matmul(x_, engine.attn(), L.wo, nullptr, rows, true, s);
      rmsnorm(xn_, x_, L.post_norm, rows, shape_.hidden, shape_.rms_eps, s);
      gate_up_silu(mid_, xn_, L.w_gate, L.w_up, rows, s);
      matmul(x_, mid_, L.w_down, nullptr, rows, true, s);
    };
    return b;
  }

  /* x = E[ids] for a step's rows, in row order (embedding, cuda_runner.cu:427). */
  void embed(const std::vector<int32_t>& ids, hipStream_t s) {
    check_rows(int(ids.size()));
    for (size_t i = 0; i < ids.size(); ++i) {
      if (ids[i] < 0 || ids[i] >= shape_.vocab) throw std::runtime_error("token id out of range");
      ids_host_.data()[i] = ids[i];
    }
    check(hipMemcpyAsync(ids_, ids_host_.data(), ids.size() * sizeof(int32_t),
                         hipMemcpyHostToDevice, s),
          "hipMemcpyAsync(ids)");
    ie::hip::embedding(x_, ids_, embed_, int(ids.size()), s);
  }

  /* Final norm of all `rows`, then logits [n, vocab] of rows [rows - n, rows)
   * (src/model.cpp:96-107: only the rows that need logits pass the LM head). */
  void logits(float* out, int rows, int n, hipStream_t s) {
    check_rows(rows);
    if (n < 0 || n > rows) throw std::runtime_error("logits: bad row count");
    rmsnorm(xn_, x_, final_norm_, rows, shape_.hidden, shape_.rms_eps, s);
    matmul(out, xn_ + size_t(rows - n) * shape_.hidden, embed_, nullptr, n, false, s);
  }

  float* x() { return x_; }    // [max_rows, hidden] residual stream
  float* xn() { return xn_; }  // [max_rows, hidden] normalised copy (after logits: the final norm)
  int max_rows() const { return max_rows_; }

 private:
  struct Layer {
    const float *input_norm, *post_norm, *bqkv;
    ie_matrix wqkv, wo, w_gate, w_up, w_down;
  };

  void check_rows(int rows) const {
    if (rows < 0 || rows > max_rows_) throw std::runtime_error("DecoderModel: more rows than max_rows");
  }
  const float* upload(const std::vector<float>& v, size_t n) {
    if (v.size() != n) throw std::runtime_error("DecoderModel: weight of the wrong size");
    float* d = mem_.alloc<float>(n);
    check(hipMemcpy(d, v.data(), n * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy(weights)");
    return d;
  }
  ie_matrix upload_matrix(const std::vector<uint16_t>& w, int rows, int cols) {
    if (w.size() != size_t(rows) * cols) throw std::runtime_error("DecoderModel: matrix of the wrong size");
    if (!int8_) {
      uint16_t* d = mem_.alloc<uint16_t>(w.size());
      check(hipMemcpy(d, w.data(), w.size() * sizeof(uint16_t), hipMemcpyHostToDevice),
            "hipMemcpy(weights)");
      return ie_matrix{d, nullptr, 0, rows, cols};
    }
    // Per row: s = max|w| / 127 (1 for a zero row), q = clamp(nearbyint(w / s)).
    std::vector<int8_t> q(w.size());
    std::vector<float> sc(rows);
    for (int r = 0; r < rows; ++r) {
      const uint16_t* row = w.data() + size_t(r) * cols;
      float amax = 0.0f;
      for (int i = 0; i < cols; ++i) amax = std::max(amax, std::fabs(bf16_value(row[i])));
      const float s = amax > 0 ? amax / 127.0f : 1.0f;
      sc[r] = s;
      for (int i = 0; i < cols; ++i) {
        const float v = std::nearbyint(bf16_value(row[i]) / s);
        q[size_t(r) * cols + i] = int8_t(std::max(-127.0f, std::min(127.0f, v)));
      }
    }
    int8_t* d = mem_.alloc<int8_t>(q.size());
    check(hipMemcpy(d, q.data(), q.size(), hipMemcpyHostToDevice), "hipMemcpy(weights)");
    return ie_matrix{d, upload(sc, sc.size()), 1, rows, cols};
  }
  static float bf16_value(uint16_t b) {
    const uint32_t bits = uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
  }

  KvConfig kv_;
  ModelShape shape_;
  int max_rows_;
  bool int8_;
  DeviceMemory mem_;
  ie_matrix embed_{};
  const float* final_norm_ = nullptr;
  std::vector<Layer> layers_;
  float *x_ = nullptr, *xn_ = nullptr, *mid_ = nullptr;
  int32_t* ids_ = nullptr;
  PinnedBuffer<int32_t> ids_host_;  // staging of a step's token ids
};

}  // namespace ie::hip

#endif  // IE_HIP_MODEL_HPP_
