// Self-test of the decode step around the paged path (include/ie_hip_model.hpp
// over include/ie_hip_engine.hpp) on the GPU against a CPU forward pass built
// from the oracle (oracle/liborc.so). TEST INFRASTRUCTURE.
//
// A 2-layer Qwen2 decoder of Qwen2.5-0.5B's layer shape (hidden 896,
// intermediate 4,864, 14 query / 2 KV heads of 64) with a 512-token vocabulary
// and seeded BF16 weights runs prompts of 40 and 17 tokens, batch-2 decode
// steps (the graph recorded, then replayed) and a batch-1 decode. After every
// step the residual stream of every row and the logits are compared with the
// reference's CPU forward restated on the oracle (src/model.cpp:46-107:
// orc_row_to_f32, orc_rmsnorm, orc_matmul, orc_rope_append_paged,
// orc_paged_attention, orc_silu_mul) on the engine's own page tables:
// max |d| / max |ref| <= 1e-5 for an f32 cache (the fp32 bar; measured about
// 2e-6 after two layers), <= 1e-3 for f16 (the appended K/V rows round to f16
// on both sides from inputs that already differ in the last float32 bits;
// measured about 6e-5).
//
// With `int8`, every matrix is stored as INT8 with row scales on both sides
// (the reference's --dtype int8).
//
// usage: model_selftest f32|f16 [int8]      exit status 0 when every check passes.
#include <cmath>
#include <cstdio>
#include <random>
#include <string>
#include <vector>

#include "ie_hip_model.hpp"
#include "oracle.h"

using namespace ie::hip;

namespace {

/* One layer's weights on the host, BF16 bits in the reference's layout. */
struct HostLayer {
  std::vector<float> input_norm, post_norm;    // [hidden]
  std::vector<uint16_t> wq, wk, wv, wo;        // [q_dim, hidden], [kv_dim, hidden] x2, [hidden, q_dim]
  std::vector<float> bq, bk, bv;               // [q_dim], [kv_dim] x2
  std::vector<uint16_t> w_gate, w_up, w_down;  // [inter, hidden] x2, [hidden, inter]
};

/* The model's weights on the host; the LM head is the embedding (tied). */
struct HostModel {
  std::vector<uint16_t> embed;    // [vocab, hidden]
  std::vector<float> final_norm;  // [hidden]
  std::vector<HostLayer> layers;
};

constexpr int kLayers = 2, NH = 14, NKV = 2, HD = 64, QD = NH * HD, KVD = NKV * HD;
constexpr int H = 896, I = 4864, V = 512, kMaxBatch = 4, kMaxSeq = 256, kPages = 64;
constexpr float kTheta = 1e6f, kEps = 1e-6f;

int g_tests = 0, g_fail = 0;

void result(bool ok, const std::string& what) {
  ++g_tests;
  if (!ok) ++g_fail;
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
}

struct Cpu {  // the reference's CPU forward on the oracle, over paged host pools
  const HostModel& m;
  int kv;
  bool int8;
  std::vector<std::vector<unsigned char>> kp, vp;
  Cpu(const HostModel& model, int kv_dtype, size_t pool_bytes, bool int8_weights)
      : m(model), kv(kv_dtype), int8(int8_weights),
        kp(kLayers, std::vector<unsigned char>(pool_bytes)),
        vp(kLayers, std::vector<unsigned char>(pool_bytes)) {}

  // A matrix as the reference stores it for --dtype int8 (src/matrix.cpp:84-97).
  struct Q8 {
    std::vector<int8_t> q;
    std::vector<float> s;
  };
  Q8 quantize(const std::vector<uint16_t>& w, int rows, int cols) {
    std::vector<float> f(w.size());
    for (size_t i = 0; i < w.size(); ++i) f[i] = orc_bf16_to_f32(w[i]);
    Q8 r{std::vector<int8_t>(w.size()), std::vector<float>(rows)};
    orc_quantize_i8(r.q.data(), r.s.data(), f.data(), rows, cols);
    return r;
  }

  std::vector<float> mm(const std::vector<float>& x, const std::vector<uint16_t>& w,
                        const std::vector<float>* b, int T, int rows, int cols) {
    std::vector<float> y(size_t(T) * rows);
    if (int8) {
      const Q8 q = quantize(w, rows, cols);
      orc_matmul(y.data(), x.data(), q.q.data(), ORC_W_I8, q.s.data(), b ? b->data() : nullptr,
                 T, rows, cols, 8);
    } else {
      orc_matmul(y.data(), x.data(), w.data(), ORC_W_BF16, nullptr, b ? b->data() : nullptr, T,
                 rows, cols, 8);
    }
    return y;
  }

  // One step; returns x after the last layer and the logits of every row.
  void step(const std::vector<int32_t>& ids, const std::vector<int32_t>& pos,
            const std::vector<int32_t>& seq, const int32_t* tables, int max_pages,
            std::vector<float>& x, std::vector<float>& logits) {
    const int T = int(ids.size());
    x.assign(size_t(T) * H, 0.0f);
    if (int8) {
      const Q8 e = quantize(m.embed, V, H);
      for (int t = 0; t < T; ++t)
        orc_row_to_f32(&x[size_t(t) * H], e.q.data(), ORC_W_I8, e.s.data(), H, ids[t]);
    } else {
      for (int t = 0; t < T; ++t)
        orc_row_to_f32(&x[size_t(t) * H], m.embed.data(), ORC_W_BF16, nullptr, H, ids[t]);
    }
    std::vector<float> xn(x.size());
    for (int l = 0; l < kLayers; ++l) {
      const HostLayer& L = m.layers[l];
      orc_rmsnorm(xn.data(), x.data(), L.input_norm.data(), T, H, kEps);
      std::vector<float> q = mm(xn, L.wq, &L.bq, T, QD, H), k = mm(xn, L.wk, &L.bk, T, KVD, H),
                         v = mm(xn, L.wv, &L.bv, T, KVD, H);
      orc_rope_append_paged(q.data(), k.data(), v.data(), kp[l].data(), vp[l].data(), kv, T,
                            pos.data(), seq.data(), tables, max_pages, kPageSize, NH, NKV, HD,
                            kTheta);
      std::vector<float> attn(size_t(T) * QD);
      orc_paged_attention(attn.data(), q.data(), kp[l].data(), vp[l].data(), kv, T, pos.data(),
                          seq.data(), tables, max_pages, kPageSize, NH, NKV, HD, 8);
      std::vector<float> o = mm(attn, L.wo, nullptr, T, H, QD);
      for (size_t i = 0; i < x.size(); ++i) x[i] += o[i];
      orc_rmsnorm(xn.data(), x.data(), L.post_norm.data(), T, H, kEps);
      std::vector<float> g = mm(xn, L.w_gate, nullptr, T, I, H), u = mm(xn, L.w_up, nullptr, T, I, H);
      orc_silu_mul(g.data(), u.data(), g.size());
      std::vector<float> d = mm(g, L.w_down, nullptr, T, H, I);
      for (size_t i = 0; i < x.size(); ++i) x[i] += d[i];
    }
    orc_rmsnorm(xn.data(), x.data(), m.final_norm.data(), T, H, kEps);
    logits = mm(xn, m.embed, nullptr, T, V, H);
  }
};

HostModel random_model(std::mt19937& rng) {
  std::normal_distribution<float> n01(0.0f, 1.0f);
  auto bf = [&](size_t n, float s) {
    std::vector<uint16_t> w(n);
    for (auto& e : w) e = orc_f32_to_bf16(s * n01(rng));
    return w;
  };
  auto f = [&](size_t n, float base, float s) {
    std::vector<float> w(n);
    for (auto& e : w) e = base + s * n01(rng);
    return w;
  };
  HostModel m;
  m.embed = bf(size_t(V) * H, 1.0f);
  m.final_norm = f(H, 1.0f, 0.1f);
  for (int l = 0; l < kLayers; ++l) {
    HostLayer L;
    L.input_norm = f(H, 1.0f, 0.1f);
    L.post_norm = f(H, 1.0f, 0.1f);
    L.wq = bf(size_t(QD) * H, 0.04f);
    L.wk = bf(size_t(KVD) * H, 0.04f);
    L.wv = bf(size_t(KVD) * H, 0.04f);
    L.wo = bf(size_t(H) * QD, 0.03f);
    L.bq = f(QD, 0.0f, 0.1f);
    L.bk = f(KVD, 0.0f, 0.1f);
    L.bv = f(KVD, 0.0f, 0.1f);
    L.w_gate = bf(size_t(I) * H, 0.03f);
    L.w_up = bf(size_t(I) * H, 0.03f);
    L.w_down = bf(size_t(H) * I, 0.015f);
    m.layers.push_back(std::move(L));
  }
  return m;
}

/* The device-side view of a HostModel: BF16 as stored, or every matrix
 * quantized to INT8 with row scales exactly as the CPU side quantizes it. */
struct Upload {
  std::vector<std::vector<int8_t>> q;
  std::vector<std::vector<float>> s;
  ModelView view;

  MatrixView matrix(const std::vector<uint16_t>& w, int rows, int cols, bool int8) {
    MatrixView m;
    m.rows = rows;
    m.cols = cols;
    if (!int8) {
      m.data = w.data();
      return m;
    }
    std::vector<float> f(w.size());
    for (size_t i = 0; i < w.size(); ++i) f[i] = orc_bf16_to_f32(w[i]);
    q.emplace_back(w.size());
    s.emplace_back(rows);
    orc_quantize_i8(q.back().data(), s.back().data(), f.data(), rows, cols);
    m.data = q.back().data();
    m.scale = s.back().data();
    m.int8 = true;
    return m;
  }

  Upload(const HostModel& h, bool int8) {
    q.reserve(64);
    s.reserve(64);
    view.embed = matrix(h.embed, V, H, int8);
    view.final_norm = h.final_norm.data();
    for (const HostLayer& L : h.layers) {
      LayerView l;
      l.input_norm = L.input_norm.data();
      l.post_norm = L.post_norm.data();
      l.wq = matrix(L.wq, QD, H, int8);
      l.wk = matrix(L.wk, KVD, H, int8);
      l.wv = matrix(L.wv, KVD, H, int8);
      l.wo = matrix(L.wo, H, QD, int8);
      l.bq = L.bq.data();
      l.bk = L.bk.data();
      l.bv = L.bv.data();
      l.w_gate = matrix(L.w_gate, I, H, int8);
      l.w_up = matrix(L.w_up, I, H, int8);
      l.w_down = matrix(L.w_down, H, I, int8);
      view.layers.push_back(l);
    }
  }
};

template <class T>
std::vector<T> download(const void* d, size_t n) {
  std::vector<T> h(n);
  check(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "download");
  return h;
}

}  // namespace

int main(int argc, char** argv) {
  const std::string kvs = argc > 1 ? argv[1] : "f32";
  const bool int8 = argc > 2 && std::string(argv[2]) == "int8";
  const int kv = kvs == "f16" ? IE_KV_F16 : IE_KV_F32;
  const double tol = kv == IE_KV_F32 ? 1e-5 : 1e-3;
  std::mt19937 rng(20261201u);
  const HostModel host = random_model(rng);
  KvConfig cfg;
  cfg.num_layers = kLayers;
  ModelShape shape;
  shape.vocab = V;
  try {
    EngineLimits lim;
    lim.max_batch = kMaxBatch;
    lim.max_seq_len = kMaxSeq;
    lim.num_pages = kPages;
    lim.step_rows = 64;
    lim.logit_rows = 64;
    KvEngine eng(cfg, lim, kv, /*use_graphs=*/true);
    const Upload up(host, int8);
    DecoderModel model(cfg, shape, up.view, eng.limits().step_rows, eng.limits().logit_rows);
    eng.set_body(model.body(eng));
    Cpu cpu(host, kv, eng.layer_pool_bytes(), int8);
    std::uniform_int_distribution<int> tok(0, V - 1);

    // One step through the engine, then the same step on the CPU; every row's
    // residual stream and logits compared.
    auto run_step = [&](const std::string& what, const std::vector<int32_t>& seqs,
                        const std::vector<int32_t>& pos, bool prefill) {
      const int T = int(seqs.size());
      std::vector<int32_t> ids(T);
      for (auto& id : ids) id = tok(rng);
      std::vector<int> all(T);
      for (int i = 0; i < T; ++i) all[i] = i;
      eng.run(std::vector<int>(seqs.begin(), seqs.end()), std::vector<int>(pos.begin(), pos.end()),
              ids, all, /*decode=*/!prefill);
      eng.sync();
      std::vector<float> x_ref, lg_ref;
      cpu.step(ids, pos, seqs, eng.host_tables(), eng.max_pages_per_seq(), x_ref, lg_ref);
      const std::vector<float> x = download<float>(model.x(), size_t(T) * H);
      const std::vector<float> lg = download<float>(model.logits(), size_t(T) * V);
      double mae = 0;
      size_t worst = 0;
      const double rx = orc_compare(x.data(), x_ref.data(), x.size(), &mae, &worst);
      const double rl = orc_compare(lg.data(), lg_ref.data(), lg.size(), &mae, &worst);
      char buf[160];
      std::snprintf(buf, sizeof(buf), "%s: residual rel %.2e, logits rel %.2e (graph %d)",
                    what.c_str(), rx, rl, int(eng.last_step().graph));
      result(rx <= tol && rl <= tol && std::isfinite(rx) && std::isfinite(rl), buf);
      return lg;
    };

    const int s0 = eng.open_sequence(), s1 = eng.open_sequence();
    std::vector<int32_t> p40(40), p17(17);
    for (int i = 0; i < 40; ++i) p40[i] = i;
    for (int i = 0; i < 17; ++i) p17[i] = i;
    run_step("prompt of 40", std::vector<int32_t>(40, s0), p40, true);
    run_step("prompt of 17", std::vector<int32_t>(17, s1), p17, true);
    for (int i = 0; i < 3; ++i)
      run_step("decode batch 2, step " + std::to_string(i), {s0, s1}, {40 + i, 17 + i}, false);
    run_step("decode batch 1", {s1}, {20}, false);

    // The device argmax of the last step's logits: the CPU scan's choice.
    {
      const std::vector<float> lg = download<float>(model.logits(), V);
      model.argmax(1, eng.stream());
      eng.sync();
      const int32_t got = download<int32_t>(model.tokens(), 1)[0];
      int32_t want = 0;
      for (int i = 1; i < V; ++i)
        if (lg[i] > lg[want]) want = i;
      result(got == want, "argmax of the logits (device) == first strict maximum (host scan)");
    }
  } catch (const std::exception& e) {
    result(false, std::string("exception: ") + e.what());
  }
  std::printf("%d checks, %d failures\n", g_tests, g_fail);
  return g_fail ? 1 : 0;
}
