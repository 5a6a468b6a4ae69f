// Self-test of the drop-in: the HIP engine behind the reference's own Runner and
// BatchRunner interfaces (src/runner.h:19-80), made by ie::hip::make_runner /
// make_batch_runner and used through std::unique_ptr<ie::Runner / BatchRunner>
// only. TEST INFRASTRUCTURE.
//
// The checker is the reference's own CPU Runner (ie::make_cpu_runner,
// src/runner.cpp:39-41, over src/model.cpp), compiled in place from the
// reference checkout into oracle/_ref/libieref_model.so: one CPU Runner per
// sequence is fed the same tokens, and every logit the GPU returns is compared
// with it (max |d| / max |ref|, the reference's compare(), src/npy.cpp:98-110):
//   f32 KV cache: <= 1e-5 (the fp32 bar; only summation orders differ);
//   f16 / bf16 KV cache: <= 1e-2 (the CPU path has no 16-bit cache: its K/V
//   stay f32 where the GPU's round to 16 bits; the value is printed).
// Model: a 2-layer Qwen2 decoder of Qwen2.5-0.5B's layer shape (hidden 896,
// intermediate 4,864, 14 query / 2 KV heads of 64, theta 1e6), a 1,000-token
// vocabulary, tied embeddings, seeded weights stored by the reference's own
// make_matrix as BF16 or INT8.
//
// Sections:
//   batch   BatchRunner: prompts (1, 37, 300 rows and a continuation), decode
//           steps of 3 sequences (logits and greedy), close and LIFO page
//           reuse, the getters, and the reference's errors;
//   runner  Runner: forward (last logits, a one-token graph step, all logits,
//           stage reports), position, reset, max_tokens;
//   invariance  4 sequences decoded together equal each decoded alone, logits
//           bit for bit, through two engines;
//   serve   the continuous-batching scheduler (include/ie_hip_serve.hpp): 24
//           requests at concurrency 1, 4 and 16 give identical tokens
//           (serve-bench --check, src/main.cpp:845-888);
//   checkpoint (with --checkpoint DIR, instead of the sections above) a model
//           directory on disk (config.json + model.safetensors, written by
//           tests/checkpoint.py) read by the reference's own loader --
//           load_config (src/config.cpp), SafeTensorsFile (src/safetensors.cpp),
//           load_weights (src/weights.cpp:89-117) -- as BF16 and as INT8, the
//           way the reference's CLI loads a model (src/main.cpp:314-325), then
//           served by make_batch_runner and by the CPU Runner from the same
//           Weights: prompt and decode logits, untied LM head, q/k/v biases.
//
// usage: runner_selftest f32|f16|bf16 [bf16|int8] [--checkpoint DIR]
// exit status 0 when every check passes.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <memory>
#include <random>
#include <string>
#include <vector>

#include "ie_hip_runner.hpp"
#include "ie_hip_serve.hpp"
#include "config.h"       // reference: src/config.h (load_config)
#include "runner.h"       // reference: src/runner.h
#include "safetensors.h"  // reference: src/safetensors.h
#include "weights.h"      // reference: src/weights.h (load_weights)

namespace {

int g_tests = 0, g_fail = 0;

void result(bool ok, const std::string& what) {
  ++g_tests;
  if (!ok) ++g_fail;
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
}

constexpr int kLayers = 2, H = 896, I = 4864, V = 1000;

ie::Config config() {
  ie::Config c;
  c.hidden_size = H;
  c.intermediate_size = I;
  c.num_layers = kLayers;
  c.num_heads = 14;
  c.num_kv_heads = 2;
  c.head_dim = 64;
  c.vocab_size = V;
  c.max_position_embeddings = 32768;
  c.rms_norm_eps = 1e-6f;
  c.rope_theta = 1e6f;
  c.tie_word_embeddings = true;
  return c;
}

ie::Weights random_weights(const ie::Config& c, ie::DType dt, uint32_t seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> n01(0.0f, 1.0f);
  auto vec = [&](size_t n, float base, float s) {
    std::vector<float> v(n);
    for (float& e : v) e = base + s * n01(rng);
    return v;
  };
  auto mat = [&](int rows, int cols, float s) {
    return ie::make_matrix(vec(size_t(rows) * cols, 0.0f, s), rows, cols, dt);
  };
  ie::Weights w;
  w.dtype = dt;
  w.embed = mat(V, H, 1.0f);
  w.final_norm = vec(H, 1.0f, 0.1f);
  for (int l = 0; l < kLayers; ++l) {
    ie::LayerWeights L;
    L.input_norm = vec(H, 1.0f, 0.1f);
    L.post_attn_norm = vec(H, 1.0f, 0.1f);
    L.wq = mat(c.q_dim(), H, 0.04f);
    L.wk = mat(c.kv_dim(), H, 0.04f);
    L.wv = mat(c.kv_dim(), H, 0.04f);
    L.wo = mat(H, c.q_dim(), 0.03f);
    L.bq = vec(c.q_dim(), 0.0f, 0.1f);
    L.bk = vec(c.kv_dim(), 0.0f, 0.1f);
    L.bv = vec(c.kv_dim(), 0.0f, 0.1f);
    L.w_gate = mat(I, H, 0.03f);
    L.w_up = mat(I, H, 0.03f);
    L.w_down = mat(H, I, 0.015f);
    w.layers.push_back(std::move(L));
  }
  return w;
}

// max |got - want| / max |want| (src/npy.cpp:98-110), NaN-safe.
double rel_err(const std::vector<float>& got, const std::vector<float>& want) {
  if (got.size() != want.size()) return INFINITY;
  double d = 0, m = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double e = std::fabs(double(got[i]) - double(want[i]));
    if (!(e <= d)) d = e;  // NaN propagates
    m = std::max(m, std::fabs(double(want[i])));
  }
  return m > 0 ? d / m : d;
}

int32_t host_argmax(const float* x, int n) {  // src/sampler.cpp:26-31
  int32_t best = 0;
  for (int i = 1; i < n; ++i)
    if (x[i] > x[best]) best = i;
  return best;
}

bool same_bits(const std::vector<float>& a, const std::vector<float>& b) {
  return a.size() == b.size() && std::memcmp(a.data(), b.data(), a.size() * sizeof(float)) == 0;
}

template <class Op>
void expect_error(const char* what, const char* needle, Op op) {
  try {
    op();
    result(false, std::string(what) + ": no error raised");
  } catch (const std::exception& e) {
    result(std::strstr(e.what(), needle) != nullptr, std::string(what) + ": \"" + e.what() + "\"");
  }
}

struct Ctx {
  ie::Config cfg;
  ie::Weights w;
  ie::hip::KvDtype kv;
  double tol;
  std::mt19937 rng{20261202u};

  std::vector<int32_t> tokens(int n) {
    std::uniform_int_distribution<int> d(0, V - 1);
    std::vector<int32_t> t(n);
    for (auto& e : t) e = d(rng);
    return t;
  }
  std::unique_ptr<ie::Runner> cpu(int max_tokens) { return ie::make_cpu_runner(cfg, w, max_tokens); }
};

void section_batch(Ctx& c) {
  std::printf("---- BatchRunner\n");
  const int kMaxBatch = 3, kMaxSeq = 512;
  std::unique_ptr<ie::BatchRunner> gpu =
      ie::hip::make_batch_runner(c.cfg, c.w, kMaxBatch, kMaxSeq, size_t(1) << 34, true, c.kv);
  result(gpu->max_batch() == kMaxBatch && gpu->max_seq_len() == kMaxSeq && gpu->page_size() == 16,
         "max_batch / max_seq_len / page_size");
  result(gpu->total_pages() == kMaxBatch * kMaxSeq / 16 && gpu->free_pages() == gpu->total_pages(),
         "pool: every sequence at full length fits the byte budget");
  result(gpu->weight_bytes() == c.w.matrix_bytes(), "weight_bytes == Weights::matrix_bytes()");
  result(gpu->device_name().rfind("hip, ", 0) == 0, "device_name: " + gpu->device_name());
  const size_t kv_elem = c.kv == ie::hip::KvDtype::F32 ? 4 : 2;
  result(gpu->kv_cache_bytes() == size_t(2) * kLayers * gpu->total_pages() * 16 * 128 * kv_elem,
         "kv_cache_bytes");

  std::vector<int> seq;
  std::vector<std::unique_ptr<ie::Runner>> ref;
  for (int i = 0; i < kMaxBatch; ++i) {
    seq.push_back(gpu->open_sequence());
    ref.push_back(c.cpu(kMaxSeq));
  }
  result(seq[0] == 0 && seq[1] == 1 && seq[2] == 2 && gpu->open_sequence() == -1,
         "open_sequence: lowest free slots, then -1");

  auto cmp = [&](const std::string& what, const std::vector<float>& got,
                 const std::vector<float>& want) {
    const double r = rel_err(got, want);
    char b[200];
    std::snprintf(b, sizeof(b), "%s: logits rel %.2e (tol %.0e)", what.c_str(), r, c.tol);
    result(r <= c.tol, b);
  };
  const int lens[3] = {37, 1, 300};
  for (int i = 0; i < 3; ++i) {
    const std::vector<int32_t> p = c.tokens(lens[i]);
    cmp("prefill " + std::to_string(lens[i]) + " tokens (seq " + std::to_string(seq[i]) + ")",
        gpu->prefill(seq[i], p), ref[i]->forward(p));
    result(gpu->sequence_length(seq[i]) == lens[i], "sequence_length after the prefill");
  }
  {
    const std::vector<int32_t> p = c.tokens(20);
    cmp("prefill continuing at 300 (20 tokens)", gpu->prefill(seq[2], p), ref[2]->forward(p));
  }
  for (int step = 0; step < 3; ++step) {
    const std::vector<int32_t> t = c.tokens(3);
    const std::vector<float> got = gpu->decode(seq, t);
    for (int i = 0; i < 3; ++i) {
      const std::vector<float> row(got.begin() + size_t(i) * V, got.begin() + size_t(i + 1) * V);
      cmp("decode step " + std::to_string(step) + ", row " + std::to_string(i), row,
          ref[i]->forward({t[i]}));
    }
  }
  // Greedy: the device argmax of the step's own logits, and the CPU's choice
  // wherever its top two are apart by more than the tolerance.
  {
    const std::vector<int32_t> t = c.tokens(3);
    const std::vector<int32_t> got = gpu->decode_greedy(seq, t);
    bool same = got.size() == 3;
    for (int i = 0; i < 3 && same; ++i) {
      const std::vector<float> want = ref[i]->forward({t[i]});
      std::vector<float> sorted(want);
      std::sort(sorted.begin(), sorted.end());
      const float gap = sorted[V - 1] - sorted[V - 2];
      const float scale = std::max(std::fabs(sorted[V - 1]), std::fabs(sorted[0]));
      if (gap > 4 * c.tol * scale) same = got[i] == host_argmax(want.data(), V);
    }
    result(same, "decode_greedy == the CPU logits' argmax (rows with a clear maximum)");
    const std::vector<int32_t> p = c.tokens(5);
    (void)ref[1]->forward(p);
    const int32_t g = gpu->prefill_greedy(seq[1], p);
    result(g >= 0 && g < V, "prefill_greedy returns a token id");
  }

  // Close and reuse: pages go back, the next sequence takes the slot and the
  // last-freed page first, and attends only to its own rows.
  const int before = gpu->free_pages();
  const int owned = (gpu->sequence_length(seq[0]) + 15) / 16;
  gpu->close_sequence(seq[0]);
  result(gpu->free_pages() == before + owned && gpu->sequence_length(seq[0]) == 0,
         "close_sequence: pages back, length 0");
  const int s3 = gpu->open_sequence();
  result(s3 == seq[0], "open_sequence reuses the closed slot");
  {
    std::unique_ptr<ie::Runner> fresh = c.cpu(kMaxSeq);
    const std::vector<int32_t> p = c.tokens(70);
    cmp("prefill on reused pages (70 tokens)", gpu->prefill(s3, p), fresh->forward(p));
    const std::vector<int32_t> t = c.tokens(1);
    const std::vector<float> got = gpu->decode({s3}, t);
    cmp("decode on reused pages", got, fresh->forward(t));
  }
  // The reference's errors; the runner stays usable after them.
  expect_error("closed sequence", "invalid or closed sequence id", [&] {
    gpu->close_sequence(seq[1]);
    gpu->decode({seq[1]}, {1});
  });
  expect_error("token out of range", "token id out of range", [&] { gpu->prefill(s3, {V}); });
  expect_error("one token per sequence", "one token per sequence",
               [&] { gpu->decode({s3, seq[2]}, {1}); });
  expect_error("too long", "sequence longer than the maximum",
               [&] { gpu->prefill(seq[2], c.tokens(kMaxSeq)); });
  {
    std::unique_ptr<ie::BatchRunner> small =
        ie::hip::make_batch_runner(c.cfg, c.w, 2, kMaxSeq, 8 * 16 * 128 * kv_elem * 2 * kLayers,
                                   true, c.kv);
    result(small->total_pages() == 8, "byte budget of 8 pages -> 8 pages");
    const int a = small->open_sequence();
    expect_error("pool exhaustion", "KV cache full: no free pages",
                 [&] { small->prefill(a, c.tokens(9 * 16)); });
  }
  {
    const std::vector<int32_t> t = c.tokens(1);
    std::unique_ptr<ie::Runner> fresh = c.cpu(kMaxSeq);
    const int s = gpu->open_sequence();
    cmp("prefill after the errors", gpu->prefill(s, t), fresh->forward(t));
  }
}

void section_runner(Ctx& c) {
  std::printf("---- Runner\n");
  const int kMax = 600;
  std::unique_ptr<ie::Runner> gpu = ie::hip::make_runner(c.cfg, c.w, kMax, true, c.kv);
  std::unique_ptr<ie::Runner> cpu = c.cpu(kMax);
  result(gpu->max_tokens() == kMax && gpu->position() == 0, "max_tokens, position 0");
  result(gpu->weight_dtype() == c.w.dtype && gpu->num_params() == c.w.num_params(),
         "weight_dtype, num_params");
  auto cmp = [&](const std::string& what, const std::vector<float>& got,
                 const std::vector<float>& want) {
    const double r = rel_err(got, want);
    char b[200];
    std::snprintf(b, sizeof(b), "%s: logits rel %.2e", what.c_str(), r);
    result(r <= c.tol && got.size() == want.size(), b);
  };
  std::vector<int32_t> p = c.tokens(45);
  cmp("forward 45 tokens (last logits)", gpu->forward(p), cpu->forward(p));
  for (int i = 0; i < 3; ++i) {
    const std::vector<int32_t> t = c.tokens(1);
    cmp("forward 1 token (graph), step " + std::to_string(i), gpu->forward(t), cpu->forward(t));
  }
  result(gpu->position() == 48, "position advanced to 48");
  p = c.tokens(21);
  cmp("forward 21 tokens, all logits [21, vocab]", gpu->forward(p, true), cpu->forward(p, true));
  // A long all-logits forward: one step of the prompt kernel for all 300 rows
  // (the runner's logit rows are sized from max_tokens).
  p = c.tokens(300);
  cmp("forward 300 tokens, all logits [300, vocab]", gpu->forward(p, true),
      cpu->forward(p, true));
  result(gpu->position() == 369, "position advanced to 369");
  // Stage reports: the same names and shapes as the CPU's, in order.
  std::vector<std::string> gs, cs;
  std::vector<std::vector<float>> gd, cd;
  p = c.tokens(5);
  gpu->forward(p, false, [&](const std::string& s, const float* d, int rows, int cols) {
    gs.push_back(s + " " + std::to_string(rows) + "x" + std::to_string(cols));
    gd.emplace_back(d, d + size_t(rows) * cols);
  });
  cpu->forward(p, false, [&](const std::string& s, const float* d, int rows, int cols) {
    cs.push_back(s + " " + std::to_string(rows) + "x" + std::to_string(cols));
    cd.emplace_back(d, d + size_t(rows) * cols);
  });
  result(gs == cs, "on_stage: the CPU's stage names and shapes (" + std::to_string(gs.size()) +
                       " stages)");
  double worst = 0;
  for (size_t i = 0; i < std::min(gd.size(), cd.size()); ++i) worst = std::max(worst, rel_err(gd[i], cd[i]));
  char b[120];
  std::snprintf(b, sizeof(b), "on_stage: every stage within tolerance (worst rel %.2e)", worst);
  result(worst <= c.tol, b);
  gpu->reset();
  cpu->reset();
  result(gpu->position() == 0, "reset: position 0");
  p = c.tokens(3);
  cmp("forward after reset", gpu->forward(p), cpu->forward(p));
}

void section_invariance(Ctx& c) {
  std::printf("---- batch invariance\n");
  const int N = 4;
  std::unique_ptr<ie::BatchRunner> a =
      ie::hip::make_batch_runner(c.cfg, c.w, N, 1024, size_t(1) << 34, true, c.kv);
  std::unique_ptr<ie::BatchRunner> b =
      ie::hip::make_batch_runner(c.cfg, c.w, N, 1024, size_t(1) << 34, true, c.kv);
  std::vector<int> sa, sb;
  const int plen[N] = {3, 130, 517, 64};
  for (int i = 0; i < N; ++i) {
    sa.push_back(a->open_sequence());
    sb.push_back(b->open_sequence());
    const std::vector<int32_t> p = c.tokens(plen[i]);
    result(same_bits(a->prefill(sa[i], p), b->prefill(sb[i], p)),
           "prefill " + std::to_string(plen[i]) + ": the two engines agree bit for bit");
  }
  bool same = true;
  for (int step = 0; step < 6; ++step) {
    const std::vector<int32_t> t = c.tokens(N);
    const std::vector<float> batch = a->decode(sa, t);  // all together
    for (int i = 0; i < N; ++i) {                        // one at a time
      const std::vector<float> one = b->decode({sb[i]}, {t[i]});
      same = same && std::memcmp(one.data(), batch.data() + size_t(i) * V, V * sizeof(float)) == 0;
    }
  }
  result(same, "decode: 4 sequences in one batch == each alone, logits bit for bit (6 steps)");
  const std::vector<int32_t> t = c.tokens(N);
  const std::vector<int32_t> ga = a->decode_greedy(sa, t);
  bool gsame = true;
  for (int i = 0; i < N; ++i) gsame = gsame && b->decode_greedy({sb[i]}, {t[i]}).at(0) == ga[i];
  result(gsame, "decode_greedy: batch == each alone");
}

void section_serve(Ctx& c) {
  std::printf("---- continuous batching (serve-bench --check)\n");
  std::vector<ie::hip::ServeRequest> reqs(24);
  std::uniform_int_distribution<int> plen(8, 160), glen(4, 24);
  for (auto& r : reqs) {
    r.prompt = c.tokens(plen(c.rng));
    r.gen = glen(c.rng);
  }
  reqs[3].gen = 1;  // finishes at its prefill
  const int max_batch = 16;
  std::unique_ptr<ie::BatchRunner> eng =
      ie::hip::make_batch_runner(c.cfg, c.w, max_batch, 256, size_t(1) << 34, true, c.kv);
  const ie::hip::ServeReport one = ie::hip::serve(*eng, reqs, 1);
  result(eng->free_pages() == eng->total_pages(), "one at a time: every page back at the end");
  bool lengths = true;
  for (size_t i = 0; i < reqs.size(); ++i)
    lengths = lengths && int(one.requests[i].tokens.size()) == reqs[i].gen;
  result(lengths && one.largest_batch == 1, "one at a time: each request its own length");
  for (int conc : {4, 16}) {
    const ie::hip::ServeReport s = ie::hip::serve(*eng, reqs, conc);
    const ie::hip::TokenMatch k = ie::hip::tokens_match(s, one);
    char b[200];
    std::snprintf(b, sizeof(b),
                  "%d running at most: %d/%d identical to one at a time (largest batch %d, %d "
                  "steps, %.0f tok/s)%s",
                  conc, k.same, k.total, s.largest_batch, s.decode_steps,
                  double(s.tokens()) / s.wall_s, k.all() ? "" : " -- first difference below");
    result(k.all() && s.largest_batch > 1, b);
    if (!k.all()) std::printf("     request %d differs from token %d\n", k.first_request, k.first_token);
    result(eng->free_pages() == eng->total_pages(), "every page back at the end");
  }
  // Admission by full-length promise: a cache of 10 pages serves requests of 6
  // pages one at a time even with 4 slots.
  {
    const size_t kv_elem = c.kv == ie::hip::KvDtype::F32 ? 4 : 2;
    std::unique_ptr<ie::BatchRunner> small = ie::hip::make_batch_runner(
        c.cfg, c.w, 4, 96, 10 * 16 * 128 * kv_elem * 2 * kLayers, true, c.kv);
    std::vector<ie::hip::ServeRequest> r(3);
    for (auto& q : r) {
      q.prompt = c.tokens(80);
      q.gen = 10;  // 90 tokens: 6 pages
    }
    const ie::hip::ServeReport s = ie::hip::serve(*small, r, 4);
    result(s.largest_batch == 1 && s.most_pages_in_use <= 6,
           "full-length promise: one 6-page request at a time in a 10-page cache");
    std::vector<ie::hip::ServeRequest> big(1);
    big[0].prompt = c.tokens(90);
    big[0].gen = 80;
    expect_error("a request larger than the cache", "KV-cache pages at full length",
                 [&] { ie::hip::serve(*small, big, 1); });
    result(small->free_pages() == small->total_pages(), "a refused request holds no pages");
  }
}


// The drop-in's `ie test-cuda` / `ie gpu-check` counterparts and kernel
// switches (src/main.cpp:272-287,1033-1045,1207-1213).
void section_cli(Ctx& c) {
  std::printf("---- run_selftest / run_device_check / kernel switches\n");
  std::fflush(stdout);
  const int failures = ie::hip::run_selftest();
  std::fflush(stdout);
  result(failures == 0, "run_selftest: every kernel family against the host CPU operations");
  const int dc = ie::hip::run_device_check();
  std::fflush(stdout);
  result(dc == 0, "run_device_check");
  // set_tensor_cores(false) and set_tc_fp16(false) switch the attention kernels
  // and the prefill rounding; a prompt's logits must stay within the bar of
  // the CPU Runner either way, and the switches restore.
  std::unique_ptr<ie::Runner> cpu = ie::make_cpu_runner(c.cfg, c.w, 256);
  const std::vector<int32_t> prompt = c.tokens(40);
  const std::vector<float> want = cpu->forward(prompt);
  for (const bool tc : {false, true})
    for (const bool fp16 : {false, true}) {
      ie::hip::set_tensor_cores(tc);
      ie::hip::set_tc_fp16(fp16);
      std::unique_ptr<ie::Runner> gpu = ie::hip::make_runner(c.cfg, c.w, 256, true, c.kv);
      const double e = rel_err(gpu->forward(prompt), want);
      char b[160];
      std::snprintf(b, sizeof(b), "tensor_cores %d, tc_fp16 %d: 40-token prompt logits rel %.2e",
                    int(tc), int(fp16), e);
      result(e <= c.tol, b);
    }
  ie::hip::set_tensor_cores(true);
  ie::hip::set_tc_fp16(true);
  ie::hip::set_cublas(false);
  expect_error("set_cublas(true)", "no cuBLAS", [] { ie::hip::set_cublas(true); });
}

void section_checkpoint(Ctx& c, const std::string& dir) {
  std::printf("---- checkpoint %s\n", dir.c_str());
  const ie::Config cfg = ie::load_config(dir + "/config.json");
  const ie::SafeTensorsFile st(dir + "/model.safetensors");
  result(cfg.num_layers == 2 && cfg.head_dim == 64 && !cfg.tie_word_embeddings &&
             st.contains("lm_head.weight") && st.contains("model.layers.1.self_attn.q_proj.bias"),
         "config.json and the safetensors index read by the reference's loader");
  for (const ie::DType dt : {ie::DType::BF16, ie::DType::I8}) {
    const std::string dn = dt == ie::DType::BF16 ? "bf16" : "int8";
    const ie::Weights w = ie::load_weights(st, cfg, dt);
    std::unique_ptr<ie::BatchRunner> gpu =
        ie::hip::make_batch_runner(cfg, w, 2, 256, size_t(64) << 20, true, c.kv);
    std::unique_ptr<ie::Runner> cpu = ie::make_cpu_runner(cfg, w, 256);
    result(gpu->weight_bytes() == w.matrix_bytes() && gpu->config().vocab_size == cfg.vocab_size,
           dn + ": weight_bytes and config of the served model");
    std::uniform_int_distribution<int> d(0, cfg.vocab_size - 1);
    std::vector<int32_t> prompt(29);
    for (auto& e : prompt) e = d(c.rng);
    const int s = gpu->open_sequence();
    const std::vector<float> gp = gpu->prefill(s, prompt), cp = cpu->forward(prompt);
    double worst = rel_err(gp, cp);
    // Decode follows the CPU's greedy tokens, so both see the same sequence
    // whatever a near-tie does; the GPU's own greedy choice is counted.
    int32_t tok = host_argmax(cp.data(), cfg.vocab_size);
    int agree = 0;
    const int steps = 6;
    for (int i = 0; i < steps; ++i) {
      const std::vector<float> g = gpu->decode({s}, {tok}), r = cpu->forward({tok});
      worst = std::max(worst, rel_err(g, r));
      const int32_t rt = host_argmax(r.data(), cfg.vocab_size);
      agree += host_argmax(g.data(), cfg.vocab_size) == rt;
      tok = rt;
    }
    char b[200];
    std::snprintf(b, sizeof(b), "%s: prefill of 29 tokens and %d decode steps, logits rel %.2e "
                  "(greedy agrees on %d of %d)", dn.c_str(), steps, worst, agree, steps);
    result(worst <= c.tol, b);
    result(gpu->sequence_length(s) == 29 + steps, dn + ": sequence length after decode");
    gpu->close_sequence(s);
    result(gpu->free_pages() == gpu->total_pages(), dn + ": pages returned on close");
  }
}

}  // namespace

int main(int argc, char** argv) {
  const std::string kvs = argc > 1 ? argv[1] : "f32";
  const std::string wts = argc > 2 ? argv[2] : "bf16";
  const std::string ckpt = argc > 4 && std::string(argv[3]) == "--checkpoint" ? argv[4] : "";
  std::printf("runner self-test: %s KV cache, %s weights, device %s\n", kvs.c_str(), wts.c_str(),
              ie::hip::device_description().c_str());
  std::fflush(stdout);
  try {
    if (!ie::hip::device_available()) {
      std::printf("FAIL no HIP device\n");
      return 2;
    }
    Ctx c;
    c.cfg = config();
    c.kv = kvs == "f16" ? ie::hip::KvDtype::F16
                        : kvs == "bf16" ? ie::hip::KvDtype::BF16 : ie::hip::KvDtype::F32;
    c.tol = c.kv == ie::hip::KvDtype::F32 ? 1e-5 : 1e-2;
    if (!ckpt.empty()) {
      section_checkpoint(c, ckpt);
    } else {
      c.w = random_weights(c.cfg, wts == "int8" ? ie::DType::I8 : ie::DType::BF16, 7u);
      section_batch(c);
      section_runner(c);
      section_invariance(c);
      section_serve(c);
      section_cli(c);
    }
  } catch (const std::exception& e) {
    std::printf("FAIL exception: %s\n", e.what());
    return 2;
  }
  std::printf("%d checks, %d failures\n", g_tests, g_fail);
  return g_fail ? 1 : 0;
}
