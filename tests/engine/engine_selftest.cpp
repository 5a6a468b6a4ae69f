// Self-test of the C++ engine layer (include/ie_hip_engine.hpp) on the GPU
// against the CPU oracle (oracle/liborc.so). TEST INFRASTRUCTURE.
//
// The reference checks its paged kernels with run_selftest
// (src/cuda/cuda_runner.cu:849-1018): rope + cache writes into two sequences,
// then attention cases -- first token, chunk edges 63/64 and 255/256, a
// 3,000-token context, a prompt continuing at 500, prompts of 1/17/300/1000
// rows, the 2nd of 2 sequences, a batch of 5 decodes, mixed prefill + decode --
// with f32 and f16 caches. Here the same situations arise from a serving
// sequence driven through KvEngine (open, prefill, decode graphs, a mixed
// direct step, close and reuse of pages, pool exhaustion), with a 2-layer
// model whose per-layer q/k/v are seeded N(0,1) rows fed by the LayerBody.
// After every step, for every layer:
//   - both page pools equal the oracle's (orc_rope_append_paged on a host
//     copy of the pools), byte for byte;
//   - the device page table equals the engine's host table;
//   - attention equals the oracle's (orc_attention over each sequence's
//     gathered contiguous copy) within 1e-5 relative error (f32 cache, the
//     reference's compare()) or 2e-3 absolute (f16/bf16);
// plus the step's path (graph / prompt / fused), page conservation and the
// errors the reference raises (KV cache full, too long, closed sequence).
//
// usage: engine_selftest f32|f16|bf16      exit status 0 when every check passes.
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include "ie_hip_engine.hpp"
#include "oracle.h"

using ie::hip::KvEngine;

namespace {

constexpr int kLayers = 2, NH = 14, NKV = 2, HD = 64, QD = NH * HD, KVD = NKV * HD;
constexpr float kTheta = 1e6f;
constexpr int kMaxBatch = 6, kMaxSeq = 4096, kPages = 500, kCap = 4096;

int g_tests = 0, g_fail = 0;

void result(bool ok, const std::string& what) {
  ++g_tests;
  if (!ok) ++g_fail;
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  std::fflush(stdout);
}

template <class T>
std::vector<T> download(const void* d, size_t n) {
  std::vector<T> h(n);
  ie::hip::check(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "download");
  return h;
}

struct Harness {
  int kv;
  std::mt19937 rng{20260101u};
  std::normal_distribution<float> normal{0.0f, 1.0f};
  KvEngine* eng = nullptr;
  // Per-layer step inputs and outputs on the device, [kCap rows].
  float *in_q[kLayers], *in_k[kLayers], *in_v[kLayers], *out[kLayers];
  int32_t* ident = nullptr;
  // The oracle's copy of every layer's pools.
  std::vector<unsigned char> kp_ref[kLayers], vp_ref[kLayers];
  int threads = 1;

  explicit Harness(int kv_dtype) : kv(kv_dtype) {
    threads = int(std::min(14u, std::max(1u, std::thread::hardware_concurrency())));
  }

  std::vector<float> randn(size_t n) {
    std::vector<float> x(n);
    for (float& e : x) e = normal(rng);
    return x;
  }

  ie::hip::LayerBody body() {
    ie::hip::LayerBody b;
    b.before_attention = [this](int l, int T, hipStream_t s) {
      ie::hip::gather_rows(eng->q(), in_q[l], ident, T, QD, s);
      ie::hip::gather_rows(eng->k(), in_k[l], ident, T, KVD, s);
      ie::hip::gather_rows(eng->v(), in_v[l], ident, T, KVD, s);
    };
    b.after_attention = [this](int l, int T, hipStream_t s) {
      ie::hip::gather_rows(out[l], eng->attn(), ident, T, QD, s);
    };
    return b;
  }

  void allocate() {
    for (int l = 0; l < kLayers; ++l) {
      for (float** p : {&in_q[l], &out[l]})
        ie::hip::check(hipMalloc(p, size_t(kCap) * QD * sizeof(float)), "hipMalloc");
      for (float** p : {&in_k[l], &in_v[l]})
        ie::hip::check(hipMalloc(p, size_t(kCap) * KVD * sizeof(float)), "hipMalloc");
    }
    std::vector<int32_t> id(kCap);
    for (int i = 0; i < kCap; ++i) id[i] = i;
    ie::hip::check(hipMalloc(&ident, kCap * sizeof(int32_t)), "hipMalloc");
    ie::hip::check(hipMemcpy(ident, id.data(), kCap * sizeof(int32_t), hipMemcpyHostToDevice),
                   "ident");
  }

  // Stale pool contents everywhere (N(0,1) in the cache's type), mirrored by
  // the oracle: pages handed out again must not leak their old rows.
  void fill_pools() {
    const size_t n = eng->layer_pool_bytes() / (kv == IE_KV_F32 ? 4 : 2);
    for (int l = 0; l < kLayers; ++l)
      for (int kvside = 0; kvside < 2; ++kvside) {
        std::vector<unsigned char>& ref = kvside ? vp_ref[l] : kp_ref[l];
        ref.resize(eng->layer_pool_bytes());
        const std::vector<float> x = randn(n);
        orc_round_to_kv(ref.data(), x.data(), n, kv);
        ie::hip::check(hipMemcpy(kvside ? eng->v_pool(l) : eng->k_pool(l), ref.data(), ref.size(),
                                 hipMemcpyHostToDevice),
                       "pool upload");
      }
  }

  int open_pages() {
    int used = 0;
    std::vector<int32_t> tmp(eng->max_pages_per_seq());
    for (int s = 0; s < eng->max_batch(); ++s)
      used += std::max(eng->sequence_pages(s, tmp.data(), int(tmp.size())), 0);
    return used;
  }

  // Runs one engine step over the given rows (`op` performs it) and checks
  // everything the step produced. want_* < 0: not checked.
  template <class Op>
  void step(const std::string& name, const std::vector<int>& rows_seq,
            const std::vector<int>& rows_pos, Op op, int want_graph, int want_prompt,
            int want_fused) {
    const int T = int(rows_seq.size());
    std::vector<float> q[kLayers], k[kLayers], v[kLayers];
    for (int l = 0; l < kLayers; ++l) {
      q[l] = randn(size_t(T) * QD);
      k[l] = randn(size_t(T) * KVD);
      v[l] = randn(size_t(T) * KVD);
      ie::hip::check(hipMemcpy(in_q[l], q[l].data(), q[l].size() * 4, hipMemcpyHostToDevice), "q");
      ie::hip::check(hipMemcpy(in_k[l], k[l].data(), k[l].size() * 4, hipMemcpyHostToDevice), "k");
      ie::hip::check(hipMemcpy(in_v[l], v[l].data(), v[l].size() * 4, hipMemcpyHostToDevice), "v");
    }
    std::printf("---- %s (%d rows)\n", name.c_str(), T);
    std::fflush(stdout);
    op();
    const ie::hip::StepInfo& si = eng->last_step();
    // Flash-decoding steps that fit one launch read the work list the engine
    // builds on the host (every KV type); prompts do not.
    const bool want_planned = !si.prompt && T <= std::max(eng->max_batch(), 16);
    char path[200];
    std::snprintf(path, sizeof(path), "%s: path graph=%d prompt=%d fused=%d planned=%d chunk=%d x %d",
                  name.c_str(), si.graph, si.prompt, si.fused, si.planned, si.chunk_tokens,
                  si.chunks);
    result(si.rows == T && (want_graph < 0 || si.graph == bool(want_graph)) &&
               (want_prompt < 0 || si.prompt == bool(want_prompt)) &&
               (want_fused < 0 || si.fused == bool(want_fused)) && si.planned == want_planned,
           path);

    const size_t tab_n = size_t(eng->max_batch()) * eng->max_pages_per_seq();
    const std::vector<int32_t> dtab = download<int32_t>(eng->device_tables(), tab_n);
    const int32_t* htab = eng->host_tables();
    result(std::memcmp(dtab.data(), htab, tab_n * 4) == 0, name + ": device page table");
    result(eng->free_pages() + open_pages() == eng->total_pages(),
           name + ": free + owned pages == total");

    for (int l = 0; l < kLayers; ++l) {
      std::vector<float> qr = q[l];
      orc_rope_append_paged(qr.data(), k[l].data(), v[l].data(), kp_ref[l].data(),
                            vp_ref[l].data(), kv, T, rows_pos.data(), rows_seq.data(), htab,
                            eng->max_pages_per_seq(), ie::hip::kPageSize, NH, NKV, HD, kTheta);
      const std::vector<unsigned char> kp = download<unsigned char>(eng->k_pool(l), kp_ref[l].size());
      const std::vector<unsigned char> vp = download<unsigned char>(eng->v_pool(l), vp_ref[l].size());
      const std::string ln = name + ": layer " + std::to_string(l);
      result(kp == kp_ref[l], ln + " K pool bit-exact");
      result(vp == vp_ref[l], ln + " V pool bit-exact");

      // Attention: each run of consecutive positions of one sequence attends
      // over one gathered copy of that sequence.
      std::vector<float> want(size_t(T) * QD);
      for (int t0 = 0; t0 < T;) {
        int t1 = t0 + 1;
        while (t1 < T && rows_seq[t1] == rows_seq[t0] && rows_pos[t1] == rows_pos[t1 - 1] + 1) ++t1;
        const int len = rows_pos[t1 - 1] + 1;
        std::vector<float> kc(size_t(len) * KVD), vc(size_t(len) * KVD);
        orc_gather_kv(kc.data(), kp_ref[l].data(), kv, htab, eng->max_pages_per_seq(),
                      ie::hip::kPageSize, rows_seq[t0], len, KVD);
        orc_gather_kv(vc.data(), vp_ref[l].data(), kv, htab, eng->max_pages_per_seq(),
                      ie::hip::kPageSize, rows_seq[t0], len, KVD);
        orc_attention(&want[size_t(t0) * QD], &qr[size_t(t0) * QD], kc.data(), vc.data(), t1 - t0,
                      rows_pos[t0], NH, NKV, HD, threads);
        t0 = t1;
      }
      const std::vector<float> got = download<float>(out[l], want.size());
      double max_abs = 0;
      size_t worst = 0;
      const double rel = orc_compare(got.data(), want.data(), want.size(), &max_abs, &worst);
      const bool ok = kv == IE_KV_F32 ? rel <= 1e-5 : max_abs <= 2e-3;
      char msg[200];
      std::snprintf(msg, sizeof(msg), "%s attention rel %.2e abs %.2e (worst at %zu)", ln.c_str(),
                    rel, max_abs, worst);
      result(ok, msg);
    }
  }

  void prefill(int seq, int T, int want_graph, int want_prompt, int want_fused, const char* what) {
    const int start = eng->sequence_length(seq);
    std::vector<int> rs(T, seq), rp(T);
    for (int i = 0; i < T; ++i) rp[i] = start + i;
    step(what, rs, rp, [&] { eng->prefill(seq, T); }, want_graph, want_prompt, want_fused);
    result(eng->sequence_length(seq) == start + T, std::string(what) + ": length advanced");
  }

  void decode(const std::vector<int>& seqs, const char* what) {
    std::vector<int> rp;
    for (int s : seqs) rp.push_back(eng->sequence_length(s));
    step(what, seqs, rp, [&] { eng->decode(seqs); }, 1, 0, kv != IE_KV_F32);
    bool adv = true;
    for (size_t i = 0; i < seqs.size(); ++i) adv = adv && eng->sequence_length(seqs[i]) == rp[i] + 1;
    result(adv, std::string(what) + ": lengths advanced");
  }

  template <class Op>
  void expect_error(const char* what, const char* needle, Op op) {
    try {
      op();
      result(false, std::string(what) + ": no error raised");
    } catch (const std::exception& e) {
      result(std::strstr(e.what(), needle) != nullptr,
             std::string(what) + ": \"" + e.what() + "\"");
    }
  }
};

}  // namespace

int main(int argc, char** argv) {
  const std::string name = argc > 1 ? argv[1] : "f16";
  const int kv = name == "f32" ? IE_KV_F32 : name == "bf16" ? IE_KV_BF16 : IE_KV_F16;
  std::printf("engine self-test, %s KV cache, %d layers, %d pages\n", name.c_str(), kLayers, kPages);
  std::fflush(stdout);
  try {
    Harness h(kv);
    h.allocate();
    ie::hip::KvConfig cfg;
    cfg.num_layers = kLayers;
    cfg.num_heads = NH;
    cfg.num_kv_heads = NKV;
    cfg.head_dim = HD;
    cfg.rope_theta = kTheta;
    ie::hip::EngineLimits lim;
    lim.max_batch = kMaxBatch;
    lim.max_seq_len = kMaxSeq;
    lim.num_pages = kPages;
    lim.step_rows = kCap;
    KvEngine eng(cfg, lim, kv, /*use_graphs=*/true, h.body());
    h.eng = &eng;
    h.fill_pools();
    std::printf("device: %s\n", eng.device_name().c_str());
    result(eng.total_pages() == kPages && eng.free_pages() == kPages && eng.page_size() == 16,
           "pool: total/free/page size");

    const int s0 = eng.open_sequence(), s1 = eng.open_sequence(), s2 = eng.open_sequence();
    result(s0 == 0 && s1 == 1 && s2 == 2, "open_sequence: lowest free slots");
    const bool f16 = kv != IE_KV_F32;
    // One-row prefill replays the batch-1 decode graph (first token).
    h.prefill(s0, 1, 1, 0, f16, "first token (seq 0, position 0)");
    h.prefill(s0, 62, 0, 1, f16, "prompt continuing at 1 (62 rows)");
    h.decode({s0}, "decode seq 0 at position 63 (chunk edge 63)");
    h.decode({s0}, "decode seq 0 at position 64 (chunk edge 64)");
    h.prefill(s1, 17, 0, 1, f16, "prompt of 17 rows (seq 1)");
    h.prefill(s2, 500, 0, 1, f16, "prompt of 500 rows (seq 2)");
    h.prefill(s2, 40, 0, 1, f16, "prompt continuing at 500 (40 rows)");
    const int s3 = eng.open_sequence();
    h.prefill(s3, 1000, 0, 1, f16, "prompt of 1000 rows (seq 3)");
    h.decode({s0, s1, s2, s3}, "batch of 4 decodes (graph recorded)");
    h.decode({s0, s1, s2, s3}, "batch of 4 decodes (graph replayed)");
    const int graphs = eng.decode_graphs();
    h.decode({s3, s0, s2, s1}, "batch of 4 decodes, rows reordered");
    result(eng.decode_graphs() == graphs, "batch size 4 replays its graph");
    const int s4 = eng.open_sequence();
    h.prefill(s4, 255, 0, 1, f16, "prompt of 255 rows (seq 4)");
    h.decode({s0, s1, s2, s3, s4}, "batch of 5 decodes (seq 4 at position 255)");
    h.decode({s0, s1, s2, s3, s4}, "batch of 5 decodes (seq 4 at position 256)");

    // Mixed step: two decodes and a 30-row prompt of a new sequence, direct.
    const int s5 = eng.open_sequence();
    {
      std::vector<int> rs = {s0, s3}, rp = {eng.sequence_length(s0), eng.sequence_length(s3)};
      for (int p = 0; p < 30; ++p) {
        rs.push_back(s5);
        rp.push_back(p);
      }
      h.step("mixed prefill + decode (32 rows)", rs, rp, [&] { eng.forward(rs, rp); }, 0, 0, 0);
      result(eng.sequence_length(s5) == 30 && eng.sequence_length(s0) == rp[0] + 1,
             "mixed step: lengths advanced");
    }
    result(eng.open_sequence() == -1, "open_sequence: -1 when every slot is busy");

    // Close two sequences; their pages go back to the free list and the next
    // sequence takes them (LIFO), so its rows land on pages with stale data.
    const int before = eng.free_pages();
    std::vector<int32_t> p1(eng.max_pages_per_seq()), p2(eng.max_pages_per_seq());
    const int n1 = eng.sequence_pages(s1, p1.data(), int(p1.size()));
    const int n2 = eng.sequence_pages(s2, p2.data(), int(p2.size()));
    eng.close_sequence(s1);
    eng.close_sequence(s2);
    result(eng.free_pages() == before + n1 + n2 && eng.sequence_length(s1) == 0,
           "close_sequence: pages returned");
    const int s6 = eng.open_sequence();
    result(s6 == s1, "open_sequence: reuses the lowest closed slot");
    h.prefill(s6, 3000, 0, 1, f16, "prompt of 3000 rows on reused pages (seq 1)");
    std::vector<int32_t> p6(eng.max_pages_per_seq());
    eng.sequence_pages(s6, p6.data(), int(p6.size()));
    result(p6[0] == p2[n2 - 1], "reused pages come LIFO (last freed first)");
    h.decode({s0, s6, s3, s4, s5}, "batch of 5 decodes incl. 3000-token context");

    // Errors, as the reference raises them; the engine stays usable.
    h.expect_error("too long", "sequence longer than the maximum",
                   [&] { eng.forward({s0}, {kMaxSeq}); });
    h.expect_error("closed sequence", "invalid or closed sequence id",
                   [&] { eng.decode({s2}); });
    eng.close_sequence(s5);
    const int s7 = eng.open_sequence();
    h.expect_error("pool exhaustion", "KV cache full: no free pages",
                   [&] { eng.prefill(s7, 16 * (eng.free_pages() + 1)); });
    result(eng.free_pages() == 0 && eng.sequence_length(s7) == 0,
           "pool exhaustion: pages taken stay with the sequence, length unchanged");
    eng.close_sequence(s7);
    h.decode({s0, s6, s3, s4}, "batch of 4 decodes after the errors");
    h.prefill(s0, 1, 1, 0, f16, "one-row prefill after the errors");
  } catch (const std::exception& e) {
    std::printf("FAIL exception: %s\n", e.what());
    return 2;
  }
  std::printf("%d checks, %d failures\n", g_tests, g_fail);
  return g_fail ? 1 : 0;
}
