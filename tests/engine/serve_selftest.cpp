// The reference's OpenAI-compatible server (src/server.cpp, its Engine at
// :104-368 started by run_server at :372-409) driven over the MI355X drop-in:
// ie::run_server(*ie::hip::make_batch_runner(...), ...), compiled from the
// reference checkout in place. TEST INFRASTRUCTURE.
//
// Model: the runner self-test's 2-layer decoder of Qwen2.5-0.5B's layer shape
// with a 1,000-token vocabulary and seeded BF16 weights. Tokenizer: a
// tokenizer.json written here for that vocabulary (byte-level BPE, no merges):
// ids 0-93 the printable ASCII characters, 94 the space ("Ġ"), 95-996 tokens
// that decode to "[id]", and the special tokens the server stops on,
// <|endoftext|> 997, <|im_start|> 998, <|im_end|> 999. Every id decodes to its
// own text, so equal reply texts mean equal tokens.
//
// Sequence (one process; the server on a thread, clients on others):
//   1. each of 10 completions requests (greedy, 4..40 tokens) served alone, in turn;
//   2. the same 10 sent at once, plus one streamed request of 200 tokens whose
//      client disconnects after its third chunk;
//   3. every burst reply equals the reply served alone (text, finish reason,
//      token count); /health shows a batch of more than one request, nothing
//      running or waiting, and every KV page free -- the cancelled request's
//      pages went back to the pool.
//
// usage: serve_selftest PORT [f32|f16|bf16]; exit status 0 when every check passes.
#include <httplib.h>

#include <unistd.h>

#include <atomic>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <fstream>
#include <memory>
#include <random>
#include <string>
#include <thread>
#include <vector>

#include <nlohmann/json.hpp>

#include "ie_hip_runner.hpp"
#include "runner.h"     // reference: src/runner.h
#include "server.h"     // reference: src/server.h (run_server)
#include "tokenizer.h"  // reference: src/tokenizer.h

namespace {

using json = nlohmann::json;

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

ie::Weights random_weights(const ie::Config& c, uint32_t seed) {
  std::mt19937 rng(seed);
  std::normal_distribution<float> n01(0.0f, 1.0f);
  auto vec = [&](size_t n, float base, float s) {
    std::vector<float> v(n);
    for (float& e : v) e = base + s * n01(rng);
    return v;
  };
  auto mat = [&](int rows, int cols, float s) {
    return ie::make_matrix(vec(size_t(rows) * cols, 0.0f, s), rows, cols, ie::DType::BF16);
  };
  ie::Weights w;
  w.dtype = ie::DType::BF16;
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

// The tokenizer described at the top, written into dir/tokenizer.json.
void write_tokenizer(const std::string& dir) {
  json vocab = json::object();
  int id = 0;
  for (int ch = '!'; ch <= '~'; ++ch) vocab[std::string(1, char(ch))] = id++;
  vocab["\xC4\xA0"] = id++;  // U+0120 "Ġ": the byte-level stand-in for a space
  for (; id < 997; ++id) vocab["[" + std::to_string(id) + "]"] = id;
  json added = json::array();
  const char* specials[3] = {"<|endoftext|>", "<|im_start|>", "<|im_end|>"};
  for (int i = 0; i < 3; ++i)
    added.push_back({{"id", 997 + i}, {"content", specials[i]}, {"special", true}});
  const json j = {{"model", {{"type", "BPE"}, {"vocab", vocab}, {"merges", json::array()}}},
                  {"added_tokens", added}};
  std::ofstream(dir + "/tokenizer.json") << j.dump();
}

struct Reply {
  int status = 0;
  std::string text, finish;
  int tokens = -1;
  bool operator==(const Reply& o) const {
    return status == o.status && text == o.text && finish == o.finish && tokens == o.tokens;
  }
};

Reply complete(int port, const std::string& prompt, int max_tokens) {
  httplib::Client cli("127.0.0.1", port);
  cli.set_read_timeout(120, 0);
  const json body = {{"prompt", prompt}, {"max_tokens", max_tokens}, {"temperature", 0}};
  Reply r;
  if (auto res = cli.Post("/v1/completions", body.dump(), "application/json")) {
    r.status = res->status;
    if (res->status == 200) {
      const json j = json::parse(res->body);
      r.text = j.at("choices").at(0).at("text").get<std::string>();
      r.finish = j.at("choices").at(0).at("finish_reason").get<std::string>();
      r.tokens = j.at("usage").at("completion_tokens").get<int>();
    } else {
      r.text = res->body;
    }
  }
  return r;
}

json health(int port) {
  httplib::Client cli("127.0.0.1", port);
  cli.set_read_timeout(10, 0);
  if (auto res = cli.Get("/health"))
    if (res->status == 200) return json::parse(res->body);
  return json();
}

}  // namespace

int main(int argc, char** argv) {
  if (argc < 2) {
    std::printf("usage: serve_selftest PORT [f32|f16|bf16]\n");
    return 2;
  }
  const int port = std::atoi(argv[1]);
  const std::string kvs = argc > 2 ? argv[2] : "f16";
  const ie::hip::KvDtype kv = kvs == "f32"    ? ie::hip::KvDtype::F32
                              : kvs == "bf16" ? ie::hip::KvDtype::BF16
                                              : ie::hip::KvDtype::F16;
  std::printf("serve self-test: the reference's run_server over ie::hip::make_batch_runner, %s KV "
              "cache, port %d\n",
              kvs.c_str(), port);
  std::fflush(stdout);
  try {
    if (!ie::hip::device_available()) {
      std::printf("FAIL no HIP device\n");
      return 2;
    }
    char tmpl[] = "/tmp/ie_serve_XXXXXX";
    const char* dir = mkdtemp(tmpl);
    if (!dir) throw std::runtime_error("mkdtemp failed");
    write_tokenizer(dir);
    static const ie::Tokenizer tok(dir);
    const ie::Config cfg = config();
    static std::unique_ptr<ie::BatchRunner> eng =
        ie::hip::make_batch_runner(cfg, random_weights(cfg, 7u), 4, 256, size_t(64) << 20, true, kv);
    result(tok.vocab_size() == V && tok.special_id("<|im_end|>") == 999,
           "tokenizer.json of the model's vocabulary read by the reference's Tokenizer");
    static ie::ServerOptions opt;
    opt.port = port;
    opt.model_id = "ie-hip-test";
    opt.sampling.temperature = 0.0f;  // greedy: the engine's device argmax
    opt.sampling.repetition_penalty = 1.0f;
    std::thread([] {
      try {
        ie::run_server(*eng, tok, opt);
      } catch (const std::exception& e) {
        std::printf("FAIL run_server: %s\n", e.what());
        std::fflush(stdout);
        std::_Exit(3);
      }
    }).detach();
    json h;
    for (int i = 0; i < 600 && h.is_null(); ++i) {
      std::this_thread::sleep_for(std::chrono::milliseconds(100));
      h = health(port);
    }
    result(!h.is_null() && h.value("kv_pages_total", 0) == eng->total_pages(),
           "the server answers /health with the drop-in's page pool");
    if (h.is_null()) std::_Exit(1);

    const std::vector<std::string> words = {"the", "page", "pool", "holds", "keys", "and",
                                            "values", "of", "every", "sequence"};
    std::vector<std::string> prompts;
    std::vector<int> lengths;
    std::mt19937 rng(99);
    for (int i = 0; i < 10; ++i) {
      std::string p;
      const int n = 2 + 3 * i;  // at most 29 words (~150 tokens) + 40 generated: inside 256
      for (int k = 0; k < n; ++k) p += (k ? " " : "") + words[rng() % words.size()];
      prompts.push_back(p);
      lengths.push_back(4 + 4 * i);
    }
    // 1. Each request alone.
    std::vector<Reply> alone;
    for (int i = 0; i < 10; ++i) alone.push_back(complete(port, prompts[i], lengths[i]));
    bool ok = true;
    for (const Reply& r : alone) ok = ok && r.status == 200 && r.tokens > 0;
    result(ok, "10 requests served one at a time");

    // 2. The same 10 at once, and a streamed request cancelled mid-stream.
    std::vector<Reply> burst(10);
    std::atomic<int> chunks{0};
    std::atomic<bool> stream_ended{false};
    std::vector<std::thread> clients;
    clients.emplace_back([&] {
      httplib::Client cli("127.0.0.1", port);
      cli.set_read_timeout(120, 0);
      const json body = {{"prompt", prompts[3]},
                         {"max_tokens", 200},
                         {"temperature", 0},
                         {"stream", true}};
      cli.Post("/v1/completions", httplib::Headers{}, body.dump(), "application/json",
               [&](const char*, size_t) { return ++chunks < 3; });  // false: disconnect
      stream_ended = true;
    });
    for (int i = 0; i < 10; ++i)
      clients.emplace_back([&, i] { burst[i] = complete(port, prompts[i], lengths[i]); });
    for (std::thread& t : clients) t.join();
    int same = 0;
    for (int i = 0; i < 10; ++i) {
      same += burst[i] == alone[i];
      if (!(burst[i] == alone[i]))
        std::printf("     request %d: %d tokens '%s' (%s) alone, %d tokens '%s' (%s) in the burst\n",
                    i, alone[i].tokens, alone[i].text.c_str(), alone[i].finish.c_str(),
                    burst[i].tokens, burst[i].text.c_str(), burst[i].finish.c_str());
    }
    result(same == 10, std::to_string(same) + "/10 burst replies identical to each served alone");
    result(stream_ended && chunks >= 3, "the streamed request's client disconnected after " +
                                            std::to_string(chunks.load()) + " chunks");

    // 3. The engine drains: the cancelled request is dropped at its next step.
    for (int i = 0; i < 300; ++i) {
      h = health(port);
      if (!h.is_null() && h.value("running", -1) == 0 && h.value("waiting", -1) == 0 &&
          h.value("kv_pages_free", -1) == h.value("kv_pages_total", -2))
        break;
      std::this_thread::sleep_for(std::chrono::milliseconds(100));
    }
    std::printf("     /health: %s\n", h.dump().c_str());
    result(h.value("running", -1) == 0 && h.value("waiting", -1) == 0,
           "nothing running or waiting after the burst");
    result(h.value("kv_pages_free", -1) == h.value("kv_pages_total", -2) &&
               eng->free_pages() == eng->total_pages(),
           "every KV page back in the pool (the cancelled request's included)");
    result(h.value("peak_batch", 0) > 1,
           "the burst ran as one batch (peak " + std::to_string(h.value("peak_batch", 0)) + ")");
    result(h.value("requests_served", 0LL) == 21, "21 requests retired (10 + 10 + the cancelled)");
  } catch (const std::exception& e) {
    std::printf("FAIL exception: %s\n", e.what());
    ++g_fail;
  }
  std::printf("%s: %d checks, %d failed\n", g_fail ? "FAILED" : "ALL PASSED", g_tests, g_fail);
  std::fflush(stdout);
  // The server thread never returns: leave without unwinding it.
  std::_Exit(g_fail ? 1 : 0);
}
