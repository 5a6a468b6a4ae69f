/* Continuous batching over any ie::BatchRunner (src/runner.h:52-80), and the
 * check that batching changes nothing: the scheduler of the reference's
 * serve-bench (src/main.cpp:669-751) and its --check (src/main.cpp:845-888).
 *
 * Contract kept from the reference, because --check results depend on it:
 *   - requests are admitted in order, while a sequence slot is free, fewer than
 *     `concurrency` run, and the cache can hold the request at FULL length
 *     (prompt + generated tokens) on top of what running requests reserved;
 *   - an admitted request is prefilled alone and greedy-decoded: its first token
 *     comes from the prefill, every later one from a decode step over all
 *     running requests;
 *   - a request leaves the batch after its last token, and its pages and its
 *     reservation are released at once, so the next request can be admitted in
 *     the same step;
 *   - a request that cannot fit even in an empty cache is an error.
 * On a batch-invariant engine every request's tokens are then the same at any
 * concurrency as served alone, which check_identical() verifies.
 *
 * Header-only C++17; needs the reference's runner.h on the include path. */
#ifndef IE_HIP_SERVE_HPP_
#define IE_HIP_SERVE_HPP_

#include <algorithm>
#include <chrono>
#include <cstdint>
#include <deque>
#include <stdexcept>
#include <string>
#include <vector>

#include "runner.h"

namespace ie::hip {

struct ServeRequest {
  std::vector<int32_t> prompt;
  int gen = 1;  // tokens to generate (>= 1)
};

struct ServeStats {
  std::vector<std::vector<int32_t>> out;  // generated tokens per request
  double seconds = 0, mean_ttft = 0, mean_latency = 0, p95_latency = 0;
  int steps = 0, peak_batch = 0, peak_pages = 0;
  long long tokens = 0;
};

class ContinuousBatcher {
 public:
  ContinuousBatcher(BatchRunner& runner, const std::vector<ServeRequest>& requests, int concurrency)
      : r_(runner), reqs_(requests), concurrency_(std::max(1, concurrency)) {
    stats_.out.resize(reqs_.size());
    ttft_.assign(reqs_.size(), 0.0);
    done_at_.assign(reqs_.size(), 0.0);
  }

  /* Serves every request to completion. */
  ServeStats run() {
    t0_ = Clock::now();
    while (finished_ < reqs_.size()) {
      admit();
      if (running_.empty()) {
        if (next_ < reqs_.size())
          throw std::runtime_error(
              "a request needs more KV-cache pages than the cache has (raise --kv-gb)");
        continue;
      }
      decode_step();
    }
    finish_stats();
    return stats_;
  }

 private:
  using Clock = std::chrono::steady_clock;
  struct Running {
    int seq;
    size_t req;
    int32_t last;  // the token the next step feeds
  };

  int pages_of(const ServeRequest& q) const {
    const int p = r_.page_size();
    return (int(q.prompt.size()) + q.gen + p - 1) / p;
  }
  double now() const { return std::chrono::duration<double>(Clock::now() - t0_).count(); }

  void admit() {
    while (next_ < reqs_.size() && int(running_.size()) < concurrency_ &&
           reserved_ + pages_of(reqs_[next_]) <= r_.total_pages()) {
      const ServeRequest& q = reqs_[next_];
      const int seq = r_.open_sequence();
      if (seq < 0) break;
      const int32_t tok = r_.prefill_greedy(seq, q.prompt);
      ttft_[next_] = now();
      stats_.out[next_].push_back(tok);
      if (q.gen <= 1) {
        r_.close_sequence(seq);
        done_at_[next_] = ttft_[next_];
        ++finished_;
      } else {
        reserved_ += pages_of(q);
        running_.push_back({seq, next_, tok});
      }
      ++next_;
    }
  }

  void decode_step() {
    std::vector<int> seqs;
    std::vector<int32_t> toks;
    for (const Running& a : running_) {
      seqs.push_back(a.seq);
      toks.push_back(a.last);
    }
    stats_.peak_batch = std::max(stats_.peak_batch, int(running_.size()));
    const std::vector<int32_t> nxt = r_.decode_greedy(seqs, toks);
    ++stats_.steps;
    stats_.peak_pages = std::max(stats_.peak_pages, r_.total_pages() - r_.free_pages());
    const double t = now();
    std::vector<Running> keep;
    keep.reserve(running_.size());
    for (size_t i = 0; i < running_.size(); ++i) {
      Running a = running_[i];
      std::vector<int32_t>& o = stats_.out[a.req];
      o.push_back(nxt[i]);
      if (int(o.size()) >= reqs_[a.req].gen) {  // done: out of the batch, pages freed
        r_.close_sequence(a.seq);
        reserved_ -= pages_of(reqs_[a.req]);
        done_at_[a.req] = t;
        ++finished_;
      } else {
        a.last = nxt[i];
        keep.push_back(a);
      }
    }
    running_.swap(keep);
  }

  void finish_stats() {
    stats_.seconds = now();
    const double n = double(reqs_.size());
    for (size_t i = 0; i < reqs_.size(); ++i) {
      stats_.tokens += (long long)stats_.out[i].size();
      stats_.mean_ttft += ttft_[i] / n;
      stats_.mean_latency += done_at_[i] / n;
    }
    std::vector<double> lat = done_at_;
    std::sort(lat.begin(), lat.end());
    if (!lat.empty()) stats_.p95_latency = lat[std::min(lat.size() - 1, size_t(0.95 * lat.size()))];
  }

  BatchRunner& r_;
  const std::vector<ServeRequest>& reqs_;
  int concurrency_;
  ServeStats stats_;
  std::vector<double> ttft_, done_at_;
  std::vector<Running> running_;
  size_t next_ = 0, finished_ = 0;
  int reserved_ = 0;  // pages promised to running requests (their full length)
  Clock::time_point t0_;
};

inline ServeStats serve(BatchRunner& runner, const std::vector<ServeRequest>& requests,
                        int concurrency) {
  return ContinuousBatcher(runner, requests, concurrency).run();
}

/* --check: how many requests produced exactly the reference run's tokens; on
 * the first that did not, which one and from which token. */
struct CheckResult {
  int identical = 0, total = 0, first_request = -1, first_token = -1;
  bool all() const { return identical == total; }
};

inline CheckResult check_identical(const ServeStats& got, const ServeStats& want) {
  CheckResult c;
  c.total = int(want.out.size());
  for (size_t i = 0; i < want.out.size(); ++i) {
    const std::vector<int32_t>& a = got.out.at(i);
    const std::vector<int32_t>& b = want.out[i];
    if (a == b) {
      ++c.identical;
      continue;
    }
    if (c.first_request < 0) {
      c.first_request = int(i);
      size_t k = 0;
      while (k < a.size() && k < b.size() && a[k] == b[k]) ++k;
      c.first_token = int(k);
    }
  }
  return c;
}

}  // namespace ie::hip

#endif  // IE_HIP_SERVE_HPP_
