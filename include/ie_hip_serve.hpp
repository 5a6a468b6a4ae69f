/* A continuous-batching scheduler over any ie::BatchRunner (src/runner.h:52-80),
 * and the comparison serve-bench's --check makes (src/main.cpp:845-888).
 *
 * What a caller may rely on (serve-bench --check depends on it):
 *   - Requests start in the order given. A request starts only when one of the
 *     scheduler's `max_running` slots is empty and the page ledger can promise
 *     it every page it will ever hold: ceil((prompt + tokens to generate) /
 *     page size), counted against the runner's total_pages() on top of the
 *     promises of requests still running. A request that waits holds back the
 *     ones behind it.
 *   - A starting request runs its prompt through prefill_greedy on its own; that
 *     gives its first token. Every later token comes from one decode_greedy step
 *     over all running requests together.
 *   - After its last token a request's sequence is closed and its promise
 *     returned to the ledger before the next requests start, so a slot and its
 *     pages are reused within the same round.
 *   - A request that could not fit even in an empty cache is refused before any
 *     request runs.
 * On an engine whose rows do not depend on the batch around them (make_batch_runner
 * is one), every request then gets the same tokens at every max_running as when
 * served alone, which tokens_match() counts.
 *
 * Header-only C++17; needs the reference's runner.h on the include path. */
#ifndef IE_HIP_SERVE_HPP_
#define IE_HIP_SERVE_HPP_

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "runner.h"

namespace ie::hip {

struct ServeRequest {
  std::vector<int32_t> prompt;
  int gen = 1;  // tokens to generate; the prefill's token is the first (at least 1)
};

/* One request's history. Times are seconds since serve() began. */
struct RequestTrace {
  std::vector<int32_t> tokens;  // greedy tokens in order, the prefill's first
  double first_token_s = 0;
  double finished_s = 0;
};

struct ServeReport {
  std::vector<RequestTrace> requests;  // in the order they were given
  double wall_s = 0;
  int decode_steps = 0;
  int largest_batch = 0;       // most requests in one decode step
  int most_pages_in_use = 0;   // total_pages() - free_pages(), after a step

  long long tokens() const {
    long long n = 0;
    for (const RequestTrace& r : requests) n += (long long)r.tokens.size();
    return n;
  }
  double mean_first_token_s() const { return mean_of(&RequestTrace::first_token_s); }
  double mean_finished_s() const { return mean_of(&RequestTrace::finished_s); }
  /* Nearest-rank 95th percentile of the finish times: the smallest time by
   * which at least 95% of the requests had finished. */
  double p95_finished_s() const {
    if (requests.empty()) return 0;
    std::vector<double> t;
    t.reserve(requests.size());
    for (const RequestTrace& r : requests) t.push_back(r.finished_s);
    const size_t rank = size_t(std::ceil(0.95 * double(t.size())));
    const size_t k = std::max<size_t>(rank, 1) - 1;
    std::nth_element(t.begin(), t.begin() + k, t.end());
    return t[k];
  }

 private:
  double mean_of(double RequestTrace::*field) const {
    if (requests.empty()) return 0;
    double s = 0;
    for (const RequestTrace& r : requests) s += r.*field;
    return s / double(requests.size());
  }
};

class BatchScheduler {
 public:
  BatchScheduler(BatchRunner& runner, int max_running)
      : runner_(runner), slots_(size_t(std::max(1, max_running))) {}

  /* Serves every request to its last token and returns what each produced. */
  ServeReport serve(const std::vector<ServeRequest>& requests) {
    const int capacity = runner_.total_pages();
    for (size_t i = 0; i < requests.size(); ++i)
      if (pages_for(requests[i]) > capacity)
        throw std::runtime_error("serve: request " + std::to_string(i) + " needs " +
                                 std::to_string(pages_for(requests[i])) +
                                 " KV-cache pages at full length; the cache has " +
                                 std::to_string(capacity) + " (raise --kv-gb)");
    report_ = ServeReport{};
    report_.requests.resize(requests.size());
    for (Slot& s : slots_) s = Slot{};
    queued_ = 0;
    promised_ = 0;
    started_ = Clock::now();

    size_t done = 0;
    while (done < requests.size()) {
      done += start_waiting(requests);
      if (occupied() == 0) {
        if (done < requests.size())
          throw std::runtime_error("serve: no sequence could be opened with nothing running "
                                   "(the runner's sequence slots are held elsewhere)");
        break;
      }
      done += step_all(requests);
    }
    report_.wall_s = elapsed();
    return report_;
  }

 private:
  using Clock = std::chrono::steady_clock;

  // A running request: which one, its sequence, the token its next step feeds
  // and the pages promised to it.
  struct Slot {
    int request = -1;  // -1: empty
    int seq = -1;
    int32_t feed = 0;
    int pages = 0;
  };

  int pages_for(const ServeRequest& q) const {
    const int n = int(q.prompt.size()) + std::max(q.gen, 1);
    return (n + runner_.page_size() - 1) / runner_.page_size();
  }
  double elapsed() const { return std::chrono::duration<double>(Clock::now() - started_).count(); }
  int occupied() const {
    int n = 0;
    for (const Slot& s : slots_) n += s.request >= 0;
    return n;
  }

  // Starts queued requests in order into empty slots while the ledger allows.
  // Returns how many of them finished at their prefill (one-token requests).
  size_t start_waiting(const std::vector<ServeRequest>& requests) {
    size_t finished = 0;
    for (Slot& s : slots_) {
      while (s.request < 0 && queued_ < requests.size()) {
        const ServeRequest& q = requests[queued_];
        const int pages = pages_for(q);
        if (promised_ + pages > runner_.total_pages()) return finished;
        const int seq = runner_.open_sequence();
        if (seq < 0) return finished;
        const int id = int(queued_++);
        RequestTrace& tr = report_.requests[size_t(id)];
        const int32_t first = runner_.prefill_greedy(seq, q.prompt);
        tr.tokens.assign(1, first);
        tr.first_token_s = elapsed();
        if (q.gen <= 1) {  // nothing to decode: the slot stays empty
          runner_.close_sequence(seq);
          tr.finished_s = tr.first_token_s;
          ++finished;
          continue;
        }
        s = Slot{id, seq, first, pages};
        promised_ += pages;
      }
      if (queued_ == requests.size()) break;
    }
    return finished;
  }

  // One decode step over every occupied slot, then the requests it completed
  // give back their slots and pages. Returns how many completed.
  size_t step_all(const std::vector<ServeRequest>& requests) {
    std::vector<int> seqs;
    std::vector<int32_t> feeds;
    std::vector<Slot*> order;
    for (Slot& s : slots_)
      if (s.request >= 0) {
        seqs.push_back(s.seq);
        feeds.push_back(s.feed);
        order.push_back(&s);
      }
    const std::vector<int32_t> next = runner_.decode_greedy(seqs, feeds);
    if (next.size() != order.size())
      throw std::runtime_error("serve: decode_greedy returned " + std::to_string(next.size()) +
                               " tokens for " + std::to_string(order.size()) + " sequences");
    ++report_.decode_steps;
    report_.largest_batch = std::max(report_.largest_batch, int(order.size()));
    report_.most_pages_in_use =
        std::max(report_.most_pages_in_use, runner_.total_pages() - runner_.free_pages());
    const double now = elapsed();
    size_t completed = 0;
    for (size_t k = 0; k < order.size(); ++k) {
      Slot& s = *order[k];
      RequestTrace& tr = report_.requests[size_t(s.request)];
      tr.tokens.push_back(next[k]);
      if (int(tr.tokens.size()) < requests[size_t(s.request)].gen) {
        s.feed = next[k];
        continue;
      }
      runner_.close_sequence(s.seq);
      promised_ -= s.pages;
      tr.finished_s = now;
      s = Slot{};
      ++completed;
    }
    return completed;
  }

  BatchRunner& runner_;
  std::vector<Slot> slots_;
  ServeReport report_;
  size_t queued_ = 0;   // requests before this index have started
  int promised_ = 0;    // pages the ledger has promised to running requests
  Clock::time_point started_;
};

inline ServeReport serve(BatchRunner& runner, const std::vector<ServeRequest>& requests,
                         int max_running) {
  return BatchScheduler(runner, max_running).serve(requests);
}

/* --check: requests whose tokens equal the reference report's, and where the
 * first mismatch is (request, token index), or -1, -1. */
struct TokenMatch {
  int same = 0, total = 0, first_request = -1, first_token = -1;
  bool all() const { return same == total; }
};

inline TokenMatch tokens_match(const ServeReport& got, const ServeReport& want) {
  TokenMatch m;
  m.total = int(want.requests.size());
  for (size_t i = 0; i < want.requests.size(); ++i) {
    static const std::vector<int32_t> none;
    const std::vector<int32_t>& a = i < got.requests.size() ? got.requests[i].tokens : none;
    const std::vector<int32_t>& b = want.requests[i].tokens;
    const auto diff = std::mismatch(a.begin(), a.end(), b.begin(), b.end());
    if (diff.first == a.end() && diff.second == b.end()) {
      ++m.same;
    } else if (m.first_request < 0) {
      m.first_request = int(i);
      m.first_token = int(diff.first - a.begin());
    }
  }
  return m;
}

}  // namespace ie::hip

#endif  // IE_HIP_SERVE_HPP_
