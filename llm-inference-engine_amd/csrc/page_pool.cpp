// Page allocator behind BatchRunner: page pool, LIFO free list, per-sequence
// page lists and the page table (host side).
//
// Reference: CudaEngine (src/cuda/cuda_runner.cu) -- ctor free list :197,
// tables :199-204, open_sequence :240-247, close_sequence :248-252,
// slot() :290-294, ensure_pages :300-313, dirty-table upload :379-383,
// pages_for :583. Semantics kept: page 0 is handed out first; a closed
// sequence's pages go back on the free list in the order it owned them (so the
// next sequence reuses its last page first); table entries are not cleared on
// close; the table is re-uploaded only after a sequence gained a page.
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "common.hpp"

struct ie_page_pool {
  struct Sequence {
    bool open = false;
    int len = 0;
    std::vector<int32_t> pages;
  };
  int num_pages = 0, max_batch = 0, max_seq_len = 0, max_pages = 0;
  std::vector<int32_t> free_list;  // back() is handed out next
  std::vector<int32_t> tables;     // [max_batch * max_pages]
  std::vector<Sequence> seqs;
  bool dirty = true;
  int32_t* staging = nullptr;       // pinned copy of `tables` for async uploads
  hipEvent_t staged = nullptr;      // the last upload from `staging`
};

namespace {

using iehip::clear_error;
using iehip::fail;

int slot(const ie_page_pool* pool, int seq) {
  if (!pool) return fail(IE_HIP_EINVAL, "null page pool");
  if (seq < 0 || seq >= pool->max_batch || !pool->seqs[seq].open)
    return fail(IE_HIP_ESEQ, "invalid or closed sequence id " + std::to_string(seq));
  return IE_HIP_OK;
}

}  // namespace

extern "C" {

int ie_pages_for(int tokens) {
  return tokens <= 0 ? 0 : (tokens + IE_HIP_PAGE_SIZE - 1) / IE_HIP_PAGE_SIZE;
}

ie_page_pool* ie_pages_create(int num_pages, int max_batch, int max_seq_len) {
  clear_error();
  if (num_pages < 1) {
    fail(IE_HIP_EINVAL, "KV cache: no pages");
    return nullptr;
  }
  if (max_batch < 1 || max_seq_len < 1) {
    fail(IE_HIP_EINVAL, "page pool: max_batch and max_seq_len must be positive");
    return nullptr;
  }
  auto* p = new ie_page_pool;
  p->num_pages = num_pages;
  p->max_batch = max_batch;
  p->max_seq_len = max_seq_len;
  p->max_pages = ie_pages_for(max_seq_len);
  p->free_list.reserve(num_pages);
  for (int i = num_pages - 1; i >= 0; --i) p->free_list.push_back(i);
  p->tables.assign(size_t(max_batch) * p->max_pages, 0);
  p->seqs.resize(max_batch);
  return p;
}

void ie_pages_destroy(ie_page_pool* pool) {
  if (!pool) return;
  if (pool->staged) {
    (void)hipEventSynchronize(pool->staged);
    (void)hipEventDestroy(pool->staged);
  }
  if (pool->staging) (void)hipHostFree(pool->staging);
  delete pool;
}

int ie_pages_open_sequence(ie_page_pool* pool) {
  clear_error();
  if (!pool) return -1;
  for (int s = 0; s < pool->max_batch; ++s)
    if (!pool->seqs[s].open) {
      pool->seqs[s] = ie_page_pool::Sequence{};
      pool->seqs[s].open = true;
      return s;
    }
  return -1;
}

int ie_pages_close_sequence(ie_page_pool* pool, int seq) {
  clear_error();
  if (int rc = slot(pool, seq)) return rc;
  auto& sq = pool->seqs[seq];
  for (int32_t page : sq.pages) pool->free_list.push_back(page);
  sq = ie_page_pool::Sequence{};
  return IE_HIP_OK;
}

int ie_pages_ensure(ie_page_pool* pool, int seq, int len) {
  clear_error();
  if (int rc = slot(pool, seq)) return rc;
  auto& sq = pool->seqs[seq];
  if (len > pool->max_seq_len)
    return fail(IE_HIP_ERANGE, "sequence longer than the maximum (" +
                                   std::to_string(pool->max_seq_len) + " tokens)");
  while (int(sq.pages.size()) * IE_HIP_PAGE_SIZE < len) {
    if (pool->free_list.empty()) return fail(IE_HIP_EFULL, "KV cache full: no free pages");
    const int32_t page = pool->free_list.back();
    pool->free_list.pop_back();
    pool->tables[size_t(seq) * pool->max_pages + sq.pages.size()] = page;
    sq.pages.push_back(page);
    pool->dirty = true;
  }
  return IE_HIP_OK;
}

int ie_pages_sequence_length(const ie_page_pool* pool, int seq) {
  if (!pool || seq < 0 || seq >= pool->max_batch || !pool->seqs[seq].open) return -1;
  return pool->seqs[seq].len;
}

int ie_pages_set_sequence_length(ie_page_pool* pool, int seq, int len) {
  clear_error();
  if (int rc = slot(pool, seq)) return rc;
  if (len < 0 || len > pool->max_seq_len)
    return fail(IE_HIP_ERANGE, "sequence longer than the maximum (" +
                                   std::to_string(pool->max_seq_len) + " tokens)");
  pool->seqs[seq].len = len;
  return IE_HIP_OK;
}

int ie_pages_sequence_pages(const ie_page_pool* pool, int seq, int32_t* out, int cap) {
  if (!pool || seq < 0 || seq >= pool->max_batch || !pool->seqs[seq].open) return 0;
  const auto& pages = pool->seqs[seq].pages;
  const int n = std::min<int>(int(pages.size()), std::max(cap, 0));
  if (out && n > 0) std::memcpy(out, pages.data(), size_t(n) * sizeof(int32_t));
  return int(pages.size());
}

int ie_pages_total_pages(const ie_page_pool* pool) { return pool ? pool->num_pages : 0; }
int ie_pages_free_pages(const ie_page_pool* pool) { return pool ? int(pool->free_list.size()) : 0; }
int ie_pages_max_batch(const ie_page_pool* pool) { return pool ? pool->max_batch : 0; }
int ie_pages_max_seq_len(const ie_page_pool* pool) { return pool ? pool->max_seq_len : 0; }
int ie_pages_max_pages_per_seq(const ie_page_pool* pool) { return pool ? pool->max_pages : 0; }
const int32_t* ie_pages_host_tables(const ie_page_pool* pool) {
  return pool ? pool->tables.data() : nullptr;
}

int ie_pages_upload_tables(ie_page_pool* pool, int32_t* device_tables, hipStream_t stream,
                           int* uploaded) {
  clear_error();
  if (uploaded) *uploaded = 0;
  if (!pool || !device_tables) return fail(IE_HIP_EINVAL, "upload_tables: null pointer");
  if (!pool->dirty) return IE_HIP_OK;
  const size_t bytes = pool->tables.size() * sizeof(int32_t);
  if (!pool->staging) {
    void* p = nullptr;
    if (int rc = iehip::check_hip(hipHostMalloc(&p, bytes, hipHostMallocDefault), "hipHostMalloc"))
      return rc;
    pool->staging = static_cast<int32_t*>(p);
    if (int rc = iehip::check_hip(hipEventCreateWithFlags(&pool->staged, hipEventDisableTiming),
                                  "hipEventCreate"))
      return rc;
  } else if (int rc = iehip::check_hip(hipEventSynchronize(pool->staged), "hipEventSynchronize")) {
    return rc;  // the previous upload must have left the staging buffer
  }
  std::memcpy(pool->staging, pool->tables.data(), bytes);
  if (int rc = iehip::check_hip(
          hipMemcpyAsync(device_tables, pool->staging, bytes, hipMemcpyHostToDevice, stream),
          "page table upload"))
    return rc;
  if (int rc = iehip::check_hip(hipEventRecord(pool->staged, stream), "hipEventRecord")) return rc;
  pool->dirty = false;
  if (uploaded) *uploaded = 1;
  return IE_HIP_OK;
}

}  // extern "C"
