/* The paged KV-cache engine over the C ABI of libie_hip.so (C++17, header-only;
 * needs hip/hip_runtime_api.h and libamdhip64 for memory, streams and graphs).
 * It is the paged-KV half of what the reference's CudaEngine does
 * (src/cuda/cuda_runner.cu:133-622) -- sequences and their pages, one forward
 * step over token rows, a graph per decode batch size -- built around one idea:
 * every capacity is fixed at construction, so nothing is allocated, resized or
 * re-recorded while serving.
 *
 * Memory. One sizing pass lays out every device region the engine will ever use
 * -- the per-layer K/V pools, the page table, the RoPE table, a step's input
 * rows, its q/k/v/attention rows and the split-K workspace -- and one
 * hipMalloc backs them all (DeviceArena); one pinned block stages a step's
 * inputs. A HIP graph recorded for a batch size therefore stays valid for the
 * engine's life.
 *
 * A step. run() takes rows (sequence, position, token id) and the rows whose
 * logits are wanted. It takes pages for every row, classifies the step (a
 * prompt -- 16+ consecutive positions of one sequence -- runs the prefill
 * kernel; other steps run flash-decoding, with RoPE + append folded into the
 * attention launch for a decode step of a 16-bit cache), packs the inputs into
 * the staging block at offsets that depend only on the row counts, and sends
 * them with ONE copy. A decode step replays its batch size's graph; any other
 * step is enqueued directly. Per layer the model's LayerBody runs its work
 * around the attention; its `begin` and `end` hooks run before the first layer
 * and after the last (the embedding, the final norm and the LM head).
 *
 * Numerics do not depend on the batch: the flash-decoding partition
 * (chunk_tokens) is fixed per engine from its capacity and KV type, and the
 * kernels' reduction orders depend on that partition and each row alone.
 *
 * Not thread-safe: one thread owns an engine, as one engine thread owns a
 * BatchRunner in the reference (src/server.h:9-17). run() only enqueues;
 * sync() waits and surfaces kernel errors. */
#ifndef IE_HIP_ENGINE_HPP_
#define IE_HIP_ENGINE_HPP_

#include <algorithm>
#include <cstring>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "ie_hip.hpp"

namespace ie::hip {

/* The model shape the path reads (the reference's Config, src/config.h:10-26). */
/* A named ROCTX range for the lifetime of the object (ie_hip_range_push/pop). */
struct TraceRange {
  explicit TraceRange(const char* name) { ie_hip_range_push(name); }
  ~TraceRange() { ie_hip_range_pop(); }
  TraceRange(const TraceRange&) = delete;
  TraceRange& operator=(const TraceRange&) = delete;
};

struct KvConfig {
  int num_layers = 24;
  int num_heads = 14;
  int num_kv_heads = 2;
  int head_dim = 64;
  float rope_theta = 1e6f;
  int q_dim() const { return num_heads * head_dim; }
  int kv_dim() const { return num_kv_heads * head_dim; }
};

/* What an engine holds, fixed at construction. */
struct EngineLimits {
  int max_batch = 1;     // sequence slots; a decode step has at most this many rows
  int max_seq_len = 0;   // tokens per sequence
  int num_pages = 0;     // pages in each layer's pool
  int step_rows = 0;     // rows one step holds (0: max(max_batch, min(max_seq_len, 4096)));
                         // a longer prompt runs as several steps
  int logit_rows = 0;    // rows one step may ask logits for (0: max(max_batch, 16))
};

/* The model's work around the engine's attention for a step of `rows` rows,
 * enqueued on `stream` (kernels and device copies only: recorded into the
 * decode graphs). Any of them may be empty. */
struct LayerBody {
  std::function<void(int rows, hipStream_t stream)> begin;
  std::function<void(int layer, int rows, hipStream_t stream)> before_attention;
  std::function<void(int layer, int rows, hipStream_t stream)> after_attention;
  std::function<void(int rows, int logit_rows, hipStream_t stream)> end;
};

/* How a step ran (for callers' logs and the tests). */
struct StepInfo {
  int rows = 0, logit_rows = 0;
  bool graph = false;   // replayed a decode graph
  bool prompt = false;  // prefill attention (rows: consecutive positions of one sequence)
  bool fused = false;   // decode: RoPE + append + attention in one launch per layer;
                        // prompt: q rotated inside the prefill kernel (append of K/V
                        // only; 16-bit caches)
  bool planned = false; // flash-decoding read a host-built work list (ie_hip_attention_plan)
  int chunk_tokens = 0, chunks = 0;  // flash-decoding partition (0 for a prompt)
};

/* One allocation carved into aligned regions: sizes are added first (add()),
 * then commit() makes the single hipMalloc and at() turns an offset into a
 * pointer. Freed as a whole with the arena. */
class DeviceArena {
 public:
  DeviceArena() = default;
  DeviceArena(const DeviceArena&) = delete;
  DeviceArena& operator=(const DeviceArena&) = delete;
  ~DeviceArena() {
    if (base_) (void)hipFree(base_);
  }
  template <class T>
  size_t add(size_t count) {
    const size_t off = (size_ + kAlign - 1) / kAlign * kAlign;
    size_ = off + std::max<size_t>(count, 1) * sizeof(T);
    return off;
  }
  void commit(const char* what) {
    if (base_) throw std::logic_error("DeviceArena: committed twice");
    check(hipMalloc(reinterpret_cast<void**>(&base_), std::max<size_t>(size_, kAlign)), what);
  }
  template <class T>
  T* at(size_t off) const {
    return reinterpret_cast<T*>(base_ + off);
  }
  size_t bytes() const { return size_; }

 private:
  static constexpr size_t kAlign = 256;
  unsigned char* base_ = nullptr;
  size_t size_ = 0;
};

/* Page-locked host memory of a fixed size, for the step's input copy. */
class PinnedBlock {
 public:
  PinnedBlock() = default;
  PinnedBlock(const PinnedBlock&) = delete;
  PinnedBlock& operator=(const PinnedBlock&) = delete;
  ~PinnedBlock() {
    if (p_) (void)hipHostFree(p_);
  }
  void allocate(size_t bytes, const char* what) {
    check(hipHostMalloc(&p_, std::max<size_t>(bytes, 64), hipHostMallocDefault), what);
  }
  template <class T>
  T* as() const {
    return static_cast<T*>(p_);
  }

 private:
  void* p_ = nullptr;
};

class KvEngine {
 public:
  /* Rows a step needs before it counts as a prompt (kPromptMinRows,
   * src/cuda/cuda_runner.cu:38). */
  static constexpr int kPromptMinRows = 16;

  /* Pages for a KV byte budget: as many as fit, never more than every
   * sequence at full length (make_batch_runner, src/cuda/cuda_runner.cu:612-622). */
  static int pages_for_budget(const KvConfig& cfg, int max_batch, int max_seq_len,
                              size_t kv_bytes, int kv_dtype) {
    const size_t page_bytes =
        size_t(2) * kPageSize * cfg.kv_dim() * kv_elem_bytes(kv_dtype) * cfg.num_layers;
    const size_t want = std::max<size_t>(1, kv_bytes / page_bytes);
    const size_t most = size_t(max_batch) * size_t(ie_pages_for(max_seq_len));
    return int(std::min(want, most));
  }

  KvEngine(const KvConfig& cfg, const EngineLimits& limits, int kv_dtype, bool use_graphs,
           LayerBody body = {})
      : cfg_(cfg), lim_(limits), kv_dtype_(kv_dtype), use_graphs_(use_graphs),
        body_(std::move(body)) {
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_F16 && kv_dtype != IE_KV_BF16)
      throw std::runtime_error("KV cache: dtype must be IE_KV_F32, IE_KV_F16 or IE_KV_BF16");
    if (cfg.num_layers < 1 || cfg.num_heads < 1 || cfg.num_kv_heads < 1 || cfg.head_dim < 2)
      throw std::runtime_error("KV cache: bad model shape");
    if (lim_.max_batch < 1 || lim_.max_seq_len < 1) throw std::runtime_error("KV cache: bad limits");
    if (lim_.num_pages < 1) throw std::runtime_error("KV cache: no pages");
    if (lim_.step_rows <= 0) lim_.step_rows = std::max(lim_.max_batch, std::min(lim_.max_seq_len, 4096));
    if (lim_.logit_rows <= 0) lim_.logit_rows = std::max(lim_.max_batch, kPromptMinRows);
    lim_.step_rows = std::max(lim_.step_rows, lim_.max_batch);
    lim_.logit_rows = std::max(lim_.logit_rows, lim_.max_batch);

    // The flash-decoding partition, fixed for the engine's life: sized for a
    // full batch of the longest sequences, so a step's numerics never depend on
    // which rows it carries.
    chunk_tokens_ = attention_chunk_tokens(lim_.max_batch, lim_.max_seq_len, kv_dtype_);
    max_chunks_ = attention_chunks(lim_.max_seq_len, chunk_tokens_);
    attn_rows_ = std::max(lim_.max_batch, kPromptMinRows);  // rows per flash-decoding launch
    // A step of up to attn_rows_ flash-decoding rows sends, with its inputs, the
    // work list the 16-bit kernel would otherwise locate on the device (row
    // positions -> the row's table -> K/V): built here from host data, it cuts
    // that chain to one load.
    plan_ints_ = attention_plan_ints(attn_rows_, max_chunks_, chunk_tokens_);

    pages_ = ie_pages_create(lim_.num_pages, lim_.max_batch, lim_.max_seq_len);
    if (!pages_) throw std::runtime_error(ie_hip_last_error());
    try {
      max_pages_per_seq_ = ie_pages_max_pages_per_seq(pages_);
      int dev = 0;
      check(hipGetDevice(&dev), "hipGetDevice");  // the device this engine's memory lives on
      hipDeviceProp_t prop{};
      check(hipGetDeviceProperties(&prop, dev), "hipGetDeviceProperties");
      static const char* const kKv[] = {"", ", f16 KV cache", ", bf16 KV cache"};
      // The marketing name is empty where the driver's id table is missing.
      name_ = std::string("hip, ") + (prop.name[0] ? prop.name : "AMD GPU") + " (" +
              prop.gcnArchName + ")" +
              (use_graphs_ ? ", graphs" : ", no graphs") + kKv[kv_dtype];
      check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
      check(hipEventCreateWithFlags(&staged_, hipEventDisableTiming), "hipEventCreate");

      // Layout: pools, table, RoPE table, step inputs, step rows, workspace.
      const int R = lim_.step_rows;
      layer_bytes_ = size_t(lim_.num_pages) * kPageSize * cfg.kv_dim() * kv_elem_bytes(kv_dtype);
      const size_t o_pools = arena_.add<unsigned char>(2 * layer_bytes_ * cfg.num_layers);
      const size_t o_tables = arena_.add<int32_t>(size_t(lim_.max_batch) * max_pages_per_seq_);
      const size_t o_rope = arena_.add<float>(size_t(lim_.max_seq_len) * cfg.head_dim);
      const size_t o_in = arena_.add<int32_t>(input_ints());
      const size_t o_q = arena_.add<float>(size_t(R) * cfg.q_dim());
      const size_t o_k = arena_.add<float>(size_t(R) * cfg.kv_dim());
      const size_t o_v = arena_.add<float>(size_t(R) * cfg.kv_dim());
      const size_t o_attn = arena_.add<float>(size_t(R) * cfg.q_dim());
      const size_t o_ws = arena_.add<unsigned char>(
          attention_workspace_bytes(attn_rows_, cfg.num_heads, cfg.head_dim, max_chunks_));
      arena_.commit("hipMalloc(KV engine)");
      pools_ = arena_.at<unsigned char>(o_pools);
      tables_ = arena_.at<int32_t>(o_tables);
      rope_ = arena_.at<float>(o_rope);
      inputs_ = arena_.at<int32_t>(o_in);
      q_ = arena_.at<float>(o_q);
      k_ = arena_.at<float>(o_k);
      v_ = arena_.at<float>(o_v);
      attn_ = arena_.at<float>(o_attn);
      workspace_ = arena_.at<unsigned char>(o_ws);
      staging_.allocate(input_ints() * sizeof(int32_t), "hipHostMalloc(step inputs)");

      // The RoPE table, built on the host with libm exactly as the reference's
      // CPU rope computes its angles, so page writes match it bit for bit.
      std::vector<float> table(size_t(lim_.max_seq_len) * cfg.head_dim);
      check(ie_hip_rope_table(table.data(), lim_.max_seq_len, cfg.head_dim, cfg.rope_theta));
      check(hipMemcpy(rope_, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice),
            "RoPE table");
      // The device table starts as the host one does (zero-filled).
      check(ie_pages_upload_tables(pages_, tables_, stream_, nullptr));
      check(hipStreamSynchronize(stream_), "KV engine setup");
    } catch (...) {
      release();
      throw;
    }
  }
  KvEngine(const KvEngine&) = delete;
  KvEngine& operator=(const KvEngine&) = delete;
  ~KvEngine() { release(); }

  // ---------------------------------------------- sequences and the pool

  int open_sequence() { return ie_pages_open_sequence(pages_); }
  void close_sequence(int seq) { check(ie_pages_close_sequence(pages_, seq)); }
  /* Tokens cached for seq: 0 for a closed slot, std::out_of_range past the slots
   * (the reference reads seqs_.at(seq).len, src/cuda/cuda_runner.cu:254). */
  int sequence_length(int seq) const {
    if (seq < 0 || seq >= lim_.max_batch) throw std::out_of_range("sequence id " + std::to_string(seq));
    return std::max(ie_pages_sequence_length(pages_, seq), 0);
  }
  bool is_open(int seq) const { return ie_pages_sequence_length(pages_, seq) >= 0; }
  int max_batch() const { return lim_.max_batch; }
  int max_seq_len() const { return lim_.max_seq_len; }
  int page_size() const { return kPageSize; }
  int total_pages() const { return ie_pages_total_pages(pages_); }
  int free_pages() const { return ie_pages_free_pages(pages_); }
  const KvConfig& config() const { return cfg_; }
  const EngineLimits& limits() const { return lim_; }
  std::string device_name() const { return name_; }
  size_t kv_cache_bytes() const { return 2 * layer_bytes_ * size_t(cfg_.num_layers); }

  // ----------------------------------------------------------- a step

  /* Queues one forward step over rows (seq[t], pos[t]) with token ids ids[t]
   * (may be empty when the LayerBody reads none) and logits wanted for rows
   * `logit_rows` (indices into the step's rows). `decode`: one row per
   * sequence, which may replay this batch size's graph. `after_layer` (direct
   * steps only) runs on the host after each layer's work is queued, and with
   * layer -1 after the body's `begin` (the embedding). Returns
   * without waiting; sync() waits. Each listed sequence's length becomes its
   * highest row position + 1 if that is longer. */
  StepInfo run(const std::vector<int>& seq, const std::vector<int>& pos,
               const std::vector<int32_t>& ids, const std::vector<int>& logit_rows, bool decode,
               const std::function<void(int layer)>& after_layer = nullptr) {
    const int T = int(seq.size()), R = int(logit_rows.size());
    if (T == 0) throw std::runtime_error("forward: no tokens");
    if (int(pos.size()) != T) throw std::runtime_error("forward: one position per row");
    if (!ids.empty() && int(ids.size()) != T) throw std::runtime_error("forward: one token per row");
    if (T > lim_.step_rows)
      throw std::runtime_error("forward: " + std::to_string(T) + " rows in one step (at most " +
                               std::to_string(lim_.step_rows) + ")");
    if (R > lim_.logit_rows) throw std::runtime_error("forward: too many logit rows in one step");
    for (int r : logit_rows)
      if (r < 0 || r >= T) throw std::runtime_error("forward: logit row out of range");
    int max_pos = 0;
    for (int t = 0; t < T; ++t) {
      if (pos[t] < 0) throw std::runtime_error("forward: negative position");
      if (!is_open(seq[t]))
        throw std::runtime_error("invalid or closed sequence id " + std::to_string(seq[t]));
      check(ie_pages_ensure(pages_, seq[t], pos[t] + 1));
      max_pos = std::max(max_pos, pos[t]);
    }
    const bool distinct = distinct_sequences(seq);
    if (decode && !distinct) throw std::runtime_error("decode: one row per sequence");

    StepInfo s;
    s.rows = T;
    s.logit_rows = R;
    s.graph = decode && use_graphs_ && !after_layer && T <= lim_.max_batch;
    s.prompt = !decode && T >= kPromptMinRows &&
               attention_prefill_supported(cfg_.num_heads, cfg_.num_kv_heads, cfg_.head_dim);
    for (int t = 1; s.prompt && t < T; ++t)
      s.prompt = seq[t] == seq[0] && pos[t] == pos[0] + t;
    if (s.prompt) {
      s.fused = rope_cache_attention_prefill_supported(kv_dtype_, cfg_.num_heads,
                                                       cfg_.num_kv_heads, cfg_.head_dim);
    } else {
      s.chunk_tokens = chunk_tokens_;
      // A recorded graph covers any position a sequence can reach; a direct
      // step only the context it has (the count does not change the sums).
      s.chunks = s.graph ? max_chunks_ : attention_chunks(max_pos + 1, chunk_tokens_);
      s.fused = distinct && rope_cache_attention_supported(kv_dtype_, cfg_.num_heads,
                                                           cfg_.num_kv_heads, cfg_.head_dim,
                                                           chunk_tokens_);
    }

    // Inputs: [seq T][pos T][ids T][logit rows R][work list], one copy. The
    // offsets depend only on T and R, so a decode graph (one per T and R) reads
    // them where it recorded.
    check(hipEventSynchronize(staged_), "staging");  // the previous step's copy is done
    int32_t* h = staging_.as<int32_t>();
    std::copy(seq.begin(), seq.end(), h);
    std::copy(pos.begin(), pos.end(), h + T);
    if (ids.empty())
      std::fill(h + 2 * T, h + 3 * T, 0);
    else
      std::copy(ids.begin(), ids.end(), h + 2 * T);
    std::copy(logit_rows.begin(), logit_rows.end(), h + 3 * T);
    size_t n_in = 3 * size_t(T) + R;
    s.planned = !s.prompt && plan_ints_ > 0 && T <= attn_rows_;
    if (s.planned) {
      const size_t off = plan_offset(T, R);
      attention_plan(h + off, plan_ints_, T, pos.data(), seq.data(),
                     ie_pages_host_tables(pages_), lim_.max_batch, max_pages_per_seq_, s.chunks,
                     s.chunk_tokens);
      n_in = off + 4 + size_t(h[off]) * ((plan_ints_ - 4) / (size_t(attn_rows_) * max_chunks_));
    }
    check(hipMemcpyAsync(inputs_, h, sizeof(int32_t) * n_in, hipMemcpyHostToDevice, stream_),
          "step inputs");
    check(hipEventRecord(staged_, stream_), "hipEventRecord");
    check(ie_pages_upload_tables(pages_, tables_, stream_, nullptr));  // only after page changes

    cur_rows_ = T;
    cur_logit_rows_ = R;
    // The step on the ROCTX timeline, named as the reference names its NVTX
    // ranges (src/cuda/cuda_runner.cu:349): one prompt, one row, several rows.
    const TraceRange range(s.prompt   ? "prefill"
                           : !decode  ? "mixed step"
                           : T == 1   ? "decode"
                                      : "decode batch");
    if (s.graph) {
      auto it = graphs_.find({T, R});
      if (it == graphs_.end()) it = graphs_.emplace(std::make_pair(T, R), record(s)).first;
      check(hipGraphLaunch(it->second, stream_), "hipGraphLaunch");
    } else {
      enqueue(s, after_layer);
    }
    for (int t = 0; t < T; ++t)
      if (pos[t] + 1 > ie_pages_sequence_length(pages_, seq[t]))
        check(ie_pages_set_sequence_length(pages_, seq[t], pos[t] + 1));
    last_ = s;
    return s;
  }

  /* Waits for the queued work; kernel faults surface here (the reference's
   * per-step synchronize, src/cuda/cuda_runner.cu:397-398). */
  void sync() { check(hipStreamSynchronize(stream_), "forward"); }

  // Steps without a model (the tests drive attention with their own q/k/v):

  /* T prompt rows appended to seq; one row replays the batch-1 decode graph. */
  void prefill(int seq, int T) {
    if (T <= 0) throw std::runtime_error("forward: no tokens");
    const int start = checked_length(seq);
    std::vector<int> rs(T, seq), rp(T);
    for (int i = 0; i < T; ++i) rp[i] = start + i;
    run(rs, rp, {}, {}, /*decode=*/T == 1);
    sync();
  }
  /* One new row for each listed sequence (a decode step). */
  void decode(const std::vector<int>& seqs) {
    std::vector<int> rp(seqs.size());
    for (size_t i = 0; i < seqs.size(); ++i) rp[i] = checked_length(seqs[i]);
    run(seqs, rp, {}, {}, /*decode=*/true);
    sync();
  }
  /* Any mix of rows in one direct step. */
  void forward(const std::vector<int>& seq, const std::vector<int>& pos) {
    run(seq, pos, {}, {}, /*decode=*/false);
    sync();
  }

  // ------------------------------ the current step's buffers (for the body)

  int32_t* ids() { return inputs_ + 2 * size_t(cur_rows_); }         // [rows]
  int32_t* logit_row_ids() { return inputs_ + 3 * size_t(cur_rows_); }  // [logit rows]
  float* q() { return q_; }        // [rows, q_dim]: the layer's queries
  float* k() { return k_; }        // [rows, kv_dim]: the layer's new keys
  float* v() { return v_; }        // [rows, kv_dim]: the layer's new values
  float* attn() { return attn_; }  // [rows, q_dim]: the layer's attention output
  hipStream_t stream() const { return stream_; }

  // ------------------------------------------------------- inspection

  const StepInfo& last_step() const { return last_; }
  int decode_graphs() const { return int(graphs_.size()); }
  int chunk_tokens() const { return chunk_tokens_; }
  /* Replaces the model's per-layer work; graphs recorded with the old one go. */
  void set_body(LayerBody body) {
    body_ = std::move(body);
    drop_graphs();
  }
  int max_pages_per_seq() const { return max_pages_per_seq_; }
  const int32_t* host_tables() const { return ie_pages_host_tables(pages_); }
  const int32_t* device_tables() const { return tables_; }
  size_t layer_pool_bytes() const { return layer_bytes_; }
  void* k_pool(int layer) { return pools_ + size_t(2 * layer) * layer_bytes_; }
  void* v_pool(int layer) { return pools_ + size_t(2 * layer + 1) * layer_bytes_; }
  int kv_dtype() const { return kv_dtype_; }
  size_t device_bytes() const { return arena_.bytes(); }
  int sequence_pages(int seq, int32_t* out, int cap) const {
    return ie_pages_sequence_pages(pages_, seq, out, cap);
  }

 private:
  /* The step's inputs, then (16-byte aligned) the work list of a planned step. */
  static size_t plan_offset(int T, int R) { return (3 * size_t(T) + size_t(R) + 3) & ~size_t(3); }
  size_t input_ints() const {
    return plan_offset(lim_.step_rows, lim_.logit_rows) + plan_ints_;
  }

  static bool distinct_sequences(const std::vector<int>& seq) {
    std::vector<int> s(seq);
    std::sort(s.begin(), s.end());
    return std::adjacent_find(s.begin(), s.end()) == s.end();
  }

  int checked_length(int seq) const {
    const int len = ie_pages_sequence_length(pages_, seq);
    if (len < 0) throw std::runtime_error("invalid or closed sequence id " + std::to_string(seq));
    return len;
  }

  KvLayout layout() const {
    KvLayout kv;
    kv.tables = tables_;
    kv.max_pages = max_pages_per_seq_;
    kv.page_size = kPageSize;
    kv.kv_dtype = kv_dtype_;
    kv.num_pages = lim_.num_pages;
    return kv;
  }

  /* Every layer of a step on stream_ (the reference's per-layer order,
   * src/cuda/cuda_runner.cu:418-446, with the model's work in the body).
   * Flash-decoding runs in launches of at most attn_rows_ rows, the rows the
   * workspace holds; a prompt runs the prefill kernel over all its rows. */
  void enqueue(const StepInfo& s, const std::function<void(int)>& after_layer) {
    const int T = s.rows, NH = cfg_.num_heads, NKV = cfg_.num_kv_heads, HD = cfg_.head_dim;
    const KvLayout kv = layout();
    const int32_t* rseq = inputs_;
    const int32_t* rpos = inputs_ + T;
    if (body_.begin) body_.begin(T, stream_);
    if (after_layer) after_layer(-1);
    for (int l = 0; l < cfg_.num_layers; ++l) {
      if (body_.before_attention) body_.before_attention(l, T, stream_);
      void* kp = k_pool(l);
      void* vp = v_pool(l);
      const int32_t* plan = inputs_ + plan_offset(T, s.logit_rows);
      if (s.prompt && s.fused) {
        rope_cache_attention_prefill(attn_, q_, k_, v_, kp, vp, rope_, lim_.max_seq_len, T, rpos,
                                     rseq, kv, NH, NKV, HD, stream_);
      } else if (s.fused && s.planned) {
        rope_cache_attention_planned(attn_, q_, k_, v_, kp, vp, rope_, lim_.max_seq_len, T, rpos,
                                     rseq, kv, s.chunks, s.chunk_tokens, workspace_, plan,
                                     plan_ints_, NH, NKV, HD, stream_);
      } else if (s.fused) {
        for (int r0 = 0; r0 < T; r0 += attn_rows_) {
          const int n = std::min(attn_rows_, T - r0);
          rope_cache_attention(attn_ + size_t(r0) * cfg_.q_dim(), q_ + size_t(r0) * cfg_.q_dim(),
                               k_ + size_t(r0) * cfg_.kv_dim(), v_ + size_t(r0) * cfg_.kv_dim(),
                               kp, vp, rope_, lim_.max_seq_len, n, rpos + r0, rseq + r0, kv,
                               s.chunks, s.chunk_tokens, workspace_, NH, NKV, HD, stream_);
        }
      } else {
        rope_and_cache(q_, k_, v_, kp, vp, rope_, lim_.max_seq_len, T, rpos, rseq, kv, NH, NKV,
                       HD, stream_);
        if (s.prompt) {
          attention_prefill(attn_, q_, kp, vp, T, rpos, rseq, kv, NH, NKV, HD, stream_);
        } else if (s.planned) {
          attention_planned(attn_, q_, kp, vp, T, rpos, rseq, kv, s.chunks, s.chunk_tokens,
                            workspace_, plan, plan_ints_, NH, NKV, HD, stream_);
        } else {
          for (int r0 = 0; r0 < T; r0 += attn_rows_) {
            const int n = std::min(attn_rows_, T - r0);
            attention(attn_ + size_t(r0) * cfg_.q_dim(), q_ + size_t(r0) * cfg_.q_dim(), kp, vp, n,
                      rpos + r0, rseq + r0, kv, s.chunks, s.chunk_tokens, workspace_, NH, NKV, HD,
                      stream_);
          }
        }
      }
      if (body_.after_attention) body_.after_attention(l, T, stream_);
      if (after_layer) after_layer(l);
    }
    if (body_.end) body_.end(T, s.logit_rows, stream_);
  }

  /* Records one decode step of s.rows sequences into a graph. */
  hipGraphExec_t record(const StepInfo& s) {
    const TraceRange range("record decode graph");
    hipGraph_t graph = nullptr;
    check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
      enqueue(s, nullptr);
    } catch (...) {
      (void)hipStreamEndCapture(stream_, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      throw;
    }
    check(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t err = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    check(err, "hipGraphInstantiate");
    return exec;
  }

  void drop_graphs() {
    for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second);
    graphs_.clear();
  }

  void release() {
    drop_graphs();
    if (stream_) (void)hipStreamSynchronize(stream_);
    if (staged_) (void)hipEventDestroy(staged_);
    staged_ = nullptr;
    if (stream_) (void)hipStreamDestroy(stream_);
    stream_ = nullptr;
    if (pages_) ie_pages_destroy(pages_);
    pages_ = nullptr;
  }

  KvConfig cfg_;
  EngineLimits lim_;
  int kv_dtype_;
  bool use_graphs_;
  LayerBody body_;
  std::string name_;
  int chunk_tokens_ = 0, max_chunks_ = 0, attn_rows_ = 0, max_pages_per_seq_ = 0;
  size_t plan_ints_ = 0;  // capacity of a step's work list

  ie_page_pool* pages_ = nullptr;  // free list, sequences, host page table
  DeviceArena arena_;
  PinnedBlock staging_;
  hipStream_t stream_ = nullptr;
  hipEvent_t staged_ = nullptr;    // the last input copy
  std::map<std::pair<int, int>, hipGraphExec_t> graphs_;  // decode graphs by (rows, logit rows)
  StepInfo last_;
  int cur_rows_ = 0, cur_logit_rows_ = 0;

  size_t layer_bytes_ = 0;
  unsigned char* pools_ = nullptr;  // [layer][K | V][page][row][kv_dim]
  int32_t* tables_ = nullptr;       // device copy of the page table
  float* rope_ = nullptr;           // [max_seq_len, head_dim] cos | sin
  int32_t* inputs_ = nullptr;       // the step's packed inputs
  float *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_ = nullptr;
  unsigned char* workspace_ = nullptr;  // flash-decoding partials
};

}  // namespace ie::hip

#endif  // IE_HIP_ENGINE_HPP_
