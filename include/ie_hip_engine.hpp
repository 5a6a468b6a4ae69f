/* The paged KV-cache half of the reference's CudaEngine
 * (src/cuda/cuda_runner.cu:133-622), in C++17 over the C ABI of libie_hip.so:
 *   - sequences and their pages (open_sequence, close_sequence, ensure_pages,
 *     the page table and its dirty upload), through ie_page_pool;
 *   - the per-layer pools, the RoPE table, the step's row buffers and the
 *     split-K workspace, sized before any graph is recorded (reserve);
 *   - one forward step over token rows (run): prompt detection, the chunk
 *     partition, and per layer RoPE + paged append then prefill or
 *     flash-decoding attention (enqueue), or both in one launch for a decode
 *     step of a 16-bit cache;
 *   - one HIP graph per decode batch size (capture_graph).
 * The model's own per-layer work (projections before attention, o_proj and the
 * MLP after it) is the caller's: a LayerBody whose two callbacks enqueue that
 * work on the engine's stream around each layer's attention. They write the
 * step's q, k, v rows (q(), k(), v()) and read attn(), and are recorded into
 * the decode graphs with everything else.
 *
 * Header-only; needs hip/hip_runtime_api.h and libamdhip64 for memory, streams
 * and graphs. Not thread-safe: one thread owns an engine, as one engine thread
 * owns a BatchRunner in the reference (src/server.h:9-17). Every step is
 * synchronous on return (src/cuda/cuda_runner.cu:397-398). */
#ifndef IE_HIP_ENGINE_HPP_
#define IE_HIP_ENGINE_HPP_

#include <algorithm>
#include <cstring>
#include <functional>
#include <map>
#include <stdexcept>
#include <string>
#include <vector>

#include "ie_hip.hpp"

namespace ie::hip {

/* The model shape the path reads (the reference's Config, src/config.h:10-26). */
struct KvConfig {
  int num_layers = 24;
  int num_heads = 14;
  int num_kv_heads = 2;
  int head_dim = 64;
  float rope_theta = 1e6f;
  int q_dim() const { return num_heads * head_dim; }
  int kv_dim() const { return num_kv_heads * head_dim; }
};

/* The model's work around layer `layer`'s attention for a step of `rows` rows,
 * enqueued on `stream` (kernels and device-to-device copies only: the body is
 * recorded into decode graphs). Either may be empty. */
struct LayerBody {
  std::function<void(int layer, int rows, hipStream_t stream)> before_attention;
  std::function<void(int layer, int rows, hipStream_t stream)> after_attention;
};

/* How the last step ran (for callers' logs and the tests). */
struct StepInfo {
  int rows = 0;
  bool graph = false;   // replayed a decode graph
  bool prompt = false;  // prefill attention (rows: consecutive positions of one sequence)
  bool fused = false;   // RoPE + append + attention in one launch per layer
  int chunk_tokens = 0, chunks = 0;  // flash-decoding partition (0 for a prompt)
};

/* Device allocations owned by the engine, freed with it (DeviceMemory,
 * src/cuda/cuda_runner.cu:51-96). */
class DeviceMemory {
 public:
  DeviceMemory() = default;
  DeviceMemory(const DeviceMemory&) = delete;
  DeviceMemory& operator=(const DeviceMemory&) = delete;
  ~DeviceMemory() {
    for (void* p : ptrs_) (void)hipFree(p);
  }
  template <class T>
  T* alloc(size_t n) {
    void* p = nullptr;
    check(hipMalloc(&p, std::max<size_t>(n * sizeof(T), 256)), "hipMalloc");
    ptrs_.push_back(p);
    return static_cast<T*>(p);
  }
  void release(void* p) {
    auto it = std::find(ptrs_.begin(), ptrs_.end(), p);
    if (it == ptrs_.end()) return;
    (void)hipFree(p);
    ptrs_.erase(it);
  }

 private:
  std::vector<void*> ptrs_;
};

/* Page-locked host staging that only grows (PinnedBuffer, src/cuda/cuda_runner.cu:100-122). */
template <class T>
class PinnedBuffer {
 public:
  PinnedBuffer() = default;
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  ~PinnedBuffer() { reset(); }
  void resize(size_t n) {
    if (n <= n_) return;
    reset();
    void* p = nullptr;
    check(hipHostMalloc(&p, n * sizeof(T), hipHostMallocDefault), "hipHostMalloc");
    p_ = static_cast<T*>(p);
    n_ = n;
  }
  T* data() { return p_; }

 private:
  void reset() {
    if (p_) (void)hipHostFree(p_);
    p_ = nullptr;
    n_ = 0;
  }
  T* p_ = nullptr;
  size_t n_ = 0;
};

class KvEngine {
 public:
  /* Rows a step needs before it counts as a prompt (kPromptMinRows,
   * src/cuda/cuda_runner.cu:38). */
  static constexpr int kPromptMinRows = 16;

  /* Pages for a KV byte budget: as many as fit, but never more than every
   * sequence at full length (make_batch_runner, src/cuda/cuda_runner.cu:612-622). */
  static int pages_for_budget(const KvConfig& cfg, int max_batch, int max_seq_len,
                              size_t kv_bytes, int kv_dtype) {
    const size_t page_bytes =
        size_t(2) * kPageSize * cfg.kv_dim() * kv_elem_bytes(kv_dtype) * cfg.num_layers;
    const size_t want = std::max<size_t>(1, kv_bytes / page_bytes);
    const size_t most = size_t(max_batch) * size_t(ie_pages_for(max_seq_len));
    return int(std::min(want, most));
  }

  /* The constructor of src/cuda/cuda_runner.cu:146-204, less the weights:
   * pools for every layer, the page table, the RoPE table (built on the host,
   * so page writes match the CPU path bit for bit) and the stream. */
  KvEngine(const KvConfig& cfg, int max_batch, int max_seq_len, int num_pages, bool use_graphs,
           int kv_dtype, LayerBody body = {})
      : cfg_(cfg), max_batch_(max_batch), max_seq_len_(max_seq_len), num_pages_(num_pages),
        use_graphs_(use_graphs), kv_dtype_(kv_dtype), body_(std::move(body)) {
    if (kv_dtype != IE_KV_F32 && kv_dtype != IE_KV_F16 && kv_dtype != IE_KV_BF16)
      throw std::runtime_error("KV cache: dtype must be IE_KV_F32, IE_KV_F16 or IE_KV_BF16");
    if (cfg.num_layers < 1 || cfg.num_heads < 1 || cfg.num_kv_heads < 1 || cfg.head_dim < 2)
      throw std::runtime_error("KV cache: bad model shape");
    pages_ = ie_pages_create(num_pages, max_batch, max_seq_len);
    if (!pages_) throw std::runtime_error(ie_hip_last_error());
    try {
      max_pages_per_seq_ = ie_pages_max_pages_per_seq(pages_);
      hipDeviceProp_t prop{};
      check(hipGetDeviceProperties(&prop, 0), "hipGetDeviceProperties");
      static const char* const kNames[] = {"", ", f16 KV cache", ", bf16 KV cache"};
      name_ = std::string("hip, ") + prop.name + " (" + prop.gcnArchName + ")" +
              (use_graphs_ ? ", graphs" : ", no graphs") + kNames[kv_dtype];
      check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");

      std::vector<float> table(size_t(max_seq_len) * cfg.head_dim);
      check(ie_hip_rope_table(table.data(), max_seq_len, cfg.head_dim, cfg.rope_theta));
      rope_table_ = mem_.alloc<float>(table.size());
      check(hipMemcpy(rope_table_, table.data(), table.size() * sizeof(float),
                      hipMemcpyHostToDevice),
            "rope table");

      layer_bytes_ = size_t(num_pages_) * kPageSize * cfg.kv_dim() * kv_elem_bytes(kv_dtype);
      k_pool_ = mem_.alloc<unsigned char>(layer_bytes_ * cfg.num_layers);
      v_pool_ = mem_.alloc<unsigned char>(layer_bytes_ * cfg.num_layers);
      tables_ = mem_.alloc<int32_t>(size_t(max_batch) * max_pages_per_seq_);
    } catch (...) {
      release();
      throw;
    }
  }
  KvEngine(const KvEngine&) = delete;
  KvEngine& operator=(const KvEngine&) = delete;
  ~KvEngine() { release(); }

  // ----------------------------------------- BatchRunner (src/runner.h:52-80)

  int open_sequence() { return ie_pages_open_sequence(pages_); }
  void close_sequence(int seq) { check(ie_pages_close_sequence(pages_, seq)); }
  /* Tokens cached for seq: 0 for a closed slot, std::out_of_range past the
   * slots (seqs_.at(seq).len, src/cuda/cuda_runner.cu:254). */
  int sequence_length(int seq) const {
    if (seq < 0 || seq >= max_batch_) throw std::out_of_range("sequence id " + std::to_string(seq));
    return std::max(ie_pages_sequence_length(pages_, seq), 0);
  }
  int max_batch() const { return max_batch_; }
  int max_seq_len() const { return max_seq_len_; }
  int page_size() const { return kPageSize; }
  int total_pages() const { return ie_pages_total_pages(pages_); }
  int free_pages() const { return ie_pages_free_pages(pages_); }
  const KvConfig& config() const { return cfg_; }
  std::string device_name() const { return name_; }
  size_t kv_cache_bytes() const { return 2 * layer_bytes_ * size_t(cfg_.num_layers); }

  /* Appends T prompt rows to seq (run_prefill, src/cuda/cuda_runner.cu:315-323):
   * one row replays the batch-1 decode graph; 16 or more run the prefill
   * attention kernel. */
  void prefill(int seq, int T) {
    if (T <= 0) throw std::runtime_error("forward: no tokens");
    const int start = checked_length(seq);
    std::vector<int> rows_seq(T, seq), rows_pos(T);
    for (int i = 0; i < T; ++i) rows_pos[i] = start + i;
    run(rows_seq, rows_pos, /*graph=*/T == 1);
    check(ie_pages_set_sequence_length(pages_, seq, start + T));
  }

  /* One new row for each listed sequence, replaying the decode graph of that
   * batch size (run_decode, src/cuda/cuda_runner.cu:325-337). */
  void decode(const std::vector<int>& seqs) {
    std::vector<int> rows_pos(seqs.size());
    for (size_t i = 0; i < seqs.size(); ++i) rows_pos[i] = checked_length(seqs[i]);
    run(seqs, rows_pos, /*graph=*/true);
    for (size_t i = 0; i < seqs.size(); ++i)
      check(ie_pages_set_sequence_length(pages_, seqs[i], rows_pos[i] + 1));
  }

  /* Any mix of rows (prompt chunks and decodes of several sequences) in one
   * direct step; each sequence's length becomes its highest row position + 1
   * if that is longer. */
  void forward(const std::vector<int>& rows_seq, const std::vector<int>& rows_pos) {
    run(rows_seq, rows_pos, /*graph=*/false);
    for (size_t t = 0; t < rows_seq.size(); ++t)
      if (rows_pos[t] + 1 > ie_pages_sequence_length(pages_, rows_seq[t]))
        check(ie_pages_set_sequence_length(pages_, rows_seq[t], rows_pos[t] + 1));
  }

  // ------------------------------------------ the step's device buffers

  float* q() { return q_; }        // [rows, q_dim]: the layer's queries (RoPE in place, or not read back)
  float* k() { return k_; }        // [rows, kv_dim]: the layer's new keys
  float* v() { return v_; }        // [rows, kv_dim]: the layer's new values
  float* attn() { return attn_; }  // [rows, q_dim]: the layer's attention output
  hipStream_t stream() const { return stream_; }
  int row_capacity() const { return cap_rows_; }

  // --------------------------------------------------------- inspection

  const StepInfo& last_step() const { return last_; }
  int decode_graphs() const { return int(graphs_.size()); }
  /* Replaces the model's per-layer work (for a body that needs the engine
   * itself, as DecoderModel's does); recorded decode graphs are dropped. */
  void set_body(LayerBody body) {
    body_ = std::move(body);
    drop_graphs();
  }
  int max_pages_per_seq() const { return max_pages_per_seq_; }
  const int32_t* host_tables() const { return ie_pages_host_tables(pages_); }
  const int32_t* device_tables() const { return tables_; }
  size_t layer_pool_bytes() const { return layer_bytes_; }
  void* k_pool(int layer) { return k_pool_ + size_t(layer) * layer_bytes_; }
  void* v_pool(int layer) { return v_pool_ + size_t(layer) * layer_bytes_; }
  int kv_dtype() const { return kv_dtype_; }
  int sequence_pages(int seq, int32_t* out, int cap) const {
    return ie_pages_sequence_pages(pages_, seq, out, cap);
  }

  /* One forward step over rows (rows_seq[t], rows_pos[t]) -- the path part of
   * CudaEngine::run (src/cuda/cuda_runner.cu:342-399): pages for every row,
   * prompt detection, the chunk partition, scratch sized before any capture,
   * the row and table uploads, then the decode graph or a direct enqueue, and
   * a synchronize that surfaces kernel errors. `graph`: a pure decode step (one
   * row per sequence) that may replay a recording. Sequence lengths are left
   * to the caller (prefill/decode/forward advance them). */
  void run(const std::vector<int>& rows_seq, const std::vector<int>& rows_pos, bool graph) {
    const int T = int(rows_seq.size());
    if (T == 0) throw std::runtime_error("forward: no tokens");
    if (int(rows_pos.size()) != T) throw std::runtime_error("forward: one position per row");
    int max_pos = 0;
    for (int t = 0; t < T; ++t) {
      if (rows_pos[t] < 0) throw std::runtime_error("forward: negative position");
      check(ie_pages_ensure(pages_, rows_seq[t], rows_pos[t] + 1));
      max_pos = std::max(max_pos, rows_pos[t]);
    }
    graph = graph && use_graphs_;
    std::vector<int> sorted(rows_seq);
    std::sort(sorted.begin(), sorted.end());
    const bool distinct = std::adjacent_find(sorted.begin(), sorted.end()) == sorted.end();
    if (graph && !distinct) throw std::runtime_error("decode: one row per sequence");

    // A prompt (16+ consecutive positions of one sequence) runs the prefill
    // kernel; the choice depends only on the rows themselves.
    bool prompt = !graph && T >= kPromptMinRows &&
                  attention_prefill_supported(cfg_.num_heads, cfg_.num_kv_heads, cfg_.head_dim);
    for (int t = 1; prompt && t < T; ++t)
      prompt = rows_seq[t] == rows_seq[0] && rows_pos[t] == rows_pos[0] + t;

    StepInfo s;
    s.rows = T;
    s.graph = graph;
    s.prompt = prompt;
    if (!prompt) {
      // A recorded graph covers every position a sequence can reach; a direct
      // launch only the context it has.
      const int ctx = graph ? max_seq_len_ : max_pos + 1;
      s.chunk_tokens = attention_chunk_tokens(T, ctx, kv_dtype_);
      s.chunks = attention_chunks(ctx, s.chunk_tokens);
      s.fused = distinct && rope_cache_attention_supported(kv_dtype_, cfg_.num_heads,
                                                           cfg_.num_kv_heads, cfg_.head_dim,
                                                           s.chunk_tokens);
    }
    reserve(T, s.chunks);  // before any capture: no allocation may happen inside a graph
    if (graph && !graphs_.count(T)) capture_graph(s);

    std::memcpy(h_row_seq_.data(), rows_seq.data(), sizeof(int) * T);
    std::memcpy(h_row_pos_.data(), rows_pos.data(), sizeof(int) * T);
    check(hipMemcpyAsync(row_seq_, h_row_seq_.data(), sizeof(int) * T, hipMemcpyHostToDevice,
                         stream_),
          "row_seq");
    check(hipMemcpyAsync(row_pos_, h_row_pos_.data(), sizeof(int) * T, hipMemcpyHostToDevice,
                         stream_),
          "row_pos");
    check(ie_pages_upload_tables(pages_, tables_, stream_, nullptr));  // only if a page changed

    if (graph)
      check(hipGraphLaunch(graphs_.at(T), stream_), "hipGraphLaunch");
    else
      enqueue(s);
    check(hipStreamSynchronize(stream_), "forward");
    last_ = s;
  }

 private:
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
    kv.num_pages = num_pages_;
    return kv;
  }

  /* Every layer of a step on stream_ (the attention block of
   * src/cuda/cuda_runner.cu:418-446, around the caller's LayerBody). */
  void enqueue(const StepInfo& s) {
    const int T = s.rows, NH = cfg_.num_heads, NKV = cfg_.num_kv_heads, HD = cfg_.head_dim;
    const KvLayout kv = layout();
    for (int l = 0; l < cfg_.num_layers; ++l) {
      if (body_.before_attention) body_.before_attention(l, T, stream_);
      void* kp = k_pool(l);
      void* vp = v_pool(l);
      if (s.fused) {
        rope_cache_attention(attn_, q_, k_, v_, kp, vp, rope_table_, max_seq_len_, T, row_pos_,
                             row_seq_, kv, s.chunks, s.chunk_tokens, workspace_, NH, NKV, HD,
                             stream_);
      } else {
        rope_and_cache(q_, k_, v_, kp, vp, rope_table_, max_seq_len_, T, row_pos_, row_seq_, kv,
                       NH, NKV, HD, stream_);
        if (s.prompt)
          attention_prefill(attn_, q_, kp, vp, T, row_pos_, row_seq_, kv, NH, NKV, HD, stream_);
        else
          attention(attn_, q_, kp, vp, T, row_pos_, row_seq_, kv, s.chunks, s.chunk_tokens,
                    workspace_, NH, NKV, HD, stream_);
      }
      if (body_.after_attention) body_.after_attention(l, T, stream_);
    }
  }

  /* Records one decode step of s.rows sequences (capture_graph,
   * src/cuda/cuda_runner.cu:470-487). */
  void capture_graph(const StepInfo& s) {
    hipGraph_t graph = nullptr;
    check(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
    try {
      enqueue(s);
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
    graphs_[s.rows] = exec;
  }

  void drop_graphs() {
    for (auto& g : graphs_) (void)hipGraphExecDestroy(g.second);
    graphs_.clear();
  }

  /* Row buffers for T rows and the split-K workspace for `chunks`, grown on
   * demand; recorded graphs hold the old addresses, so growth drops them
   * (reserve, src/cuda/cuda_runner.cu:492-541). */
  void reserve(int T, int chunks) {
    if (T > cap_rows_) {
      drop_graphs();
      for (void* p : {(void*)row_seq_, (void*)row_pos_, (void*)q_, (void*)k_, (void*)v_,
                      (void*)attn_})
        mem_.release(p);
      cap_rows_ = std::max(T, 16);
      const size_t n = size_t(cap_rows_);
      row_seq_ = mem_.alloc<int>(n);
      row_pos_ = mem_.alloc<int>(n);
      q_ = mem_.alloc<float>(n * cfg_.q_dim());
      k_ = mem_.alloc<float>(n * cfg_.kv_dim());
      v_ = mem_.alloc<float>(n * cfg_.kv_dim());
      attn_ = mem_.alloc<float>(n * cfg_.q_dim());
      h_row_seq_.resize(n);
      h_row_pos_.resize(n);
    }
    const size_t ws = chunks > 0
        ? attention_workspace_bytes(T, cfg_.num_heads, cfg_.head_dim, chunks) : 0;
    if (ws > cap_ws_) {
      drop_graphs();
      mem_.release(workspace_);
      workspace_ = mem_.alloc<unsigned char>(ws);
      cap_ws_ = ws;
    }
  }

  void release() {
    drop_graphs();
    if (stream_) (void)hipStreamDestroy(stream_);
    stream_ = nullptr;
    if (pages_) ie_pages_destroy(pages_);
    pages_ = nullptr;
  }

  KvConfig cfg_;
  int max_batch_ = 1, max_seq_len_ = 0, num_pages_ = 0, max_pages_per_seq_ = 0;
  bool use_graphs_ = true;
  int kv_dtype_ = IE_KV_F32;
  LayerBody body_;
  std::string name_;
  DeviceMemory mem_;
  hipStream_t stream_ = nullptr;
  std::map<int, hipGraphExec_t> graphs_;  // decode graphs by batch size
  StepInfo last_;

  ie_page_pool* pages_ = nullptr;  // free list, sequences, host page table
  int32_t* tables_ = nullptr;      // device copy of the page table
  float* rope_table_ = nullptr;    // [max_seq_len, head_dim] cos | sin
  unsigned char *k_pool_ = nullptr, *v_pool_ = nullptr;  // [layer][page][row][kv_dim]
  size_t layer_bytes_ = 0;

  int cap_rows_ = 0;
  size_t cap_ws_ = 0;
  int *row_seq_ = nullptr, *row_pos_ = nullptr;
  float *q_ = nullptr, *k_ = nullptr, *v_ = nullptr, *attn_ = nullptr;
  unsigned char* workspace_ = nullptr;  // flash-decoding partials (part_o + part_ml)
  PinnedBuffer<int> h_row_seq_, h_row_pos_;
};

}  // namespace ie::hip

#endif  // IE_HIP_ENGINE_HPP_
