// CPU oracle for the paged KV-cache path. TEST INFRASTRUCTURE ONLY: the HIP
// library never links this file; tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py load it as the checker. See oracle.h for what
// pins each function.
//
// Build: oracle/Makefile (g++ -O3 -mavx2 -mfma -ffp-contract=off).
#include "oracle.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <condition_variable>
#include <cstring>
#include <fstream>
#include <functional>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <utility>
#include <vector>

#include <immintrin.h>

namespace {

// ------------------------------------------------------------ thread pool ---
// The reference's pool semantics (src/threadpool.cpp:27-90): `n` threads in
// total including the caller, [0, n) split evenly as chunk i = [n*i/T,
// n*(i+1)/T), the caller runs chunk 0, workers spin ~200 us before sleeping.
class Pool {
 public:
  explicit Pool(int threads) : n_threads_(std::max(1, threads)) {
    for (int i = 1; i < n_threads_; ++i) workers_.emplace_back([this, i] { worker(i); });
  }
  ~Pool() {
    {
      std::lock_guard<std::mutex> g(mu_);
      stop_ = true;
      gen_.fetch_add(1);
    }
    cv_.notify_all();
    for (auto& t : workers_) t.join();
  }
  int threads() const { return n_threads_; }
  void run(int64_t n, const std::function<void(int64_t, int64_t)>& fn) {
    if (n <= 0) return;
    if (n_threads_ == 1 || n == 1) {
      fn(0, n);
      return;
    }
    fn_ = &fn;
    n_ = n;
    pending_.store(n_threads_ - 1, std::memory_order_relaxed);
    {
      std::lock_guard<std::mutex> g(mu_);
      gen_.fetch_add(1, std::memory_order_release);
    }
    cv_.notify_all();
    chunk(0);
    while (pending_.load(std::memory_order_acquire) != 0) _mm_pause();
  }

 private:
  void chunk(int i) {
    const int64_t b = n_ * i / n_threads_, e = n_ * (i + 1) / n_threads_;
    if (b < e) (*fn_)(b, e);
  }
  void worker(int i) {
    uint64_t seen = 0;
    for (;;) {
      uint64_t g = gen_.load(std::memory_order_acquire);
      if (g == seen) {
        const auto until = std::chrono::steady_clock::now() + std::chrono::microseconds(200);
        while ((g = gen_.load(std::memory_order_acquire)) == seen &&
               std::chrono::steady_clock::now() < until)
          for (int k = 0; k < 64; ++k) _mm_pause();
        if (g == seen) {
          std::unique_lock<std::mutex> lk(mu_);
          cv_.wait(lk, [&] { return gen_.load(std::memory_order_acquire) != seen; });
          g = gen_.load(std::memory_order_acquire);
        }
      }
      seen = g;
      if (stop_) return;
      chunk(i);
      pending_.fetch_sub(1, std::memory_order_acq_rel);
    }
  }
  int n_threads_;
  std::vector<std::thread> workers_;
  const std::function<void(int64_t, int64_t)>* fn_ = nullptr;
  int64_t n_ = 0;
  std::atomic<uint64_t> gen_{0};
  std::atomic<int> pending_{0};
  bool stop_ = false;
  std::mutex mu_;
  std::condition_variable cv_;
};

Pool& pool_with(int threads) {
  static std::unique_ptr<Pool> pool;
  static std::mutex mu;
  std::lock_guard<std::mutex> g(mu);
  if (!pool || pool->threads() != threads) pool = std::make_unique<Pool>(threads);
  return *pool;
}

size_t kv_elem_bytes(int dtype) { return dtype == ORC_KV_F32 ? 4 : 2; }

float load_kv(const void* pool, size_t i, int dtype) {
  if (dtype == ORC_KV_F32) return static_cast<const float*>(pool)[i];
  const uint16_t h = static_cast<const uint16_t*>(pool)[i];
  return dtype == ORC_KV_F16 ? orc_f16_to_f32(h) : orc_bf16_to_f32(h);
}

void store_kv(void* pool, size_t i, float x, int dtype) {
  if (dtype == ORC_KV_F32)
    static_cast<float*>(pool)[i] = x;
  else
    static_cast<uint16_t*>(pool)[i] = dtype == ORC_KV_F16 ? orc_f32_to_f16(x) : orc_f32_to_bf16(x);
}

// One head's rotation at one position, src/ops.cpp:45-53 with GCC's
// contraction written out.
inline void rotate_head(float* v, const float* cos_i, const float* sin_i, int half) {
  for (int i = 0; i < half; ++i) {
    const float c = cos_i[i], s = sin_i[i];
    const float x0 = v[i], x1 = v[i + half];
    v[i] = std::fma(x0, c, -(x1 * s));
    v[i + half] = std::fma(x1, c, x0 * s);
  }
}

// The dot product of src/ops.cpp:91-92 as GCC -O3 -mavx2 -mfma compiles it:
// the products of each 8-wide (then one 4-wide) block are rounded separately
// (vmulps) and added to the running sum in index order (vaddss); only the
// scalar tail of fewer than 4 elements is fused (vfmadd231ss).
inline float dot_as_compiled(const float* a, const float* b, int n) {
  float dot = 0.0f;
  int d = 0;
  for (; d + 8 <= n; d += 8)
    for (int j = 0; j < 8; ++j) dot = dot + a[d + j] * b[d + j];
  if (n - d >= 4) {
    for (int j = 0; j < 4; ++j) dot = dot + a[d + j] * b[d + j];
    d += 4;
  }
  for (; d < n; ++d) dot = std::fma(a[d], b[d], dot);
  return dot;
}

// The per-(head, token) body of src/ops.cpp:80-104. The value loop is fused
// (vfmadd213ps / vfmadd213ss), one fma per element in position order.
void attend_one(float* ot, const float* qt, const float* k, const float* v, int p, int kvh,
                size_t kv_stride, int head_dim, float scale, float* scores) {
  for (int s = 0; s <= p; ++s) {
    const float* ks = k + size_t(s) * kv_stride + size_t(kvh) * head_dim;
    scores[s] = dot_as_compiled(qt, ks, head_dim) * scale;
  }
  orc_softmax(scores, p + 1);
  for (int d = 0; d < head_dim; ++d) ot[d] = 0.0f;
  for (int s = 0; s <= p; ++s) {
    const float* vs = v + size_t(s) * kv_stride + size_t(kvh) * head_dim;
    const float w = scores[s];
    for (int d = 0; d < head_dim; ++d) ot[d] = std::fma(w, vs[d], ot[d]);
  }
}

}  // namespace

extern "C" {

void orc_inv_freq(float* inv_freq, int head_dim, float theta) {
  const int half = head_dim / 2;
  for (int i = 0; i < half; ++i)
    inv_freq[i] = 1.0f / powf(theta, float(2 * i) / float(head_dim));
}

void orc_rope_table(float* table, int n_pos, int head_dim, float theta) {
  const int half = head_dim / 2;
  std::vector<float> inv(half);
  orc_inv_freq(inv.data(), head_dim, theta);
  for (int p = 0; p < n_pos; ++p) {
    const float pos = float(p);
    float* row = table + size_t(p) * head_dim;
    for (int i = 0; i < half; ++i) {
      const float angle = pos * inv[i];
      row[i] = cosf(angle);
      row[half + i] = sinf(angle);
    }
  }
}

void orc_rope(float* x, int T, int n_heads, int head_dim, int pos0, float theta) {
  const int half = head_dim / 2;
  std::vector<float> inv(half), c(half), s(half);
  orc_inv_freq(inv.data(), head_dim, theta);
  for (int t = 0; t < T; ++t) {
    const float pos = float(pos0 + t);
    for (int i = 0; i < half; ++i) {
      const float angle = pos * inv[i];
      c[i] = cosf(angle);
      s[i] = sinf(angle);
    }
    for (int h = 0; h < n_heads; ++h)
      rotate_head(x + (size_t(t) * n_heads + h) * head_dim, c.data(), s.data(), half);
  }
}

void orc_softmax(float* x, int n) {
  float mx = x[0];
  for (int i = 1; i < n; ++i) mx = std::fmax(mx, x[i]);
  float sum = 0.0f;
  for (int i = 0; i < n; ++i) {
    x[i] = expf(x[i] - mx);
    sum += x[i];
  }
  for (int i = 0; i < n; ++i) x[i] /= sum;
}

void orc_attention(float* out, const float* q, const float* k, const float* v, int T, int pos0,
                   int n_heads, int n_kv_heads, int head_dim, int threads) {
  const int group = n_heads / n_kv_heads;
  const float scale = 1.0f / std::sqrt(float(head_dim));
  const size_t q_stride = size_t(n_heads) * head_dim;
  const size_t kv_stride = size_t(n_kv_heads) * head_dim;
  auto body = [&](int64_t h0, int64_t h1) {
    std::vector<float> scores(size_t(pos0) + T);
    for (int h = int(h0); h < int(h1); ++h) {
      const int kvh = h / group;
      for (int t = 0; t < T; ++t)
        attend_one(out + t * q_stride + size_t(h) * head_dim, q + t * q_stride + size_t(h) * head_dim,
                   k, v, pos0 + t, kvh, kv_stride, head_dim, scale, scores.data());
    }
  };
  if (threads <= 1)
    body(0, n_heads);
  else
    pool_with(threads).run(n_heads, body);
}

int orc_physical_cores(void) {
  std::ifstream f("/proc/cpuinfo");
  std::set<std::pair<int, int>> seen;
  std::string line;
  int phys = 0, core = -1;
  auto value = [](const std::string& l) { return std::stoi(l.substr(l.find(':') + 1)); };
  while (std::getline(f, line)) {
    if (line.rfind("physical id", 0) == 0)
      phys = value(line);
    else if (line.rfind("core id", 0) == 0)
      core = value(line);
    else if (line.empty() && core >= 0) {
      seen.insert({phys, core});
      core = -1;
    }
  }
  if (core >= 0) seen.insert({phys, core});
  const int n = int(seen.size());
  const int logical = int(std::max(1u, std::thread::hardware_concurrency()));
  return (n > 0 && n <= logical) ? n : logical;
}

// IEEE binary16 from float32, round to nearest even, by integer arithmetic.
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t exp = (x >> 23) & 0xFFu;
  uint32_t man = x & 0x7FFFFFu;
  if (exp == 0xFFu) {  // inf / NaN (NaN keeps a quiet payload bit)
    return uint16_t(sign | 0x7C00u | (man ? (0x200u | (man >> 13)) : 0u));
  }
  const int e = int(exp) - 127 + 15;  // biased binary16 exponent
  if (e >= 31) return uint16_t(sign | 0x7C00u);  // overflow
  if (e <= 0) {                                   // subnormal or zero in binary16
    if (e < -10) return uint16_t(sign);           // below half the smallest subnormal
    man |= 0x800000u;                              // implicit bit
    const int shift = 14 - e;                      // 24-bit significand -> 10-bit field
    const uint32_t kept = man >> shift;
    const uint32_t rem = man & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1);
    uint32_t r = kept + ((rem > halfway || (rem == halfway && (kept & 1u))) ? 1u : 0u);
    return uint16_t(sign | r);  // a carry into bit 10 makes the smallest normal: correct
  }
  uint32_t h = (uint32_t(e) << 10) | (man >> 13);
  const uint32_t rem = man & 0x1FFFu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;  // may carry into the exponent / inf
  return uint16_t(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1Fu;
  uint32_t man = h & 0x3FFu;
  uint32_t x;
  if (exp == 0) {
    if (man == 0) {
      x = sign;
    } else {  // subnormal: normalise
      int e = -1;
      do {
        man <<= 1;
        ++e;
      } while (!(man & 0x400u));
      x = sign | (uint32_t(127 - 15 - e) << 23) | ((man & 0x3FFu) << 13);
    }
  } else if (exp == 0x1F) {
    x = sign | 0x7F800000u | (man << 13);
  } else {
    x = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  float f;
  std::memcpy(&f, &x, 4);
  return f;
}

uint16_t orc_f32_to_bf16(float f) {
  uint32_t bits;
  std::memcpy(&bits, &f, 4);
  if ((bits & 0x7F800000u) == 0x7F800000u) return uint16_t(bits >> 16);
  bits += 0x7FFFu + ((bits >> 16) & 1u);
  return uint16_t(bits >> 16);
}

float orc_bf16_to_f32(uint16_t h) {
  const uint32_t bits = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

void orc_round_to_kv(void* dst, const float* src, size_t n, int kv_dtype) {
  for (size_t i = 0; i < n; ++i) store_kv(dst, i, src[i], kv_dtype);
}

void orc_widen_kv(float* dst, const void* src, size_t n, int kv_dtype) {
  for (size_t i = 0; i < n; ++i) dst[i] = load_kv(src, i, kv_dtype);
}

size_t orc_kv_offset(const int32_t* tables, int max_pages, int page_size, int seq, int pos,
                     int kv_dim) {
  const int page = tables[size_t(seq) * max_pages + pos / page_size];
  return (size_t(page) * page_size + pos % page_size) * kv_dim;
}

void orc_rope_append_paged(float* q, const float* k, const float* v, void* k_pool, void* v_pool,
                           int kv_dtype, int T, const int32_t* row_pos, const int32_t* row_seq,
                           const int32_t* tables, int max_pages, int page_size, int n_heads,
                           int n_kv_heads, int head_dim, float theta) {
  const size_t q_dim = size_t(n_heads) * head_dim, kv_dim = size_t(n_kv_heads) * head_dim;
  std::vector<float> kr(kv_dim);
  for (int t = 0; t < T; ++t) {
    const int pos = row_pos[t];
    orc_rope(q + size_t(t) * q_dim, 1, n_heads, head_dim, pos, theta);
    std::memcpy(kr.data(), k + size_t(t) * kv_dim, kv_dim * sizeof(float));
    orc_rope(kr.data(), 1, n_kv_heads, head_dim, pos, theta);
    const size_t dst = orc_kv_offset(tables, max_pages, page_size, row_seq[t], pos, int(kv_dim));
    for (size_t i = 0; i < kv_dim; ++i) {
      store_kv(k_pool, dst + i, kr[i], kv_dtype);
      store_kv(v_pool, dst + i, v[size_t(t) * kv_dim + i], kv_dtype);
    }
  }
}

void orc_gather_kv(float* dst, const void* pool, int kv_dtype, const int32_t* tables,
                   int max_pages, int page_size, int seq, int len, int kv_dim) {
  for (int p = 0; p < len; ++p) {
    const size_t src = orc_kv_offset(tables, max_pages, page_size, seq, p, kv_dim);
    for (int i = 0; i < kv_dim; ++i) dst[size_t(p) * kv_dim + i] = load_kv(pool, src + i, kv_dtype);
  }
}

void orc_paged_attention(float* out, const float* q, const void* k_pool, const void* v_pool,
                         int kv_dtype, int T, const int32_t* row_pos, const int32_t* row_seq,
                         const int32_t* tables, int max_pages, int page_size, int n_heads,
                         int n_kv_heads, int head_dim, int threads) {
  const size_t q_dim = size_t(n_heads) * head_dim;
  const int kv_dim = n_kv_heads * head_dim;
  std::vector<float> kc, vc;
  for (int t = 0; t < T; ++t) {
    const int pos = row_pos[t];
    kc.resize(size_t(pos + 1) * kv_dim);
    vc.resize(kc.size());
    orc_gather_kv(kc.data(), k_pool, kv_dtype, tables, max_pages, page_size, row_seq[t], pos + 1,
                  kv_dim);
    orc_gather_kv(vc.data(), v_pool, kv_dtype, tables, max_pages, page_size, row_seq[t], pos + 1,
                  kv_dim);
    orc_attention(out + size_t(t) * q_dim, q + size_t(t) * q_dim, kc.data(), vc.data(), 1, pos,
                  n_heads, n_kv_heads, head_dim, threads);
  }
}

void orc_gather_rows(float* dst, const float* src, const int32_t* rows, int R, int dim) {
  for (int r = 0; r < R; ++r)
    std::memcpy(dst + size_t(r) * dim, src + size_t(rows[r]) * dim, size_t(dim) * sizeof(float));
}

namespace {

float weight_at(const void* w, int w_dtype, size_t i) {
  if (w_dtype == ORC_W_F32) return static_cast<const float*>(w)[i];
  if (w_dtype == ORC_W_BF16) return orc_bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
  return float(static_cast<const int8_t*>(w)[i]);
}

}  // namespace

void orc_matmul(float* y, const float* x, const void* w, int w_dtype, const float* scale,
                const float* bias, int T, int rows, int cols, int threads) {
  auto body = [&](int64_t r0, int64_t r1) {
    for (int64_t o = r0; o < r1; ++o) {
      const size_t base = size_t(o) * cols;
      const float s = w_dtype == ORC_W_I8 ? scale[o] : 1.0f;
      const float b = bias ? bias[o] : 0.0f;
      for (int t = 0; t < T; ++t) {
        const float* xt = x + size_t(t) * cols;
        float acc = 0.0f;
        if (w_dtype == ORC_W_F32) {  // compiled without contraction there
          for (int k = 0; k < cols; ++k) acc += weight_at(w, w_dtype, base + k) * xt[k];
        } else {
          for (int k = 0; k < cols; ++k) acc = std::fma(weight_at(w, w_dtype, base + k), xt[k], acc);
        }
        y[size_t(t) * rows + o] = acc * s + b;
      }
    }
  };
  pool_with(threads).run(rows, body);
}

void orc_quantize_i8(int8_t* q, float* scale, const float* w, int rows, int cols) {
  for (int r = 0; r < rows; ++r) {
    const float* row = w + size_t(r) * cols;
    float amax = 0.0f;
    for (int i = 0; i < cols; ++i) amax = std::max(amax, std::fabs(row[i]));
    const float s = amax > 0 ? amax / 127.0f : 1.0f;
    scale[r] = s;
    for (int i = 0; i < cols; ++i) {
      const float v = std::nearbyint(row[i] / s);
      q[size_t(r) * cols + i] = int8_t(std::max(-127.0f, std::min(127.0f, v)));
    }
  }
}

void orc_row_to_f32(float* out, const void* w, int w_dtype, const float* scale, int cols, int r) {
  const size_t base = size_t(r) * cols;
  for (int i = 0; i < cols; ++i) {
    const float v = weight_at(w, w_dtype, base + i);
    out[i] = w_dtype == ORC_W_I8 ? scale[r] * v : v;
  }
}

void orc_rmsnorm(float* y, const float* x, const float* weight, int T, int dim, float eps) {
  for (int t = 0; t < T; ++t) {
    const float* xt = x + size_t(t) * dim;
    float* yt = y + size_t(t) * dim;
    float sum_sq = 0.0f;
    for (int i = 0; i < dim; ++i) sum_sq += xt[i] * xt[i];  // not contracted there
    const float inv_rms = 1.0f / std::sqrt(sum_sq / float(dim) + eps);
    for (int i = 0; i < dim; ++i) yt[i] = xt[i] * inv_rms * weight[i];
  }
}

void orc_silu_mul(float* gate, const float* up, size_t n) {
  for (size_t i = 0; i < n; ++i) {
    const float g = gate[i];
    gate[i] = g / (1.0f + std::exp(-g)) * up[i];
  }
}

double orc_compare(const float* got, const float* want, size_t n, double* max_abs_err,
                   size_t* worst_index) {
  double max_err = 0, max_ref = 0;
  size_t worst = 0;
  for (size_t i = 0; i < n; ++i) {
    const double err = std::fabs(double(got[i]) - double(want[i]));
    if (!(err <= max_err)) {
      max_err = err;
      worst = i;
    }
    max_ref = std::fmax(max_ref, std::fabs(double(want[i])));
  }
  if (max_abs_err) *max_abs_err = max_err;
  if (worst_index) *worst_index = worst;
  return max_ref > 0 ? max_err / max_ref : max_err;
}

}  // extern "C"
