// ie::hip::run_selftest and ie::hip::run_device_check: the drop-in's
// counterparts of cuda::run_selftest (src/cuda/cuda_runner.h:36-37, run by
// `ie test-cuda`, src/main.cpp:1033-1045) and cuda::run_device_check
// (src/cuda/device_check.h:7, `ie gpu-check`, src/main.cpp:1207-1213).
//
// run_selftest checks each kernel family of libie_hip.so against the host
// program's own CPU operations (the reference's ie::rope, ie::attention,
// ie::rmsnorm and ie::matmul, src/ops.h and src/matrix.h, linked into every
// build of the engine) on seeded random data, at the path's bars: page bytes,
// rotated queries and gathered rows bit for bit; attention within 1e-5 of the
// largest output (f32 caches) or 2e-3 absolute (f16 / bf16 caches); rmsnorm and
// the BF16 matmul within 1e-5 of the largest output. It prints one line per
// check and returns the number that failed.
//
// run_device_check prints the device's properties, checks a copy by this
// library's gather kernel against the host, and times device-to-device copies
// (the runtime's and the gather kernel's) against the nominal 8 TB/s.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <string>
#include <vector>

#include "ie_hip.hpp"
#include "ie_hip_runner.hpp"
#include "matrix.h"
#include "ops.h"

namespace ie::hip {
namespace {

constexpr int kNH = 14, kNKV = 2, kHD = 64, kKVD = kNKV * kHD, kQD = kNH * kHD, kPage = 16;
constexpr float kTheta = 1e6f;

// f32 -> IEEE binary16 bits, round to nearest even, subnormals kept: the
// conversion the f16 pages hold.
uint16_t f16_bits(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
  if (ax > 0x7F800000u) return uint16_t(sign | 0x7E00u);   // NaN
  if (ax >= 0x47800000u) return uint16_t(sign | 0x7C00u);  // >= 2^16, inf
  if (ax >= 0x38800000u) {                                 // normal: >= 2^-14
    uint32_t r = ax - 0x38000000u;                         // exponent bias 127 -> 15
    r += 0xFFFu + ((r >> 13) & 1u);
    return uint16_t(sign | (r >> 13));                     // a carry may round up to inf
  }
  const int e = int(ax >> 23);  // below 2^-14: a multiple of 2^-24
  if (e < 102) return uint16_t(sign);
  const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
  const int shift = 126 - e;
  uint32_t m = mant >> shift;
  const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
  if (rem > half || (rem == half && (m & 1u))) ++m;
  return uint16_t(sign | m);
}
float f16_value(uint16_t h) {
  const uint32_t sign = uint32_t(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
  float v;
  if (e == 0)
    v = std::ldexp(float(m), -24);
  else if (e == 31)
    v = m ? NAN : INFINITY;
  else
    v = std::ldexp(float(m | 0x400u), int(e) - 25);
  uint32_t b;
  std::memcpy(&b, &v, 4);
  b |= sign;
  std::memcpy(&v, &b, 4);
  return v;
}
// bf16 by the reference's own rounding (make_matrix, src/matrix.cpp).
std::vector<uint16_t> bf16_bits(const std::vector<float>& x) {
  return make_matrix(x, 1, int(x.size()), DType::BF16).bf16;
}
float bf16_value(uint16_t h) {
  const uint32_t b = uint32_t(h) << 16;
  float v;
  std::memcpy(&v, &b, 4);
  return v;
}

const char* kv_name(int kv) { return kv == IE_KV_F32 ? "f32" : kv == IE_KV_F16 ? "f16" : "bf16"; }

// A device buffer for the checks (freed on scope exit).
struct Buf {
  void* p = nullptr;
  explicit Buf(size_t bytes) { check(hipMalloc(&p, std::max<size_t>(bytes, 16)), "hipMalloc"); }
  ~Buf() { (void)hipFree(p); }
  Buf(const Buf&) = delete;
  Buf& operator=(const Buf&) = delete;
  template <class T>
  T* as() const { return static_cast<T*>(p); }
};
template <class T>
void put(const Buf& b, const std::vector<T>& h) {
  check(hipMemcpy(b.p, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy");
}
template <class T>
std::vector<T> get(const Buf& b, size_t n) {
  std::vector<T> h(n);
  check(hipMemcpy(h.data(), b.p, n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy");
  return h;
}

struct Tally {
  int run = 0, failed = 0;
  void report(bool ok, const std::string& what, double err, double bar) {
    ++run;
    failed += !ok;
    std::printf("  %-4s %-58s err %.3g (bar %.3g)\n", ok ? "ok" : "FAIL", what.c_str(), err, bar);
  }
};

double rel_err(const std::vector<float>& got, const std::vector<float>& want) {
  double d = 0, m = 0;
  for (size_t i = 0; i < want.size(); ++i) {
    if (!std::isfinite(got[i])) return INFINITY;
    d = std::max(d, double(std::fabs(got[i] - want[i])));
    m = std::max(m, double(std::fabs(want[i])));
  }
  return m > 0 ? d / m : d;
}
double abs_err(const std::vector<float>& got, const std::vector<float>& want) {
  double d = 0;
  for (size_t i = 0; i < want.size(); ++i) {
    if (!std::isfinite(got[i])) return INFINITY;
    d = std::max(d, double(std::fabs(got[i] - want[i])));
  }
  return d;
}

// A pool of `pages` pages of one KV type with N(0,1) contents: the device
// bytes and the same values widened to f32 for the host reference.
struct Pool {
  int kv;
  std::vector<float> wide;     // [pages * 16, 128]
  std::vector<uint16_t> bits;  // 16-bit types
  Pool(int kv_dtype, int pages, std::mt19937& rng) : kv(kv_dtype) {
    std::normal_distribution<float> nd;
    wide.resize(size_t(pages) * kPage * kKVD);
    for (float& x : wide) x = nd(rng);
    if (kv == IE_KV_F16) {
      bits.resize(wide.size());
      for (size_t i = 0; i < wide.size(); ++i) {
        bits[i] = f16_bits(wide[i]);
        wide[i] = f16_value(bits[i]);
      }
    } else if (kv == IE_KV_BF16) {
      bits = bf16_bits(wide);
      for (size_t i = 0; i < wide.size(); ++i) wide[i] = bf16_value(bits[i]);
    }
  }
  size_t bytes() const { return wide.size() * (kv == IE_KV_F32 ? 4 : 2); }
  void upload(const Buf& b) const {
    if (kv == IE_KV_F32)
      put(b, wide);
    else
      put(b, bits);
  }
};

// Pages handed out as one shuffled permutation: table [seqs, max_pages].
std::vector<int32_t> shuffled_tables(const std::vector<int>& lens, int max_pages, int pages,
                                     std::mt19937& rng) {
  std::vector<int32_t> perm(pages);
  for (int i = 0; i < pages; ++i) perm[i] = i;
  std::shuffle(perm.begin(), perm.end(), rng);
  std::vector<int32_t> tab(lens.size() * size_t(max_pages), 0);
  int next = 0;
  for (size_t s = 0; s < lens.size(); ++s)
    for (int p = 0; p < (lens[s] + kPage - 1) / kPage; ++p) tab[s * max_pages + p] = perm[next++];
  return tab;
}

// The first L positions of sequence s, copied out of the pool (host).
std::vector<float> gathered(const std::vector<float>& pool, const std::vector<int32_t>& tab,
                            int max_pages, int s, int L) {
  std::vector<float> out(size_t(L) * kKVD);
  for (int p = 0; p < L; ++p) {
    const size_t row = size_t(tab[size_t(s) * max_pages + p / kPage]) * kPage + p % kPage;
    std::copy_n(pool.begin() + row * kKVD, kKVD, out.begin() + size_t(p) * kKVD);
  }
  return out;
}

void check_rope_append(Tally& t, int kv, std::mt19937& rng) {
  const std::vector<int> pos = {0, 15, 16, 300, 1023};
  const int R = int(pos.size()), max_pages = 1024 / kPage, pages = R * max_pages;
  std::vector<int> lens;
  for (int p : pos) lens.push_back(p + 1);
  const std::vector<int32_t> tab = shuffled_tables(lens, max_pages, pages, rng);
  Pool kp(kv, pages, rng), vp(kv, pages, rng);
  std::normal_distribution<float> nd;
  std::vector<float> q(size_t(R) * kQD), k(size_t(R) * kKVD), v(size_t(R) * kKVD);
  for (float& x : q) x = nd(rng);
  for (float& x : k) x = nd(rng);
  for (float& x : v) x = nd(rng);
  std::vector<float> table(size_t(1024) * kHD);
  check(ie_hip_rope_table(table.data(), 1024, kHD, kTheta));
  std::vector<int32_t> rpos(pos.begin(), pos.end()), rseq(R);
  for (int i = 0; i < R; ++i) rseq[i] = i;

  Buf dq(q.size() * 4), dk(k.size() * 4), dv(v.size() * 4), dkp(kp.bytes()), dvp(vp.bytes()),
      dtab(tab.size() * 4), drope(table.size() * 4), dpos(R * 4), dseq(R * 4);
  put(dq, q);
  put(dk, k);
  put(dv, v);
  kp.upload(dkp);
  vp.upload(dvp);
  put(dtab, tab);
  put(drope, table);
  put(dpos, rpos);
  put(dseq, rseq);
  KvLayout lay;
  lay.tables = dtab.as<int32_t>();
  lay.max_pages = max_pages;
  lay.kv_dtype = kv;
  lay.num_pages = pages;
  rope_and_cache(dq.as<float>(), dk.as<float>(), dv.as<float>(), dkp.p, dvp.p,
                 drope.as<float>(), 1024, R, dpos.as<int>(), dseq.as<int>(), lay, kNH, kNKV, kHD,
                 nullptr);
  check(hipDeviceSynchronize(), "rope_and_cache");

  // Host: the reference's rope on q and k, then the rows stored in the cache's type.
  std::vector<float> qr = q, kr = k;
  size_t bad_pages = 0;
  for (int i = 0; i < R; ++i) {
    ie::rope(qr.data() + size_t(i) * kQD, 1, kNH, kHD, pos[i], kTheta);
    ie::rope(kr.data() + size_t(i) * kKVD, 1, kNKV, kHD, pos[i], kTheta);
  }
  const std::vector<float> got_q = get<float>(dq, q.size());
  const bool q_ok = std::memcmp(got_q.data(), qr.data(), q.size() * 4) == 0;
  for (int which = 0; which < 2; ++which) {
    const Pool& pool = which ? vp : kp;
    const Buf& dev = which ? dvp : dkp;
    const std::vector<float>& rows = which ? v : kr;
    // The expected pool: the old one with each row's slot replaced.
    std::vector<float> want_wide = pool.wide;
    std::vector<uint16_t> want_bits = pool.bits;
    for (int i = 0; i < R; ++i) {
      const size_t row = size_t(tab[size_t(i) * max_pages + pos[i] / kPage]) * kPage + pos[i] % kPage;
      for (int d = 0; d < kKVD; ++d) {
        const float x = rows[size_t(i) * kKVD + d];
        if (kv == IE_KV_F32) want_wide[row * kKVD + d] = x;
        if (kv == IE_KV_F16) want_bits[row * kKVD + d] = f16_bits(x);
      }
      if (kv == IE_KV_BF16) {
        const std::vector<float> one(rows.begin() + size_t(i) * kKVD,
                                     rows.begin() + size_t(i + 1) * kKVD);
        const std::vector<uint16_t> b = bf16_bits(one);
        std::copy(b.begin(), b.end(), want_bits.begin() + row * kKVD);
      }
    }
    if (kv == IE_KV_F32) {
      const std::vector<float> g = get<float>(dev, want_wide.size());
      bad_pages += std::memcmp(g.data(), want_wide.data(), g.size() * 4) != 0;
    } else {
      const std::vector<uint16_t> g = get<uint16_t>(dev, want_bits.size());
      bad_pages += std::memcmp(g.data(), want_bits.data(), g.size() * 2) != 0;
    }
  }
  t.report(q_ok, std::string("rope(q), ") + kv_name(kv) + " cache", q_ok ? 0 : 1, 0);
  t.report(bad_pages == 0, std::string("rope + paged append: page bytes, ") + kv_name(kv),
           double(bad_pages), 0);
}

void check_attention(Tally& t, int kv, std::mt19937& rng) {
  const std::vector<int> lens = {1, 17, 64, 255, 256, 1000, 3000};
  const int R = int(lens.size()), max_len = 3000, max_pages = (max_len + kPage - 1) / kPage;
  int pages = 0;
  for (int L : lens) pages += (L + kPage - 1) / kPage;
  pages += 3;
  const std::vector<int32_t> tab = shuffled_tables(lens, max_pages, pages, rng);
  Pool kp(kv, pages, rng), vp(kv, pages, rng);
  std::normal_distribution<float> nd;
  std::vector<float> q(size_t(R) * kQD);
  for (float& x : q) x = nd(rng);
  std::vector<int32_t> rpos(R), rseq(R);
  for (int i = 0; i < R; ++i) {
    rpos[i] = lens[i] - 1;
    rseq[i] = i;
  }
  const int ct = attention_chunk_tokens(R, max_len, kv), nc = attention_chunks(max_len, ct);
  Buf dq(q.size() * 4), dout(q.size() * 4), dkp(kp.bytes()), dvp(vp.bytes()),
      dtab(tab.size() * 4), dpos(R * 4), dseq(R * 4),
      dws(attention_workspace_bytes(R, kNH, kHD, nc));
  put(dq, q);
  kp.upload(dkp);
  vp.upload(dvp);
  put(dtab, tab);
  put(dpos, rpos);
  put(dseq, rseq);
  KvLayout lay;
  lay.tables = dtab.as<int32_t>();
  lay.max_pages = max_pages;
  lay.kv_dtype = kv;
  lay.num_pages = pages;
  attention(dout.as<float>(), dq.as<float>(), dkp.p, dvp.p, R, dpos.as<int>(), dseq.as<int>(),
            lay, nc, ct, dws.p, kNH, kNKV, kHD, nullptr);
  check(hipDeviceSynchronize(), "attention");
  const std::vector<float> got = get<float>(dout, q.size());
  std::vector<float> want(q.size());
  for (int i = 0; i < R; ++i)
    ie::attention(want.data() + size_t(i) * kQD, q.data() + size_t(i) * kQD,
                  gathered(kp.wide, tab, max_pages, i, lens[i]).data(),
                  gathered(vp.wide, tab, max_pages, i, lens[i]).data(), 1, lens[i] - 1, kNH, kNKV,
                  kHD);
  const bool f32 = kv == IE_KV_F32;
  const double err = f32 ? rel_err(got, want) : abs_err(got, want), bar = f32 ? 1e-5 : 2e-3;
  t.report(err <= bar,
           std::string("flash-decoding, contexts 1..3000, ") + kv_name(kv) + " cache, " +
               std::to_string(ct) + "-token chunks",
           err, bar);

  // A prompt: rows 100..399 of one sequence, causal, over its own pages.
  const int P0 = 100, T = 300, L = P0 + T;
  const std::vector<int32_t> ptab = shuffled_tables({L}, (L + kPage - 1) / kPage, pages, rng);
  std::vector<float> pq(size_t(T) * kQD);
  for (float& x : pq) x = nd(rng);
  std::vector<int32_t> ppos(T), pseq(T, 0);
  for (int i = 0; i < T; ++i) ppos[i] = P0 + i;
  Buf dpq(pq.size() * 4), dpout(pq.size() * 4), dptab(ptab.size() * 4), dppos(T * 4), dpseq(T * 4);
  put(dpq, pq);
  put(dptab, ptab);
  put(dppos, ppos);
  put(dpseq, pseq);
  lay.tables = dptab.as<int32_t>();
  lay.max_pages = (L + kPage - 1) / kPage;
  attention_prefill(dpout.as<float>(), dpq.as<float>(), dkp.p, dvp.p, T, dppos.as<int>(),
                    dpseq.as<int>(), lay, kNH, kNKV, kHD, nullptr);
  check(hipDeviceSynchronize(), "attention_prefill");
  const std::vector<float> pgot = get<float>(dpout, pq.size());
  std::vector<float> pwant(pq.size());
  ie::attention(pwant.data(), pq.data(), gathered(kp.wide, ptab, lay.max_pages, 0, L).data(),
                gathered(vp.wide, ptab, lay.max_pages, 0, L).data(), T, P0, kNH, kNKV, kHD);
  const double perr = f32 ? rel_err(pgot, pwant) : abs_err(pgot, pwant);
  t.report(perr <= bar, std::string("prefill, 300 rows from position 100, ") + kv_name(kv), perr,
           bar);
}

void check_dense(Tally& t, std::mt19937& rng) {
  std::normal_distribution<float> nd;
  const int T = 5, in = 512, out = 896;
  std::vector<float> x(size_t(T) * in), w(size_t(out) * in), norm(in), bias(out);
  for (float& a : x) a = nd(rng);
  for (float& a : w) a = 0.05f * nd(rng);
  for (float& a : norm) a = 1.0f + 0.1f * nd(rng);
  for (float& a : bias) a = nd(rng);
  const Matrix W = make_matrix(w, out, in, DType::BF16);
  Buf dx(x.size() * 4), dy(size_t(T) * out * 4), dn(x.size() * 4), dw(W.bf16.size() * 2),
      dnorm(norm.size() * 4), dbias(bias.size() * 4);
  put(dx, x);
  put(dw, W.bf16);
  put(dnorm, norm);
  put(dbias, bias);
  rmsnorm(dn.as<float>(), dx.as<float>(), dnorm.as<float>(), T, in, 1e-6f, nullptr);
  const ie_matrix dm{dw.p, nullptr, 0, out, in};
  matmul(dy.as<float>(), dx.as<float>(), dm, dbias.as<float>(), T, false, nullptr);
  check(hipDeviceSynchronize(), "dense");
  std::vector<float> want_n(x.size()), want_y(size_t(T) * out);
  ie::rmsnorm(want_n.data(), x.data(), norm.data(), T, in, 1e-6f);
  ie::matmul(want_y.data(), x.data(), W, bias.data(), T);
  const double en = rel_err(get<float>(dn, x.size()), want_n);
  const double ey = rel_err(get<float>(dy, want_y.size()), want_y);
  t.report(en <= 1e-5, "rmsnorm [5 x 512]", en, 1e-5);
  t.report(ey <= 1e-5, "matmul, BF16 weights [896 x 512], 5 rows, bias", ey, 1e-5);

  // Gather: rows picked out exactly.
  const std::vector<int32_t> pick = {4, 0, 2, 2};
  Buf dpick(pick.size() * 4), dg(pick.size() * in * 4);
  put(dpick, pick);
  gather_rows(dg.as<float>(), dx.as<float>(), dpick.as<int>(), int(pick.size()), in, nullptr);
  check(hipDeviceSynchronize(), "gather_rows");
  const std::vector<float> g = get<float>(dg, pick.size() * in);
  bool same = true;
  for (size_t r = 0; r < pick.size(); ++r)
    same = same && std::memcmp(g.data() + r * in, x.data() + size_t(pick[r]) * in, in * 4) == 0;
  t.report(same, "gather_rows", same ? 0 : 1, 0);
}

}  // namespace

int run_selftest() {
  if (!device_available()) {
    std::printf("No HIP device found.\n");
    return 1;
  }
  std::printf("Self-test of %s against the host CPU operations:\n", device_description().c_str());
  Tally t;
  std::mt19937 rng(1234);
  try {
    for (int kv : {IE_KV_F32, IE_KV_F16, IE_KV_BF16}) {
      check_rope_append(t, kv, rng);
      check_attention(t, kv, rng);
    }
    check_dense(t, rng);
  } catch (const std::exception& e) {
    std::printf("  FAIL %s\n", e.what());
    ++t.failed;
  }
  std::printf("%s: %d checks, %d failed\n", t.failed ? "FAILED" : "ALL PASSED", t.run, t.failed);
  return t.failed;
}

int run_device_check() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    std::printf("No HIP device found.\n");
    return 1;
  }
  try {
    int dev = 0;
    check(hipGetDevice(&dev), "hipGetDevice");
    hipDeviceProp_t p{};
    check(hipGetDeviceProperties(&p, dev), "hipGetDeviceProperties");
    size_t free_b = 0, total_b = 0;
    check(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo");
    int rt = 0, drv = 0;
    check(hipRuntimeGetVersion(&rt), "hipRuntimeGetVersion");
    check(hipDriverGetVersion(&drv), "hipDriverGetVersion");
    std::printf("GPU               : %s (%s), device %d of %d\n", p.name[0] ? p.name : "AMD GPU",
                p.gcnArchName, dev, n);
    std::printf("Compute units     : %d, wavefront %d, %d MHz\n", p.multiProcessorCount,
                p.warpSize, p.clockRate / 1000);
    std::printf("HBM               : %.2f GiB total, %.2f GiB free\n", total_b / 1073741824.0,
                free_b / 1073741824.0);
    std::printf("L2 cache          : %d KiB per XCD\n", p.l2CacheSize / 1024);
    std::printf("LDS per workgroup : %zu KiB\n", p.sharedMemPerBlock / 1024);
    std::printf("HIP runtime       : %d, driver %d\n\n", rt, drv);

    // Correctness: 1M floats copied by this library's gather kernel.
    const int rows = 4096, dim = 256;
    std::vector<float> h(size_t(rows) * dim);
    for (size_t i = 0; i < h.size(); ++i) h[i] = float(i) * 0.5f - 7.0f;
    std::vector<int32_t> idx(rows);
    for (int i = 0; i < rows; ++i) idx[i] = rows - 1 - i;
    Buf src(h.size() * 4), dst(h.size() * 4), didx(idx.size() * 4);
    put(src, h);
    put(didx, idx);
    gather_rows(dst.as<float>(), src.as<float>(), didx.as<int>(), rows, dim, nullptr);
    check(hipDeviceSynchronize(), "gather_rows");
    const std::vector<float> g = get<float>(dst, h.size());
    bool ok = true;
    for (int r = 0; r < rows && ok; ++r)
      ok = std::memcmp(g.data() + size_t(r) * dim, h.data() + size_t(rows - 1 - r) * dim,
                       dim * 4) == 0;
    std::printf("Row gather (1M floats)      : %s\n", ok ? "ok" : "MISMATCH");

    // Bandwidth: 1 GiB device-to-device, the runtime's copy and the gather
    // kernel over the same bytes (read + write), best of 5.
    const size_t bytes = size_t(1) << 30;
    const int grow = int(bytes / (dim * 4));
    Buf a(bytes), b(bytes), gidx(size_t(grow) * 4);
    check(hipMemset(a.p, 0, bytes), "hipMemset");
    std::vector<int32_t> ident(grow);
    for (int i = 0; i < grow; ++i) ident[i] = i;
    put(gidx, ident);
    hipEvent_t e0, e1;
    check(hipEventCreate(&e0), "hipEventCreate");
    check(hipEventCreate(&e1), "hipEventCreate");
    auto best_of = [&](auto&& body) {
      float best = 1e30f;
      for (int i = 0; i < 6; ++i) {
        check(hipEventRecord(e0, nullptr), "hipEventRecord");
        body();
        check(hipEventRecord(e1, nullptr), "hipEventRecord");
        check(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms = 0;
        check(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        if (i) best = std::min(best, ms);  // the first run warms up
      }
      return best;
    };
    const float ms_copy = best_of([&] {
      check(hipMemcpyAsync(b.p, a.p, bytes, hipMemcpyDeviceToDevice, nullptr), "hipMemcpyAsync");
    });
    const float ms_gather = best_of([&] {
      gather_rows(b.as<float>(), a.as<float>(), gidx.as<int>(), grow, dim, nullptr);
    });
    check(hipEventDestroy(e0), "hipEventDestroy");
    check(hipEventDestroy(e1), "hipEventDestroy");
    const double gbs_copy = 2.0 * bytes / (ms_copy * 1e-3) / 1e9;
    const double gbs_gather = 2.0 * bytes / (ms_gather * 1e-3) / 1e9;
    std::printf("Device copy, 1 GiB          : %.0f GB/s read + write (%.0f%% of 8 TB/s)\n",
                gbs_copy, gbs_copy / 80.0);
    std::printf("Gather kernel copy, 1 GiB   : %.0f GB/s read + write (%.0f%% of 8 TB/s)\n",
                gbs_gather, gbs_gather / 80.0);
    return ok ? 0 : 1;
  } catch (const std::exception& e) {
    std::printf("device check failed: %s\n", e.what());
    return 1;
  }
}

}  // namespace ie::hip
