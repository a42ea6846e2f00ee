// Standalone Branchcraft driver for MI355X: `branchcraft test | bench |
// tree-bench [--quick] [--output FILE]` and `branchcraft config N`.
//
// The command line, the test cases and their 3e-4 gates, the benchmark
// sweeps, the timing protocol (5 warm-ups, then 7 trials of 20 launches,
// median) and the CSV columns are the reference driver's contract (src/main.cu
// of Haaziq386/branchcraft-cuda: cases :252-352, protocol :354-373, columns
// :451-453 and :495-496, command line :527-553); `config N` adds the five
// benchmark configurations with the CPU oracle timed on this host.  Kernels
// are reached only through the C ABI (include/branchcraft.hpp) and the HIP
// runtime serves device memory and events.  This is test and measurement
// tooling: it links the CPU oracle (oracle/bc_oracle.c) as its checker.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <functional>
#include <iomanip>
#include <iostream>
#include <memory>
#include <numeric>
#include <random>
#include <sstream>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "bc_oracle.h"
#include "branchcraft.hpp"

namespace drv {

using branchcraft::kPageSize;
using branchcraft::Shape;
using bits16 = uint16_t;  // FP16 bit patterns on the host

// ---- errors and device memory ------------------------------------------------

[[noreturn]] void fail(const std::string& what) { throw std::runtime_error(what); }

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}
#define HIP_OK(call) ::drv::hip_ok((call), #call)

int pages_for(int tokens) { return (tokens + kPageSize - 1) / kPageSize; }

// An owned device array of `size()` elements of T.  Host vectors of any
// element type of the same width copy in and out bit for bit (FP16 bit
// patterns into `half` arrays).
template <class T>
class DevArray {
 public:
  DevArray() = default;
  explicit DevArray(size_t n) : n_(n) {
    void* p = nullptr;
    HIP_OK(hipMalloc(&p, std::max<size_t>(n, 1) * sizeof(T)));
    mem_.reset(static_cast<T*>(p));
  }
  template <class U>
  static DevArray copy_of(const std::vector<U>& host) {
    DevArray a(host.size());
    a.write(host);
    return a;
  }
  template <class U>
  void write(const std::vector<U>& host) {
    static_assert(sizeof(U) == sizeof(T), "element widths must agree");
    if (host.size() != n_) fail("host/device size mismatch");
    HIP_OK(hipMemcpy(mem_.get(), host.data(), n_ * sizeof(T), hipMemcpyHostToDevice));
  }
  template <class U = T>
  std::vector<U> read() const {
    static_assert(sizeof(U) == sizeof(T), "element widths must agree");
    std::vector<U> host(n_);
    HIP_OK(hipMemcpy(host.data(), mem_.get(), n_ * sizeof(T), hipMemcpyDeviceToHost));
    return host;
  }
  T* get() const { return mem_.get(); }
  size_t size() const { return n_; }

 private:
  struct Release {
    void operator()(T* p) const { (void)hipFree(p); }
  };
  std::unique_ptr<T, Release> mem_;
  size_t n_ = 0;
};

// ---- deterministic inputs ------------------------------------------------------
// The engine is std::mt19937 (fully specified); normals (Box-Muller), integers
// below a bound (rejection) and shuffles (Fisher-Yates) are written out here,
// so the inputs do not depend on the standard library's distributions.

class Gen {
 public:
  explicit Gen(uint32_t seed) : eng_(seed) {}
  uint32_t below(uint32_t n) {
    const uint32_t cut = 0xffffffffu - 0xffffffffu % n;
    for (;;) {
      const uint32_t x = eng_();
      if (x < cut) return x % n;
    }
  }
  float normal(float sigma) {
    const double u = open01(), w = open01();
    return (float)(sigma * std::sqrt(-2.0 * std::log(u)) * std::cos(6.283185307179586 * w));
  }
  std::vector<bits16> halves(size_t n, float sigma) {
    std::vector<bits16> out(n);
    for (auto& x : out) x = oracle_f2h(normal(sigma));
    return out;
  }
  std::vector<int> permutation(int n) {
    std::vector<int> p(n);
    std::iota(p.begin(), p.end(), 0);
    for (int i = n - 1; i > 0; --i) std::swap(p[i], p[below((uint32_t)i + 1)]);
    return p;
  }

 private:
  double open01() { return (eng_() + 0.5) * (1.0 / 4294967296.0); }
  std::mt19937 eng_;
};

// A paged KV cache on the host: queries, K/V pools, page table, lengths.
struct PagedHost {
  Shape shape;
  std::vector<bits16> q, k, v;
  std::vector<int> table, lengths;
  size_t out_elems() const { return (size_t)shape.batch * shape.query_heads * shape.dim; }
};

struct CacheSpec {
  int batch, hq, hkv, dim;
  std::vector<int> lengths;
  uint32_t seed = 17;
  float sigma = 0.5f;
  int spare_pages = 7;  // free pages past the used ones
};

// Sequences take their pages in order from a shuffled pool (the reference
// fixture's shape, src/main.cu:48-79); K, V and Q are N(0, sigma) FP16.
PagedHost make_cache(const CacheSpec& c) {
  if ((int)c.lengths.size() != c.batch) fail("length count mismatch");
  int need = 0, longest = 0;
  for (int n : c.lengths) {
    need += pages_for(n);
    longest = std::max(longest, n);
  }
  PagedHost h;
  h.shape = {c.batch, c.hq, c.hkv, c.dim, std::max(1, pages_for(longest)), need + c.spare_pages};
  h.lengths = c.lengths;
  Gen gen(c.seed);
  const std::vector<int> pool = gen.permutation(h.shape.physical_pages);
  h.table.assign((size_t)c.batch * h.shape.max_pages, -1);
  auto next = pool.begin();
  for (int b = 0; b < c.batch; ++b)
    for (int p = 0; p < pages_for(c.lengths[b]); ++p) h.table[(size_t)b * h.shape.max_pages + p] = *next++;
  const size_t pool_elems = (size_t)h.shape.physical_pages * kPageSize * c.hkv * c.dim;
  h.q = gen.halves(h.out_elems(), c.sigma);
  h.k = gen.halves(pool_elems, c.sigma);
  h.v = gen.halves(pool_elems, c.sigma);
  return h;
}

std::vector<float> oracle_of(const PagedHost& h, int threads = 1) {
  std::vector<float> out(h.out_elems());
  const Shape& s = h.shape;
  oracle_decode(s.batch, s.query_heads, s.kv_heads, s.dim, s.max_pages, h.q.data(), h.k.data(),
                h.v.data(), h.table.data(), h.lengths.data(), out.data(), threads);
  return out;
}

float worst_gap(const std::vector<float>& a, const std::vector<float>& b) {
  if (a.size() != b.size()) fail("comparison size mismatch");
  return oracle_max_abs_error(a.data(), b.data(), a.size());
}

// The cache on the device, with an FP32 output and split scratch for up to
// `max_splits` splits (the reference's Scratch sizes).
class PagedDevice {
 public:
  PagedDevice(const PagedHost& h, int max_splits)
      : shape_(h.shape),
        q_(DevArray<half>::copy_of(h.q)),
        k_(DevArray<half>::copy_of(h.k)),
        v_(DevArray<half>::copy_of(h.v)),
        table_(DevArray<int>::copy_of(h.table)),
        lengths_(DevArray<int>::copy_of(h.lengths)),
        out_(h.out_elems()),
        acc_((size_t)max_splits * h.out_elems()),
        ml_((size_t)max_splits * h.shape.batch * h.shape.query_heads * 2) {}

  branchcraft::Inputs inputs() const {
    return {q_.get(), k_.get(), v_.get(), table_.get(), lengths_.get(), out_.get()};
  }
  branchcraft::Scratch scratch() const { return {acc_.get(), ml_.get()}; }
  hipError_t decode(int splits) const {
    return branchcraft::decode(shape_, inputs(), scratch(), splits);
  }
  std::vector<float> decode_now(int splits) const {
    HIP_OK(decode(splits));
    HIP_OK(hipDeviceSynchronize());
    return out_.read();
  }
  const Shape& shape() const { return shape_; }
  DevArray<half>& q() { return q_; }
  DevArray<half>& k() { return k_; }
  DevArray<half>& v() { return v_; }
  DevArray<int>& table() { return table_; }
  DevArray<int>& lengths() { return lengths_; }

 private:
  Shape shape_;
  DevArray<half> q_, k_, v_;
  DevArray<int> table_, lengths_;
  DevArray<float> out_, acc_, ml_;
};

// ---- trees ---------------------------------------------------------------------

enum class Parents { kBinary, kRandom };

struct TreeHost {
  PagedHost prefix;  // every request's table row names the same prefix pages
  int nodes = 0;
  std::vector<bits16> dq, dk, dv;
  std::vector<int> parent;
};

// `batch` requests over one shared `prefix_len`-token prefix (32 query and 8
// KV heads; the reference tree fixture's shape, src/main.cu:145-179), each
// with `nodes` draft tokens; parents (n-1)/2 or uniform in [0, n-1].
TreeHost make_tree(int batch, int prefix_len, int nodes, int dim, uint32_t seed = 31,
                   float sigma = 0.5f, Parents kind = Parents::kBinary) {
  const PagedHost one = make_cache({1, 32, 8, dim, {prefix_len}, seed, sigma});
  TreeHost t;
  t.nodes = nodes;
  PagedHost& p = t.prefix;
  p.shape = {batch, 32, 8, dim, one.shape.max_pages + 2, one.shape.physical_pages + 2 * batch};
  p.lengths.assign(batch, prefix_len);
  p.table.assign((size_t)batch * p.shape.max_pages, -1);
  for (int b = 0; b < batch; ++b) {
    std::copy_n(one.table.begin(), pages_for(prefix_len), p.table.begin() + (size_t)b * p.shape.max_pages);
    p.q.insert(p.q.end(), one.q.begin(), one.q.end());
  }
  const size_t pool_elems = (size_t)p.shape.physical_pages * kPageSize * 8 * dim;
  p.k = one.k;
  p.v = one.v;
  p.k.resize(pool_elems, 0);
  p.v.resize(pool_elems, 0);
  Gen gen(seed + 99);
  t.dq = gen.halves((size_t)batch * nodes * 32 * dim, sigma);
  t.dk = gen.halves((size_t)batch * nodes * 8 * dim, sigma);
  t.dv = gen.halves(t.dk.size(), sigma);
  t.parent.resize((size_t)batch * nodes);
  for (int b = 0; b < batch; ++b)
    for (int n = 0; n < nodes; ++n)
      t.parent[(size_t)b * nodes + n] =
          n == 0 ? -1 : kind == Parents::kRandom ? (int)gen.below((uint32_t)n) : (n - 1) / 2;
  return t;
}

std::vector<float> oracle_of(const TreeHost& t, int threads = 1) {
  const Shape& s = t.prefix.shape;
  std::vector<float> out(t.dq.size());
  oracle_tree(s.batch, t.nodes, s.query_heads, s.kv_heads, s.dim, s.max_pages, t.prefix.k.data(),
              t.prefix.v.data(), t.prefix.table.data(), t.prefix.lengths.data(), t.dq.data(),
              t.dk.data(), t.dv.data(), t.parent.data(), out.data(), threads);
  return out;
}

// A tree on the device; verification runs through the workspace call.
class TreeDevice {
 public:
  explicit TreeDevice(const TreeHost& t)
      : prefix_(t.prefix, 1),
        dq_(DevArray<half>::copy_of(t.dq)),
        dk_(DevArray<half>::copy_of(t.dk)),
        dv_(DevArray<half>::copy_of(t.dv)),
        parent_(DevArray<int>::copy_of(t.parent)),
        out_(t.dq.size()),
        ws_(branchcraft::tree_verify_workspace_size(t.prefix.shape, t.nodes)),
        nodes_(t.nodes) {}

  hipError_t verify() const {
    const branchcraft::TreeInputs in{prefix_.inputs(), dq_.get(), dk_.get(), dv_.get(),
                                     parent_.get(), out_.get()};
    return branchcraft::tree_verify(prefix_.shape(), in, nodes_, ws_.get(), ws_.size());
  }
  std::vector<float> verify_now() const {
    HIP_OK(verify());
    HIP_OK(hipDeviceSynchronize());
    return out_.read();
  }
  PagedDevice& prefix() { return prefix_; }
  const DevArray<half>& draft_q() const { return dq_; }
  const DevArray<half>& draft_k() const { return dk_; }
  const DevArray<half>& draft_v() const { return dv_; }

 private:
  PagedDevice prefix_;
  DevArray<half> dq_, dk_, dv_;
  DevArray<int> parent_;
  DevArray<float> out_;
  DevArray<char> ws_;
  int nodes_;
};

// Every candidate as its own paged sequence: prefix then its root-to-node
// path (the expanded-prefix baseline, src/main.cu:375-423), built by the
// oracle's restatement.
PagedHost expand(const TreeHost& t) {
  const Shape& ps = t.prefix.shape;
  int longest = 0, used = 0;
  oracle_expand_tree(ps.batch, t.nodes, ps.kv_heads, ps.dim, ps.max_pages, t.prefix.k.data(),
                     t.prefix.v.data(), t.prefix.table.data(), t.prefix.lengths.data(), t.dk.data(),
                     t.dv.data(), t.parent.data(), &longest, &used, nullptr, nullptr, nullptr,
                     nullptr);
  PagedHost f;
  const int seqs = ps.batch * t.nodes;
  f.shape = {seqs, ps.query_heads, ps.kv_heads, ps.dim, std::max(1, longest), used + 7};
  f.lengths.resize(seqs);
  f.table.resize((size_t)seqs * f.shape.max_pages);
  f.k.resize((size_t)f.shape.physical_pages * kPageSize * ps.kv_heads * ps.dim);
  f.v.resize(f.k.size());
  oracle_expand_tree(ps.batch, t.nodes, ps.kv_heads, ps.dim, ps.max_pages, t.prefix.k.data(),
                     t.prefix.v.data(), t.prefix.table.data(), t.prefix.lengths.data(), t.dk.data(),
                     t.dv.data(), t.parent.data(), &longest, &used, f.lengths.data(),
                     f.table.data(), f.k.data(), f.v.data());
  f.q = t.dq;
  return f;
}

// ---- measurement -----------------------------------------------------------------

// The reference timing protocol: kWarm launches, then kTrials trials of kReps
// back-to-back launches between two events, each trial waited for; the
// median trial's time per launch, in microseconds.
struct Protocol {
  static constexpr int kWarm = 5, kTrials = 7, kReps = 20;

  static double median_us(const std::function<hipError_t()>& launch) {
    hipEvent_t ev[2];
    for (auto& e : ev) HIP_OK(hipEventCreate(&e));
    for (int i = 0; i < kWarm; ++i) HIP_OK(launch());
    HIP_OK(hipDeviceSynchronize());
    std::vector<double> per_launch;
    for (int t = 0; t < kTrials; ++t) {
      HIP_OK(hipEventRecord(ev[0]));
      for (int i = 0; i < kReps; ++i) HIP_OK(launch());
      HIP_OK(hipEventRecord(ev[1]));
      HIP_OK(hipEventSynchronize(ev[1]));
      float ms = 0.f;
      HIP_OK(hipEventElapsedTime(&ms, ev[0], ev[1]));
      per_launch.push_back(1e3 * ms / kReps);
    }
    for (auto& e : ev) HIP_OK(hipEventDestroy(e));
    std::nth_element(per_launch.begin(), per_launch.begin() + kTrials / 2, per_launch.end());
    return per_launch[kTrials / 2];
  }
};

struct Device {
  std::string name, arch;
  int cus = 0, runtime = 0;

  static Device current() {
    Device d;
    int id = 0;
    HIP_OK(hipGetDevice(&id));
    hipDeviceProp_t prop{};
    HIP_OK(hipGetDeviceProperties(&prop, id));
    d.arch = prop.gcnArchName;
    d.arch = d.arch.substr(0, d.arch.find(':'));
    d.name = prop.name;
    while (!d.name.empty() && (d.name.back() == ' ' || d.name.back() == '\n')) d.name.pop_back();
    // Some boxes leave the marketing name blank; the CSV's gpu column then
    // names the architecture.
    if (d.name.empty()) d.name = "AMD " + d.arch;
    HIP_OK(hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, id));
    HIP_OK(hipRuntimeGetVersion(&d.runtime));
    return d;
  }
};

// One CSV file in the reference's column schema: times and ratios with three
// decimals, the max difference in scientific notation with eight.
class Csv {
 public:
  Csv(const std::string& path, const char* header) : out_(path) {
    if (!out_) fail("cannot open output: " + path);
    out_ << header << '\n';
  }
  Csv& text(const std::string& s) { return put(s); }
  Csv& quoted(const std::string& s) { return put('"' + s + '"'); }
  Csv& num(long long x) { return put(std::to_string(x)); }
  Csv& fix3(double x) { return put(format(x, std::ios::fixed, 3)); }
  Csv& sci8(double x) { return put(format(x, std::ios::scientific, 8)); }
  void end_row() {
    out_ << '\n';
    out_.flush();
    first_ = true;
  }

 private:
  static std::string format(double x, std::ios::fmtflags how, int digits) {
    std::ostringstream s;
    s.setf(how, std::ios::floatfield);
    s << std::setprecision(digits) << x;
    return s.str();
  }
  Csv& put(const std::string& field) {
    if (!first_) out_ << ',';
    out_ << field;
    first_ = false;
    return *this;
  }
  std::ofstream out_;
  bool first_ = true;
};

template <class F>
double wall_seconds(F&& f) {
  const auto t0 = std::chrono::steady_clock::now();
  f();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

// Algorithmic bytes of a decode: each attended token's K and V once, Q, the
// output, the used page-table entries and the lengths.
double decode_bytes(const Shape& s, const std::vector<int>& lengths, int out_bytes) {
  double tokens = 0, pages = 0;
  for (int n : lengths) {
    tokens += n;
    pages += pages_for(n);
  }
  return tokens * s.kv_heads * s.dim * 4.0 + (double)s.batch * s.query_heads * s.dim * (2 + out_bytes) +
         pages * 4 + s.batch * 4;
}

void report(const char* what, double us, double bytes, double cpu1, double cpun, int cores) {
  std::cout << std::fixed << std::setprecision(3) << what << ": " << us << " us/call, "
            << bytes / us / 1e3 << " GB/s (" << 100.0 * bytes / us / 1e3 / 8000.0
            << "% of 8 TB/s); CPU oracle " << cpu1 * 1e3 << " ms on 1 thread, " << cpun * 1e3
            << " ms on " << cores << " threads\n";
}

// ---- test mode -----------------------------------------------------------------------

constexpr float kGate = 3e-4f;  // the reference driver's gate (src/main.cu:259, :335)

// Decode against the oracle over the reference's cases and split counts
// (src/main.cu:318-341), plus 64 splits; then the API rejections
// (src/main.cu:343-349).
void test_decode() {
  struct Case {
    int batch, hq, hkv, dim;
    std::vector<int> lengths;
  };
  const Case cases[] = {
      {1, 8, 2, 64, {0}},  {1, 8, 2, 64, {1}},           {1, 8, 2, 64, {16}},
      {1, 8, 2, 64, {17}}, {3, 10, 2, 64, {0, 37, 91}}, {3, 12, 3, 128, {7, 128, 257}},
      {2, 32, 8, 128, {513, 3}},
  };
  const int split_counts[] = {1, 2, 4, 8, 16, 64};
  int passed = 0;
  for (const Case& c : cases) {
    const PagedHost host = make_cache({c.batch, c.hq, c.hkv, c.dim, c.lengths});
    const std::vector<float> want = oracle_of(host);
    const PagedDevice dev(host, BC_MAX_SPLITS);
    for (int splits : split_counts) {
      const float err = worst_gap(want, dev.decode_now(splits));
      if (!(err <= kGate)) {
        std::ostringstream m;
        m << "FAIL B=" << c.batch << " D=" << c.dim << " splits=" << splits
          << " max_abs_error=" << std::to_string(err);
        fail(m.str());
      }
      ++passed;
    }
  }
  const PagedHost host = make_cache({1, 8, 2, 64, {17}});
  const PagedDevice dev(host, 2);
  Shape wrong_dim = host.shape;
  wrong_dim.dim = 96;
  const bool rejected =
      branchcraft::decode(wrong_dim, dev.inputs(), dev.scratch(), 1) == hipErrorInvalidValue &&
      branchcraft::decode(host.shape, dev.inputs(), {nullptr, nullptr}, 2) == hipErrorInvalidValue;
  if (!rejected) fail("invalid API arguments were accepted");
  std::cout << "PASS " << passed << " CPU-oracle checks across empty, page-boundary,"
            << " ragged, GQA, D64/D128, and split-KV cases.\n";
}

// Two requests share a 17-token prefix whose second page is partial.  The
// first request accepts the path 0 -> 1 -> 3: its shared partial page is
// cloned into the pool's last page, the three nodes are committed into slots
// 1-3 of the clone, and decode over the committed table must then equal the
// tree's output for node 3, leave the sibling request unchanged, and come
// back exactly after the table is rolled back (src/main.cu:264-313).
class CommitScenario {
 public:
  CommitScenario() : host_(make_tree(2, 17, 7, 128, 49)), dev_(host_) {}

  void run() {
    tree_out_ = dev_.verify_now();
    before_ = dev_.prefix().decode_now(1);
    clone_and_commit();
    check_pages();
    check_committed_decode();
    check_rollback();
  }

 private:
  static constexpr int kPath[3] = {0, 1, 3};

  const Shape& shape() const { return host_.prefix.shape; }
  int fresh_page() const { return shape().physical_pages - 1; }
  int shared_page() const { return host_.prefix.table[1]; }
  size_t query_elems() const { return (size_t)shape().query_heads * shape().dim; }

  void clone_and_commit() {
    PagedDevice& p = dev_.prefix();
    const auto src = DevArray<int>::copy_of(std::vector<int>{shared_page()});
    const auto dst = DevArray<int>::copy_of(std::vector<int>{fresh_page()});
    HIP_OK(branchcraft::copy_pages(shape(), p.k().get(), p.v().get(), src.get(), dst.get(), 1));
    const auto nodes = DevArray<int>::copy_of(std::vector<int>(kPath, kPath + 3));
    const auto pages = DevArray<int>::copy_of(std::vector<int>(3, fresh_page()));
    const auto slots = DevArray<int>::copy_of(std::vector<int>{1, 2, 3});
    HIP_OK(branchcraft::commit_path(shape(), dev_.draft_k().get(), dev_.draft_v().get(),
                                    p.k().get(), p.v().get(), nodes.get(), pages.get(), slots.get(),
                                    0, host_.nodes, 3));
    HIP_OK(hipDeviceSynchronize());
  }

  // The pool after the clone and the commit, bit for bit, against the
  // oracle's restatement of both steps.
  void check_pages() {
    std::vector<bits16> k = host_.prefix.k, v = host_.prefix.v;
    const int src[1] = {shared_page()}, dst[1] = {fresh_page()};
    oracle_copy_pages(shape().kv_heads, shape().dim, shape().physical_pages, k.data(), v.data(), src,
                      dst, 1);
    const int pages[3] = {fresh_page(), fresh_page(), fresh_page()}, slots[3] = {1, 2, 3};
    oracle_commit(shape().batch, host_.nodes, shape().kv_heads, shape().dim, shape().physical_pages,
                  host_.dk.data(), host_.dv.data(), k.data(), v.data(), kPath, pages, slots, 0, 3);
    if (dev_.prefix().k().read<bits16>() != k || dev_.prefix().v().read<bits16>() != v)
      fail("commit pages differ from the oracle");
  }

  // Request 0 now ends with the accepted nodes and asks with node 3's query.
  void check_committed_decode() {
    PagedDevice& p = dev_.prefix();
    std::vector<int> table = host_.prefix.table, lengths = host_.prefix.lengths;
    table[1] = fresh_page();
    lengths[0] += 3;
    p.table().write(table);
    p.lengths().write(lengths);
    HIP_OK(hipMemcpy(p.q().get(), dev_.draft_q().get() + 3 * query_elems(),
                     query_elems() * sizeof(bits16), hipMemcpyDeviceToDevice));
    const std::vector<float> after = p.decode_now(1);
    float accepted = 0.f, sibling = 0.f;
    for (size_t i = 0; i < query_elems(); ++i) {
      accepted = std::max(accepted, std::fabs(after[i] - tree_out_[3 * query_elems() + i]));
      sibling = std::max(sibling, std::fabs(after[query_elems() + i] - before_[query_elems() + i]));
    }
    if (!(accepted <= kGate) || !(sibling <= 1e-7f))
      fail("commit changed accepted path or shared sibling");
  }

  void check_rollback() {
    PagedDevice& p = dev_.prefix();
    p.table().write(host_.prefix.table);
    p.lengths().write(host_.prefix.lengths);
    p.q().write(host_.prefix.q);
    if (!(worst_gap(before_, p.decode_now(1)) <= 1e-7f)) fail("rollback failed");
  }

  TreeHost host_;
  TreeDevice dev_;
  std::vector<float> tree_out_, before_;
};

// Tree verification against the oracle (empty, partial-page and
// multi-page prefixes; src/main.cu:253-262), then the commit scenario.
void test_tree() {
  struct Case {
    int prefix, dim;
  };
  int passed = 0;
  for (const Case c : {Case{0, 64}, Case{17, 64}, Case{257, 128}}) {
    const TreeHost t = make_tree(2, c.prefix, 7, c.dim);
    const float err = worst_gap(oracle_of(t), TreeDevice(t).verify_now());
    if (!(err <= kGate)) fail("tree CPU-oracle mismatch, max error=" + std::to_string(err));
    ++passed;
  }
  CommitScenario().run();
  std::cout << "PASS " << passed << " tree CPU-oracle cases plus shared-page"
            << " commit, sibling isolation, and rollback.\n";
}

// ---- bench / tree-bench sweeps ------------------------------------------------------------

// Decode sweep (src/main.cu:446-488): per batch and context, splits 1
// against the library's choice, the chosen split's output checked against
// splits 1.
void bench_decode(const std::string& path, bool quick) {
  const Device dev = Device::current();
  Csv csv(path,
          "gpu,sm,cuda_runtime,batch,query_heads,kv_heads,head_dim,context,"
          "page_size,splits,single_us,split_us,speedup,max_abs_diff,kv_mib");
  const std::vector<int> batches = quick ? std::vector<int>{1, 8} : std::vector<int>{1, 4, 16, 32};
  const std::vector<int> contexts =
      quick ? std::vector<int>{256, 2048} : std::vector<int>{256, 1024, 4096, 8192};
  for (int batch : batches)
    for (int context : contexts) {
      std::vector<int> lengths(batch);
      for (int i = 0; i < batch; ++i) lengths[i] = context - (i % 4) * context / 8;
      const PagedHost host =
          make_cache({batch, 32, 8, 128, lengths, (uint32_t)(17 + batch + context)});
      const PagedDevice gpu(host, BC_MAX_SPLITS);
      const int splits = branchcraft::auto_splits(host.shape, context, dev.cus, BC_MAX_SPLITS);
      const float diff = worst_gap(gpu.decode_now(1), gpu.decode_now(splits));
      if (!(diff <= kGate)) fail("benchmark split output mismatch");
      const double single = Protocol::median_us([&] { return gpu.decode(1); });
      const double chosen = splits == 1 ? single : Protocol::median_us([&] { return gpu.decode(splits); });
      const double kv_mib = (double)(host.k.size() + host.v.size()) * sizeof(bits16) / (1 << 20);
      const double tokens = std::accumulate(lengths.begin(), lengths.end(), 0.0);
      csv.quoted(dev.name).text(dev.arch).num(dev.runtime).num(batch).num(32).num(8).num(128)
          .num(context).num(kPageSize).num(splits).fix3(single).fix3(chosen).fix3(single / chosen)
          .sci8(diff).fix3(kv_mib).end_row();
      std::cout << "B=" << batch << " S=" << context << " split=" << splits << " single=" << single
                << "us chosen=" << chosen << "us speedup=" << single / chosen
                << " GB/s=" << tokens * 4096.0 / chosen / 1e3 << " diff=" << diff << '\n';
    }
  std::cout << "Wrote " << path << '\n';
}

// Tree sweep (src/main.cu:490-525): the tree call against the expanded-prefix
// decode, their outputs checked against each other, and the KV bytes each
// holds.
void bench_tree(const std::string& path, bool quick) {
  const Device dev = Device::current();
  Csv csv(path,
          "gpu,sm,cuda_runtime,requests,tree_nodes,prefix_tokens,query_heads,"
          "kv_heads,head_dim,page_size,tree_us,expanded_us,latency_ratio,"
          "max_abs_diff,shared_kv_mib,expanded_kv_mib,memory_saving_pct");
  const std::vector<int> batches = quick ? std::vector<int>{1, 4} : std::vector<int>{1, 4, 8};
  const std::vector<int> contexts =
      quick ? std::vector<int>{256, 1024} : std::vector<int>{256, 1024, 2048};
  const double bytes_per_slot = 8.0 * 128 * sizeof(bits16) * 2;
  for (int batch : batches)
    for (int context : contexts) {
      const TreeHost t = make_tree(batch, context, 7, 128, (uint32_t)(91 + batch + context));
      const PagedHost flat_host = expand(t);
      const TreeDevice tree(t);
      const PagedDevice flat(flat_host, 1);
      const float diff = worst_gap(tree.verify_now(), flat.decode_now(1));
      if (!(diff <= kGate)) fail("expanded-cache output mismatch");
      const double tree_us = Protocol::median_us([&] { return tree.verify(); });
      const double flat_us = Protocol::median_us([&] { return flat.decode(1); });
      const double shared_slots = (double)pages_for(context) * kPageSize + batch * t.nodes;
      double flat_slots = 0;
      for (int n : flat_host.lengths) flat_slots += (double)pages_for(n) * kPageSize;
      const double shared_mib = shared_slots * bytes_per_slot / (1 << 20);
      const double flat_mib = flat_slots * bytes_per_slot / (1 << 20);
      const double saving = 100.0 * (1.0 - shared_mib / flat_mib);
      csv.quoted(dev.name).text(dev.arch).num(dev.runtime).num(batch).num(7).num(context).num(32)
          .num(8).num(128).num(kPageSize).fix3(tree_us).fix3(flat_us).fix3(flat_us / tree_us)
          .sci8(diff).fix3(shared_mib).fix3(flat_mib).fix3(saving).end_row();
      std::cout << "tree B=" << batch << " S=" << context << " tree=" << tree_us
                << "us expanded=" << flat_us << "us ratio=" << flat_us / tree_us
                << "x KV saved=" << saving << "%\n";
    }
  std::cout << "Wrote " << path << '\n';
}

// ---- config N: the benchmark configurations ------------------------------------------------

int host_threads() { return (int)std::max(1u, std::thread::hardware_concurrency()); }

// Configs 1 and 4: paged decode with the library's split count; FP32 output
// at the reference decode gate (src/main.cu:335).
void config_decode(int n, const Device& dev) {
  PagedHost host;
  if (n == 1) {
    host = make_cache({1, 32, 8, 128, {512}, 1, 1.0f, 32});  // 64-page pool
  } else {
    Gen gen(4);
    std::vector<int> lengths(4);
    for (int& x : lengths) x = 16384 + (int)gen.below(16385);
    host = make_cache({4, 32, 8, 128, lengths, 4, 1.0f, 16});
  }
  const PagedDevice gpu(host, BC_MAX_SPLITS);
  const int longest = *std::max_element(host.lengths.begin(), host.lengths.end());
  const int splits = branchcraft::auto_splits(host.shape, longest, dev.cus, BC_MAX_SPLITS);
  std::vector<float> want;
  const double cpu1 = wall_seconds([&] { want = oracle_of(host, 1); });
  const double cpun = wall_seconds([&] { (void)oracle_of(host, host_threads()); });
  const float err = worst_gap(want, gpu.decode_now(splits));
  const double us = Protocol::median_us([&] { return gpu.decode(splits); });
  std::cout << "config " << n << " splits=" << splits << " max_abs_error=" << err << '\n';
  report("paged decode", us, decode_bytes(host.shape, host.lengths, 4), cpu1, cpun, host_threads());
  if (!(err <= kGate)) fail("config parity failed");
}

// Configs 2 and 3: tree verification (random parents) at the reference tree
// gate (src/main.cu:259), with the expanded-prefix decode beside it.
void config_tree(int n, const Device& dev) {
  const int batch = n == 2 ? 1 : 8, prefix = n == 2 ? 2048 : 2053;
  const TreeHost t = make_tree(batch, prefix, 7, 128, (uint32_t)(100 + n), 1.0f, Parents::kRandom);
  const TreeDevice gpu(t);
  std::vector<float> want;
  const double cpu1 = wall_seconds([&] { want = oracle_of(t, 1); });
  const double cpun = wall_seconds([&] { (void)oracle_of(t, host_threads()); });
  const float err = worst_gap(want, gpu.verify_now());
  const double us = Protocol::median_us([&] { return gpu.verify(); });
  const double bytes = prefix * 4096.0 + batch * 7.0 * (8 * 128 * 4 + 32 * 128 * 6);
  std::cout << "config " << n << " max_abs_error=" << err << '\n';
  report("tree_verify", us, bytes, cpu1, cpun, host_threads());
  const PagedHost flat_host = expand(t);
  const PagedDevice flat(flat_host, BC_MAX_SPLITS);
  const int splits = branchcraft::auto_splits(flat_host.shape, prefix + 7, dev.cus, BC_MAX_SPLITS);
  const double one = Protocol::median_us([&] { return flat.decode(1); });
  const double auto_split = Protocol::median_us([&] { return flat.decode(splits); });
  std::cout << std::fixed << std::setprecision(3) << "expanded-prefix decode: " << one
            << " us (splits 1), " << auto_split << " us (splits " << splits
            << "); expanded/tree = " << std::min(one, auto_split) / us << "x\n";
  if (!(err <= kGate)) fail("config parity failed");
}

// Config 5: packed decode over a [20000, 2, 16, 8, 128] FP16 cache, batch 64,
// contexts U[128, 4096], FP16 output gated at 2e-3 plus half an FP16 ulp of
// the expected value (the output's own rounding).
void config_packed() {
  constexpr int B = 64, kBlocks = 20000, kMaxPages = 256, HQ = 32, HKV = 8, D = 128;
  Gen gen(5);
  std::vector<int> lengths(B), table((size_t)B * kMaxPages, -1);
  for (int& x : lengths) x = 128 + (int)gen.below(3969);
  const std::vector<int> order = gen.permutation(kBlocks);
  auto next = order.begin();
  for (int b = 0; b < B; ++b)
    for (int p = 0; p < pages_for(lengths[b]); ++p) table[(size_t)b * kMaxPages + p] = *next++;
  const std::vector<bits16> cache = gen.halves((size_t)kBlocks * 2 * 16 * HKV * D, 1.0f);
  const std::vector<bits16> q = gen.halves((size_t)B * HQ * D, 1.0f);
  const auto dcache = DevArray<half>::copy_of(cache);
  const auto dq = DevArray<half>::copy_of(q);
  const auto dtable = DevArray<int>::copy_of(table);
  const auto dlengths = DevArray<int>::copy_of(lengths);
  DevArray<half> dout(q.size());
  const Shape s{B, HQ, HKV, D, kMaxPages, kBlocks};
  DevArray<char> ws(branchcraft::packed_decode_workspace_size(s));
  // Element strides of [block, K/V, slot, head, dim].
  const long long block = 2LL * 16 * HKV * D, head = D, slot = (long long)HKV * D,
                  kv = 16LL * HKV * D;
  const float scale = 1.0f / std::sqrt((float)D);
  auto launch = [&] {
    return branchcraft::packed_decode(s, dq.get(), dcache.get(), dtable.get(), dlengths.get(),
                                      dout.get(), block, head, slot, kv, scale, ws.get(), ws.size());
  };
  std::vector<float> want(q.size()), scratch_out(q.size());
  auto oracle = [&](std::vector<float>& out, int threads) {
    oracle_packed_decode(B, HQ, HKV, D, kMaxPages, q.data(), cache.data(), table.data(),
                         lengths.data(), block, head, slot, kv, scale, out.data(), nullptr, threads);
  };
  const double cpu1 = wall_seconds([&] { oracle(want, 1); });
  const double cpun = wall_seconds([&] { oracle(scratch_out, host_threads()); });
  HIP_OK(launch());
  HIP_OK(hipDeviceSynchronize());
  const std::vector<bits16> got = dout.read<bits16>();
  float err = 0.f, over = -1.f;
  for (size_t i = 0; i < got.size(); ++i) {
    const float diff = std::fabs(oracle_h2f(got[i]) - want[i]);
    const bits16 h = oracle_f2h(std::fabs(want[i]));
    const float ulp = oracle_h2f((bits16)(h + 1)) - oracle_h2f(h);
    err = std::max(err, diff);
    over = std::max(over, diff - (2e-3f + 0.5f * ulp));
  }
  const double us = Protocol::median_us(launch);
  std::cout << "config 5 max_abs_error(fp16 out vs fp32 oracle)=" << err << '\n';
  report("packed decode", us, decode_bytes(s, lengths, 2), cpu1, cpun, host_threads());
  if (!(over <= 0.f)) fail("config parity failed");
}

void run_config(int n) {
  const Device dev = Device::current();
  std::cout << "device " << dev.name << " (" << dev.arch << ", " << dev.cus
            << " CUs); host threads " << std::thread::hardware_concurrency() << '\n';
  switch (n) {
    case 1:
    case 4:
      config_decode(n, dev);
      break;
    case 2:
    case 3:
      config_tree(n, dev);
      break;
    case 5:
      config_packed();
      break;
    default:
      fail("config must be 1..5");
  }
}

// ---- command line ----------------------------------------------------------------------------

int main_impl(const std::vector<std::string>& args) {
  if (args.empty()) {
    std::cerr << "Usage: branchcraft test | bench | tree-bench [--quick] [--output FILE]"
                 " | config N\n";
    return 2;
  }
  const std::string& mode = args[0];
  if (mode == "test") {
    test_decode();
    test_tree();
    return 0;
  }
  if (mode == "config") {
    if (args.size() < 2) fail("config needs N (1..5)");
    run_config(std::stoi(args[1]));
    return 0;
  }
  if (mode != "bench" && mode != "tree-bench") fail("unknown mode: " + mode);
  bool quick = false;
  std::string path = mode == "bench" ? "decode_results.csv" : "tree_results.csv";
  for (size_t i = 1; i < args.size(); ++i) {
    if (args[i] == "--quick") quick = true;
    else if (args[i] == "--output" && i + 1 < args.size()) path = args[++i];
    else fail("unknown or incomplete argument: " + args[i]);
  }
  if (mode == "bench") bench_decode(path, quick);
  else bench_tree(path, quick);
  return 0;
}

}  // namespace drv

int main(int argc, char** argv) {
  try {
    return drv::main_impl(std::vector<std::string>(argv + 1, argv + argc));
  } catch (const std::exception& e) {
    std::cerr << "ERROR: " << e.what() << '\n';
    return 1;
  }
}
