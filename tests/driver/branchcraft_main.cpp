// Standalone Branchcraft driver for MI355X: `branchcraft test | bench |
// tree-bench [--quick] [--output FILE]` and `branchcraft config N`.
//
// Restates the reference driver (src/main.cu of Haaziq386/branchcraft-cuda):
// the same test cases and 3e-4 gates (:252-352), the same benchmark sweeps,
// timing protocol (5 warm-ups, 7 trials x 20 launches, median; :354-373) and
// CSV columns (:451-453, :495-496), plus `config N` for the five benchmark
// configurations with the CPU oracle timed on this host.  Kernels are reached
// only through the C ABI (include/branchcraft.hpp); the HIP runtime is used
// for device memory and events.  This is test and measurement tooling: it
// links the CPU oracle (oracle/bc_oracle.c) as its checker.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "bc_oracle.h"
#include "branchcraft.hpp"

using branchcraft::kPageSize;
using branchcraft::Shape;
using h16 = uint16_t;

#define CHECK(call)                                                               \
  do {                                                                            \
    hipError_t e_ = (call);                                                       \
    if (e_ != hipSuccess)                                                         \
      throw std::runtime_error(std::string(#call) + ": " + hipGetErrorString(e_)); \
  } while (0)

template <typename T>
struct DeviceBuffer {
  T* ptr = nullptr;
  size_t count = 0;
  DeviceBuffer() = default;
  explicit DeviceBuffer(size_t n) : count(n) {
    CHECK(hipMalloc(reinterpret_cast<void**>(&ptr), std::max<size_t>(1, n) * sizeof(T)));
  }
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  ~DeviceBuffer() {
    if (ptr) (void)hipFree(ptr);
  }
  void upload(const std::vector<T>& v) { upload<T>(v); }
  // Host data of another element type with the same size: FP16 bit patterns
  // (uint16_t) into `half` buffers.
  template <typename U>
  void upload(const std::vector<U>& v) {
    static_assert(sizeof(U) == sizeof(T), "same element size");
    if (v.size() != count) throw std::runtime_error("upload size mismatch");
    CHECK(hipMemcpy(ptr, v.data(), count * sizeof(T), hipMemcpyHostToDevice));
  }
  template <typename U = T>
  std::vector<U> download() const {
    static_assert(sizeof(U) == sizeof(T), "same element size");
    std::vector<U> v(count);
    CHECK(hipMemcpy(v.data(), ptr, count * sizeof(T), hipMemcpyDeviceToHost));
    return v;
  }
};

// ---- portable fixtures ----------------------------------------------------
// std::mt19937 is fully specified; the normal and shuffle steps are written
// here (Box-Muller, Fisher-Yates) so fixtures do not depend on the library.

struct Rng {
  std::mt19937 gen;
  explicit Rng(uint32_t seed) : gen(seed) {}
  double uniform01() { return (gen() + 0.5) * (1.0 / 4294967296.0); }
  uint32_t below(uint32_t n) {  // unbiased integer in [0, n)
    const uint32_t lim = 0xffffffffu - 0xffffffffu % n;
    uint32_t x;
    do x = gen(); while (x >= lim);
    return x % n;
  }
  float normal(float sigma) {
    const double u1 = uniform01(), u2 = uniform01();
    return (float)(sigma * std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
  void shuffle(std::vector<int>& v) {
    for (size_t i = v.size(); i > 1; --i) std::swap(v[i - 1], v[below((uint32_t)i)]);
  }
  void fill(std::vector<h16>& v, float sigma) {
    for (auto& x : v) x = oracle_f2h(normal(sigma));
  }
};

struct Fixture {
  Shape shape;
  std::vector<h16> q, k, v;
  std::vector<int> pages, lengths;
};

// Shuffled page ids, `spare` extra pages, N(0, sigma) FP16 (src/main.cu:48-79).
Fixture make_fixture(int batch, int hq, int hkv, int dim, std::vector<int> lengths,
                     uint32_t seed = 17, float sigma = 0.5f, int spare = 7) {
  if ((int)lengths.size() != batch) throw std::runtime_error("length count mismatch");
  const int max_len = *std::max_element(lengths.begin(), lengths.end());
  const int max_pages = std::max(1, (max_len + kPageSize - 1) / kPageSize);
  int used = 0;
  for (int n : lengths) used += (n + kPageSize - 1) / kPageSize;
  const int phys = used + spare;
  Fixture f{{batch, hq, hkv, dim, max_pages, phys}, {}, {}, {}, {}, {}};
  f.lengths = std::move(lengths);
  f.pages.assign((size_t)batch * max_pages, -1);
  Rng rng(seed);
  std::vector<int> ids(phys);
  std::iota(ids.begin(), ids.end(), 0);
  rng.shuffle(ids);
  int cur = 0;
  for (int b = 0; b < batch; ++b)
    for (int p = 0; p < (f.lengths[b] + kPageSize - 1) / kPageSize; ++p)
      f.pages[(size_t)b * max_pages + p] = ids[cur++];
  f.q.resize((size_t)batch * hq * dim);
  f.k.resize((size_t)phys * kPageSize * hkv * dim);
  f.v.resize(f.k.size());
  rng.fill(f.q, sigma);
  rng.fill(f.k, sigma);
  rng.fill(f.v, sigma);
  return f;
}

std::vector<float> cpu_decode(const Fixture& f, int threads = 1) {
  const Shape s = f.shape;
  std::vector<float> out((size_t)s.batch * s.query_heads * s.dim);
  oracle_decode(s.batch, s.query_heads, s.kv_heads, s.dim, s.max_pages, f.q.data(),
                f.k.data(), f.v.data(), f.pages.data(), f.lengths.data(), out.data(), threads);
  return out;
}

float max_abs_error(const std::vector<float>& a, const std::vector<float>& b) {
  if (a.size() != b.size()) throw std::runtime_error("comparison size mismatch");
  return oracle_max_abs_error(a.data(), b.data(), a.size());
}

struct GpuFixture {
  DeviceBuffer<half> q, k, v;
  DeviceBuffer<int> pages, lengths;
  DeviceBuffer<float> output, partial_a, partial_ml;
  Shape shape;
  int max_splits;
  explicit GpuFixture(const Fixture& f, int max_splits = BC_MAX_SPLITS)
      : q(f.q.size()), k(f.k.size()), v(f.v.size()), pages(f.pages.size()),
        lengths(f.lengths.size()),
        output((size_t)f.shape.batch * f.shape.query_heads * f.shape.dim),
        partial_a((size_t)max_splits * output.count),
        partial_ml((size_t)max_splits * f.shape.batch * f.shape.query_heads * 2),
        shape(f.shape), max_splits(max_splits) {
    q.upload(f.q);
    k.upload(f.k);
    v.upload(f.v);
    pages.upload(f.pages);
    lengths.upload(f.lengths);
  }
  branchcraft::Inputs inputs() { return {q.ptr, k.ptr, v.ptr, pages.ptr, lengths.ptr, output.ptr}; }
  branchcraft::Scratch scratch() { return {partial_a.ptr, partial_ml.ptr}; }
  hipError_t launch(int splits) { return branchcraft::decode(shape, inputs(), scratch(), splits); }
  void run(int splits) {
    CHECK(launch(splits));
    CHECK(hipDeviceSynchronize());
  }
};

// ---- tree fixtures ----------------------------------------------------------

struct TreeFixture {
  Fixture prefix;
  int nodes;
  std::vector<h16> draft_q, draft_k, draft_v;
  std::vector<int> parent;
};

// All requests share one prefix page list and query (src/main.cu:145-179);
// parents binary (n-1)/2 or uniform in [0, n-1].
TreeFixture make_tree_fixture(int batch, int prefix_len, int nodes, int dim, uint32_t seed = 31,
                              float sigma = 0.5f, bool random_parents = false) {
  Fixture base = make_fixture(1, 32, 8, dim, {prefix_len}, seed, sigma);
  TreeFixture t{};
  t.nodes = nodes;
  Fixture& f = t.prefix;
  f.shape = {batch, 32, 8, dim, base.shape.max_pages + 2, base.shape.physical_pages + batch * 2};
  f.lengths.assign(batch, prefix_len);
  f.pages.assign((size_t)batch * f.shape.max_pages, -1);
  for (int b = 0; b < batch; ++b)
    for (int p = 0; p < (prefix_len + kPageSize - 1) / kPageSize; ++p)
      f.pages[(size_t)b * f.shape.max_pages + p] = base.pages[p];
  f.q.resize((size_t)batch * 32 * dim);
  for (int b = 0; b < batch; ++b)
    std::copy(base.q.begin(), base.q.end(), f.q.begin() + (size_t)b * 32 * dim);
  f.k = std::move(base.k);
  f.v = std::move(base.v);
  f.k.resize((size_t)f.shape.physical_pages * kPageSize * 8 * dim, 0);
  f.v.resize(f.k.size(), 0);
  Rng rng(seed + 99);
  t.draft_q.resize((size_t)batch * nodes * 32 * dim);
  t.draft_k.resize((size_t)batch * nodes * 8 * dim);
  t.draft_v.resize(t.draft_k.size());
  rng.fill(t.draft_q, sigma);
  rng.fill(t.draft_k, sigma);
  rng.fill(t.draft_v, sigma);
  t.parent.resize((size_t)batch * nodes);
  for (int b = 0; b < batch; ++b)
    for (int n = 0; n < nodes; ++n)
      t.parent[(size_t)b * nodes + n] =
          n == 0 ? -1 : (random_parents ? (int)rng.below((uint32_t)n) : (n - 1) / 2);
  return t;
}

std::vector<float> cpu_tree(const TreeFixture& t, int threads = 1) {
  const Shape s = t.prefix.shape;
  std::vector<float> out(t.draft_q.size());
  oracle_tree(s.batch, t.nodes, s.query_heads, s.kv_heads, s.dim, s.max_pages,
              t.prefix.k.data(), t.prefix.v.data(), t.prefix.pages.data(),
              t.prefix.lengths.data(), t.draft_q.data(), t.draft_k.data(), t.draft_v.data(),
              t.parent.data(), out.data(), threads);
  return out;
}

struct TreeGpu {
  GpuFixture prefix;
  DeviceBuffer<half> draft_q, draft_k, draft_v;
  DeviceBuffer<int> parent;
  DeviceBuffer<float> output;
  DeviceBuffer<char> workspace;
  int nodes;
  explicit TreeGpu(const TreeFixture& t)
      : prefix(t.prefix, 1), draft_q(t.draft_q.size()), draft_k(t.draft_k.size()),
        draft_v(t.draft_v.size()), parent(t.parent.size()), output(t.draft_q.size()),
        workspace(branchcraft::tree_verify_workspace_size(t.prefix.shape, t.nodes)),
        nodes(t.nodes) {
    draft_q.upload(t.draft_q);
    draft_k.upload(t.draft_k);
    draft_v.upload(t.draft_v);
    parent.upload(t.parent);
  }
  branchcraft::TreeInputs inputs() {
    return {prefix.inputs(), draft_q.ptr, draft_k.ptr, draft_v.ptr, parent.ptr, output.ptr};
  }
  hipError_t launch() {
    return branchcraft::tree_verify(prefix.shape, inputs(), nodes, workspace.ptr,
                                    workspace.count);
  }
  void run() {
    CHECK(launch());
    CHECK(hipDeviceSynchronize());
  }
};

// ---- timing -------------------------------------------------------------------

template <typename F>
double median_latency_us(F&& launch, int repeats = 20) {
  hipEvent_t start, stop;
  CHECK(hipEventCreate(&start));
  CHECK(hipEventCreate(&stop));
  for (int i = 0; i < 5; ++i) CHECK(launch());
  CHECK(hipDeviceSynchronize());
  std::vector<double> times;
  for (int trial = 0; trial < 7; ++trial) {
    CHECK(hipEventRecord(start));
    for (int i = 0; i < repeats; ++i) CHECK(launch());
    CHECK(hipEventRecord(stop));
    CHECK(hipEventSynchronize(stop));
    float ms = 0;
    CHECK(hipEventElapsedTime(&ms, start, stop));
    times.push_back((double)ms * 1000.0 / repeats);
  }
  CHECK(hipEventDestroy(start));
  CHECK(hipEventDestroy(stop));
  std::sort(times.begin(), times.end());
  return times[times.size() / 2];
}

int cu_count() {
  int dev = 0, n = 0;
  CHECK(hipGetDevice(&dev));
  CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
  return n;
}

std::string device_arch() {
  hipDeviceProp_t prop{};
  CHECK(hipGetDeviceProperties(&prop, 0));
  std::string a = prop.gcnArchName;
  return a.substr(0, a.find(':'));
}

// The marketing name when the runtime reports one; some boxes leave
// hipDeviceProp_t::name blank, and the CSV's gpu column then names the
// architecture instead.
std::string device_name() {
  hipDeviceProp_t prop{};
  CHECK(hipGetDeviceProperties(&prop, 0));
  std::string n = prop.name;
  while (!n.empty() && (n.back() == ' ' || n.back() == '\n')) n.pop_back();
  return n.empty() ? "AMD " + device_arch() : n;
}

int runtime_version() {
  int v = 0;
  CHECK(hipRuntimeGetVersion(&v));
  return v;
}

// ---- test mode ------------------------------------------------------------------

void run_tests() {
  struct Case {
    int b, hq, hkv, d;
    std::vector<int> lens;
  };
  const std::vector<Case> cases = {
      {1, 8, 2, 64, {0}},           {1, 8, 2, 64, {1}},         {1, 8, 2, 64, {16}},
      {1, 8, 2, 64, {17}},          {3, 10, 2, 64, {0, 37, 91}}, {3, 12, 3, 128, {7, 128, 257}},
      {2, 32, 8, 128, {513, 3}},
  };
  int checks = 0;
  for (const auto& c : cases) {
    Fixture f = make_fixture(c.b, c.hq, c.hkv, c.d, c.lens);
    const auto expected = cpu_decode(f);
    GpuFixture gpu(f);
    for (int splits : {1, 2, 4, 8, 16, 64}) {
      gpu.run(splits);
      const float error = max_abs_error(expected, gpu.output.download());
      if (!(error <= 3e-4f))
        throw std::runtime_error("FAIL B=" + std::to_string(c.b) + " D=" + std::to_string(c.d) +
                                 " splits=" + std::to_string(splits) +
                                 " max_abs_error=" + std::to_string(error));
      ++checks;
    }
  }
  // The API rejects unsupported dimensions and missing split scratch
  // (src/main.cu:343-349).
  Fixture f = make_fixture(1, 8, 2, 64, {17});
  GpuFixture gpu(f);
  Shape bad = f.shape;
  bad.dim = 96;
  if (branchcraft::decode(bad, gpu.inputs(), gpu.scratch(), 1) != hipErrorInvalidValue ||
      branchcraft::decode(f.shape, gpu.inputs(), {nullptr, nullptr}, 2) != hipErrorInvalidValue)
    throw std::runtime_error("invalid API arguments were accepted");
  std::cout << "PASS " << checks << " CPU-oracle checks across empty, page-boundary,"
            << " ragged, GQA, D64/D128, and split-KV cases.\n";
}

void run_tree_tests() {
  int checks = 0;
  for (const auto& spec : std::vector<std::pair<int, int>>{{0, 64}, {17, 64}, {257, 128}}) {
    TreeFixture t = make_tree_fixture(2, spec.first, 7, spec.second);
    TreeGpu gpu(t);
    gpu.run();
    const float error = max_abs_error(cpu_tree(t), gpu.output.download());
    if (!(error <= 3e-4f))
      throw std::runtime_error("tree CPU-oracle mismatch, max error=" + std::to_string(error));
    ++checks;
  }
  // Two requests share a partial final page: clone it, write the accepted
  // root->leaf path, check against tree attention, then roll back
  // (src/main.cu:264-313).
  TreeFixture t = make_tree_fixture(2, 17, 7, 128, 49);
  TreeGpu gpu(t);
  gpu.run();
  const auto tree_out = gpu.output.download();
  gpu.prefix.run(1);
  const auto before = gpu.prefix.output.download();
  const int new_page = t.prefix.shape.physical_pages - 1;
  const int old_page = t.prefix.pages[1];
  DeviceBuffer<int> src(1), dst(1), path(3), dest_pages(3), dest_slots(3);
  src.upload({old_page});
  dst.upload({new_page});
  CHECK(branchcraft::copy_pages(t.prefix.shape, gpu.prefix.k.ptr, gpu.prefix.v.ptr, src.ptr,
                                dst.ptr, 1));
  path.upload({0, 1, 3});
  dest_pages.upload({new_page, new_page, new_page});
  dest_slots.upload({1, 2, 3});
  CHECK(branchcraft::commit_path(t.prefix.shape, gpu.draft_k.ptr, gpu.draft_v.ptr,
                                 gpu.prefix.k.ptr, gpu.prefix.v.ptr, path.ptr, dest_pages.ptr,
                                 dest_slots.ptr, 0, t.nodes, 3));
  CHECK(hipDeviceSynchronize());
  // The device pages must equal the oracle's clone + commit, bit for bit.
  std::vector<h16> ek = t.prefix.k, ev = t.prefix.v;
  const int sp[1] = {old_page}, dp[1] = {new_page};
  oracle_copy_pages(8, 128, t.prefix.shape.physical_pages, ek.data(), ev.data(), sp, dp, 1);
  const int pn[3] = {0, 1, 3}, pg[3] = {new_page, new_page, new_page}, sl[3] = {1, 2, 3};
  oracle_commit(2, t.nodes, 8, 128, t.prefix.shape.physical_pages, t.draft_k.data(),
                t.draft_v.data(), ek.data(), ev.data(), pn, pg, sl, 0, 3);
  if (gpu.prefix.k.download<h16>() != ek || gpu.prefix.v.download<h16>() != ev)
    throw std::runtime_error("commit pages differ from the oracle");
  auto committed_pages = t.prefix.pages;
  auto committed_lengths = t.prefix.lengths;
  committed_pages[1] = new_page;
  committed_lengths[0] += 3;
  gpu.prefix.pages.upload(committed_pages);
  gpu.prefix.lengths.upload(committed_lengths);
  const size_t query_elems = (size_t)t.prefix.shape.query_heads * t.prefix.shape.dim;
  CHECK(hipMemcpy(gpu.prefix.q.ptr, gpu.draft_q.ptr + 3 * query_elems, query_elems * sizeof(h16),
                  hipMemcpyDeviceToDevice));
  gpu.prefix.run(1);
  const auto after = gpu.prefix.output.download();
  float accepted_error = 0, sibling_error = 0;
  for (size_t i = 0; i < query_elems; ++i) {
    accepted_error = std::max(accepted_error, std::fabs(after[i] - tree_out[3 * query_elems + i]));
    sibling_error =
        std::max(sibling_error, std::fabs(after[query_elems + i] - before[query_elems + i]));
  }
  if (!(accepted_error <= 3e-4f) || !(sibling_error <= 1e-7f))
    throw std::runtime_error("commit changed accepted path or shared sibling");
  gpu.prefix.pages.upload(t.prefix.pages);
  gpu.prefix.lengths.upload(t.prefix.lengths);
  gpu.prefix.q.upload(t.prefix.q);
  gpu.prefix.run(1);
  if (!(max_abs_error(before, gpu.prefix.output.download()) <= 1e-7f))
    throw std::runtime_error("rollback failed");
  std::cout << "PASS " << checks << " tree CPU-oracle cases plus shared-page"
            << " commit, sibling isolation, and rollback.\n";
}

// ---- bench / tree-bench -------------------------------------------------------------

void run_bench(const std::string& path, bool quick) {
  std::ofstream out(path);
  if (!out) throw std::runtime_error("cannot open output: " + path);
  out << "gpu,sm,cuda_runtime,batch,query_heads,kv_heads,head_dim,context,"
         "page_size,splits,single_us,split_us,speedup,max_abs_diff,kv_mib\n";
  const int cus = cu_count();
  const std::string name = device_name(), arch = device_arch();
  const int rt = runtime_version();
  const auto batches = quick ? std::vector<int>{1, 8} : std::vector<int>{1, 4, 16, 32};
  const auto contexts = quick ? std::vector<int>{256, 2048} : std::vector<int>{256, 1024, 4096, 8192};
  for (int b : batches)
    for (int context : contexts) {
      std::vector<int> lengths(b);
      for (int i = 0; i < b; ++i) lengths[i] = context - (i % 4) * context / 8;
      Fixture f = make_fixture(b, 32, 8, 128, lengths, 17 + b + context);
      GpuFixture gpu(f);
      const int splits = branchcraft::auto_splits(f.shape, context, cus, BC_MAX_SPLITS);
      gpu.run(1);
      const auto baseline = gpu.output.download();
      gpu.run(splits);
      const float diff = max_abs_error(baseline, gpu.output.download());
      if (!(diff <= 3e-4f)) throw std::runtime_error("benchmark split output mismatch");
      const double single = median_latency_us([&] { return gpu.launch(1); });
      const double split = splits == 1 ? single : median_latency_us([&] { return gpu.launch(splits); });
      const double kv_mib = double(f.k.size() + f.v.size()) * sizeof(h16) / (1024. * 1024.);
      double tokens = 0;
      for (int n : lengths) tokens += n;
      out << '"' << name << '"' << ',' << arch << ',' << rt << ',' << b << ",32,8,128," << context
          << ',' << kPageSize << ',' << splits << ',' << std::fixed << std::setprecision(3)
          << single << ',' << split << ',' << single / split << ',' << std::scientific
          << std::setprecision(8) << diff << std::fixed << std::setprecision(3) << ',' << kv_mib
          << '\n';
      out.flush();
      std::cout << "B=" << b << " S=" << context << " split=" << splits << " single=" << single
                << "us chosen=" << split << "us speedup=" << single / split
                << " GB/s=" << tokens * 4096.0 / split / 1e3 << " diff=" << diff << '\n';
    }
  std::cout << "Wrote " << path << '\n';
}

// Each candidate becomes its own paged sequence (src/main.cu:375-423).
Fixture make_expanded_fixture(const TreeFixture& t) {
  const Shape ps = t.prefix.shape;
  int smax = 0, total = 0;
  oracle_expand_tree(ps.batch, t.nodes, ps.kv_heads, ps.dim, ps.max_pages, t.prefix.k.data(),
                     t.prefix.v.data(), t.prefix.pages.data(), t.prefix.lengths.data(),
                     t.draft_k.data(), t.draft_v.data(), t.parent.data(), &smax, &total,
                     nullptr, nullptr, nullptr, nullptr);
  const int seqs = ps.batch * t.nodes;
  Fixture f{{seqs, ps.query_heads, ps.kv_heads, ps.dim, std::max(1, smax), total + 7},
            {}, {}, {}, {}, {}};
  f.lengths.resize(seqs);
  f.pages.resize((size_t)seqs * f.shape.max_pages);
  f.k.resize((size_t)(total + 7) * kPageSize * ps.kv_heads * ps.dim);
  f.v.resize(f.k.size());
  oracle_expand_tree(ps.batch, t.nodes, ps.kv_heads, ps.dim, ps.max_pages, t.prefix.k.data(),
                     t.prefix.v.data(), t.prefix.pages.data(), t.prefix.lengths.data(),
                     t.draft_k.data(), t.draft_v.data(), t.parent.data(), &smax, &total,
                     f.lengths.data(), f.pages.data(), f.k.data(), f.v.data());
  f.q = t.draft_q;
  return f;
}

void run_tree_bench(const std::string& path, bool quick) {
  std::ofstream out(path);
  if (!out) throw std::runtime_error("cannot open output: " + path);
  out << "gpu,sm,cuda_runtime,requests,tree_nodes,prefix_tokens,query_heads,"
         "kv_heads,head_dim,page_size,tree_us,expanded_us,latency_ratio,"
         "max_abs_diff,shared_kv_mib,expanded_kv_mib,memory_saving_pct\n";
  const std::string name = device_name(), arch = device_arch();
  const int rt = runtime_version();
  const auto batches = quick ? std::vector<int>{1, 4} : std::vector<int>{1, 4, 8};
  const auto contexts = quick ? std::vector<int>{256, 1024} : std::vector<int>{256, 1024, 2048};
  for (int b : batches)
    for (int context : contexts) {
      TreeFixture t = make_tree_fixture(b, context, 7, 128, 91 + b + context);
      Fixture expanded = make_expanded_fixture(t);
      TreeGpu tree(t);
      GpuFixture flat(expanded, 1);
      tree.run();
      flat.run(1);
      const float diff = max_abs_error(tree.output.download(), flat.output.download());
      if (!(diff <= 3e-4f)) throw std::runtime_error("expanded-cache output mismatch");
      const double tree_us = median_latency_us([&] { return tree.launch(); });
      const double expanded_us = median_latency_us([&] { return flat.launch(1); });
      const double bytes_per_token = 8.0 * 128 * sizeof(h16) * 2;
      const double shared_tokens =
          double((context + kPageSize - 1) / kPageSize * kPageSize) + b * t.nodes;
      double expanded_slots = 0;
      for (int len : expanded.lengths) expanded_slots += (len + kPageSize - 1) / kPageSize * kPageSize;
      const double shared_mib = shared_tokens * bytes_per_token / (1024. * 1024.);
      const double expanded_mib = expanded_slots * bytes_per_token / (1024. * 1024.);
      out << '"' << name << '"' << ',' << arch << ',' << rt << ',' << b << ",7," << context
          << ",32,8,128,16," << std::fixed << std::setprecision(3) << tree_us << ','
          << expanded_us << ',' << expanded_us / tree_us << ',' << std::scientific
          << std::setprecision(8) << diff << std::fixed << std::setprecision(3) << ','
          << shared_mib << ',' << expanded_mib << ',' << 100. * (1. - shared_mib / expanded_mib)
          << '\n';
      out.flush();
      std::cout << "tree B=" << b << " S=" << context << " tree=" << tree_us
                << "us expanded=" << expanded_us << "us ratio=" << expanded_us / tree_us
                << "x KV saved=" << 100. * (1. - shared_mib / expanded_mib) << "%\n";
    }
  std::cout << "Wrote " << path << '\n';
}

// ---- config N: the benchmark configurations ---------------------------------------------

template <typename F>
double cpu_seconds(F&& f) {
  const auto t0 = std::chrono::steady_clock::now();
  f();
  return std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
}

double decode_bytes(const Fixture& f, int out_bytes) {
  double tokens = 0, pages = 0;
  for (int n : f.lengths) {
    tokens += n;
    pages += (n + kPageSize - 1) / kPageSize;
  }
  const Shape s = f.shape;
  return tokens * s.kv_heads * s.dim * 4.0 + (double)s.batch * s.query_heads * s.dim * (2 + out_bytes) +
         pages * 4 + s.batch * 4;
}

void report(const char* what, double us, double bytes, double cpu1, double cpun, int cores) {
  std::cout << std::fixed << std::setprecision(3) << what << ": " << us << " us/call, "
            << bytes / us / 1e3 << " GB/s (" << 100.0 * bytes / us / 1e3 / 8000.0
            << "% of 8 TB/s); CPU oracle " << cpu1 * 1e3 << " ms on 1 thread, " << cpun * 1e3
            << " ms on " << cores << " threads\n";
}

void run_config(int n) {
  const int cores = (int)std::max(1u, std::thread::hardware_concurrency());
  const int cus = cu_count();
  std::cout << "device " << device_name() << " (" << device_arch() << ", " << cus
            << " CUs); host threads " << std::thread::hardware_concurrency() << '\n';
  if (n == 1 || n == 4) {
    Fixture f;
    if (n == 1) {
      f = make_fixture(1, 32, 8, 128, {512}, 1, 1.0f, 32);  // 64-page pool
    } else {
      Rng rng(4);
      std::vector<int> lens(4);
      for (int& x : lens) x = 16384 + (int)rng.below(16385);
      f = make_fixture(4, 32, 8, 128, lens, 4, 1.0f, 16);
    }
    GpuFixture gpu(f);
    const int splits = branchcraft::auto_splits(
        f.shape, *std::max_element(f.lengths.begin(), f.lengths.end()), cus, BC_MAX_SPLITS);
    std::vector<float> ref1, refn;
    const double c1 = cpu_seconds([&] { ref1 = cpu_decode(f, 1); });
    const double cn = cpu_seconds([&] { refn = cpu_decode(f, cores); });
    gpu.run(splits);
    const float err = max_abs_error(ref1, gpu.output.download());
    const double us = median_latency_us([&] { return gpu.launch(splits); });
    std::cout << "config " << n << " splits=" << splits << " max_abs_error=" << err << '\n';
    report("paged decode", us, decode_bytes(f, 4), c1, cn, cores);
    // FP32 output: the reference driver's decode gate (src/main.cu:335).
    if (!(err <= 3e-4f)) throw std::runtime_error("config parity failed");
  } else if (n == 2 || n == 3) {
    const int batch = n == 2 ? 1 : 8, prefix = n == 2 ? 2048 : 2053;
    TreeFixture t = make_tree_fixture(batch, prefix, 7, 128, 100 + n, 1.0f, true);
    TreeGpu gpu(t);
    std::vector<float> ref1, refn;
    const double c1 = cpu_seconds([&] { ref1 = cpu_tree(t, 1); });
    const double cn = cpu_seconds([&] { refn = cpu_tree(t, cores); });
    gpu.run();
    const float err = max_abs_error(ref1, gpu.output.download());
    const double us = median_latency_us([&] { return gpu.launch(); });
    const double bytes = prefix * 4096.0 + batch * 7.0 * (8 * 128 * 4 + 32 * 128 * 6);
    std::cout << "config " << n << " max_abs_error=" << err << '\n';
    report("tree_verify", us, bytes, c1, cn, cores);
    Fixture expanded = make_expanded_fixture(t);
    GpuFixture flat(expanded);
    const int splits = branchcraft::auto_splits(expanded.shape, prefix + 7, cus, BC_MAX_SPLITS);
    const double e1 = median_latency_us([&] { return flat.launch(1); });
    const double es = median_latency_us([&] { return flat.launch(splits); });
    std::cout << std::fixed << std::setprecision(3) << "expanded-prefix decode: " << e1
              << " us (splits 1), " << es << " us (splits " << splits << "); expanded/tree = "
              << std::min(e1, es) / us << "x\n";
    // The reference driver's tree gate (src/main.cu:259).
    if (!(err <= 3e-4f)) throw std::runtime_error("config parity failed");
  } else if (n == 5) {
    // [20000, 2, 16, 8, 128] cache, batch 64, contexts U[128, 4096]
    const int B = 64, NB = 20000, maxp = 256, hq = 32, hkv = 8, d = 128;
    Rng rng(5);
    std::vector<int> lens(B), pages((size_t)B * maxp, -1), perm(NB);
    for (int& x : lens) x = 128 + (int)rng.below(3969);
    std::iota(perm.begin(), perm.end(), 0);
    rng.shuffle(perm);
    int cur = 0;
    for (int b = 0; b < B; ++b)
      for (int p = 0; p < (lens[b] + 15) / 16; ++p) pages[(size_t)b * maxp + p] = perm[cur++];
    std::vector<h16> cache((size_t)NB * 2 * 16 * hkv * d), q((size_t)B * hq * d);
    rng.fill(cache, 1.0f);
    rng.fill(q, 1.0f);
    DeviceBuffer<half> dcache(cache.size()), dq(q.size()), dout(q.size());
    DeviceBuffer<int> dpages(pages.size()), dlens(lens.size());
    dcache.upload(cache);
    dq.upload(q);
    dpages.upload(pages);
    dlens.upload(lens);
    const Shape s{B, hq, hkv, d, maxp, NB};
    DeviceBuffer<char> ws(branchcraft::packed_decode_workspace_size(s));
    const long long bs = 2 * 16 * hkv * d, hs = d, ss = hkv * d, kvs = 16 * hkv * d;
    const float scale = 1.0f / std::sqrt((float)d);
    auto launch = [&] {
      return branchcraft::packed_decode(s, dq.ptr, dcache.ptr, dpages.ptr, dlens.ptr, dout.ptr, bs,
                                        hs, ss, kvs, scale, ws.ptr, ws.count);
    };
    std::vector<float> ref1((size_t)B * hq * d), refn(ref1.size());
    const double c1 = cpu_seconds([&] {
      oracle_packed_decode(B, hq, hkv, d, maxp, q.data(), cache.data(), pages.data(), lens.data(),
                           bs, hs, ss, kvs, scale, ref1.data(), nullptr, 1);
    });
    const double cn = cpu_seconds([&] {
      oracle_packed_decode(B, hq, hkv, d, maxp, q.data(), cache.data(), pages.data(), lens.data(),
                           bs, hs, ss, kvs, scale, refn.data(), nullptr, cores);
    });
    CHECK(launch());
    CHECK(hipDeviceSynchronize());
    const auto out16 = dout.download<h16>();
    // FP16 output: the north star's 2e-3 plus half an FP16 ulp of the
    // expected value (the output's own rounding).
    float err = 0, excess = -1.f;
    for (size_t i = 0; i < out16.size(); ++i) {
      const float diff = std::fabs(oracle_h2f(out16[i]) - ref1[i]);
      const uint16_t h = oracle_f2h(std::fabs(ref1[i]));
      const float ulp = oracle_h2f((uint16_t)(h + 1)) - oracle_h2f(h);
      err = std::max(err, diff);
      excess = std::max(excess, diff - (2e-3f + 0.5f * ulp));
    }
    const double us = median_latency_us(launch);
    Fixture geom{s, {}, {}, {}, {}, lens};
    std::cout << "config 5 max_abs_error(fp16 out vs fp32 oracle)=" << err << '\n';
    report("packed decode", us, decode_bytes(geom, 2), c1, cn, cores);
    if (!(excess <= 0.f)) throw std::runtime_error("config parity failed");
  } else {
    throw std::runtime_error("config must be 1..5");
  }
}

int main(int argc, char** argv) {
  try {
    if (argc < 2) {
      std::cerr << "Usage: branchcraft test | bench | tree-bench [--quick] [--output FILE]"
                   " | config N\n";
      return 2;
    }
    const std::string mode = argv[1];
    if (mode == "test") {
      run_tests();
      run_tree_tests();
    } else if (mode == "config") {
      if (argc < 3) throw std::runtime_error("config needs N (1..5)");
      run_config(std::stoi(argv[2]));
    } else if (mode == "bench" || mode == "tree-bench") {
      bool quick = false;
      std::string output = mode == "bench" ? "decode_results.csv" : "tree_results.csv";
      for (int i = 2; i < argc; ++i) {
        const std::string arg = argv[i];
        if (arg == "--quick") quick = true;
        else if (arg == "--output" && i + 1 < argc) output = argv[++i];
        else throw std::runtime_error("unknown or incomplete argument: " + arg);
      }
      if (mode == "bench") run_bench(output, quick);
      else run_tree_bench(output, quick);
    } else {
      throw std::runtime_error("unknown mode: " + mode);
    }
    return 0;
  } catch (const std::exception& e) {
    std::cerr << "ERROR: " << e.what() << '\n';
    return 1;
  }
}
