// PyTorch dispatcher binding of the Branchcraft gfx950 kernels.
//
// Mirrors bindings/torch_ops.cpp of the reference (schemas at :144-148,
// impls under the CUDA dispatch key at :150-154; on PyTorch-ROCm the CUDA
// key is the HIP device key).  Each impl validates its tensors with
// TORCH_CHECK (RuntimeError on failure, same rules as the reference), then
// calls the C ABI in include/branchcraft.h on the current HIP stream of the
// tensors' device, which it makes current for the call.
// Workspaces for split launches come from PyTorch's caching allocator, which
// keeps the ops safe under HIP graph capture.
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <atomic>

#include "branchcraft.h"

namespace {

void check_dev_contig(const at::Tensor& t, const char* name, at::ScalarType dtype) {
  TORCH_CHECK(t.is_cuda(), name, " must be a GPU tensor");
  TORCH_CHECK(t.is_contiguous(), name, " must be contiguous");
  TORCH_CHECK(t.scalar_type() == dtype, name, " has wrong dtype");
}

void check_launch(int err, const char* op) {
  TORCH_CHECK(err == 0, op, ": ",
              err == BC_ERROR_INVALID_VALUE ? "invalid argument"
                                            : hipGetErrorString((hipError_t)err));
}

bc_stream_t current_stream() {
  return reinterpret_cast<bc_stream_t>(c10::hip::getCurrentHIPStream().stream());
}

const bc_half* hptr(const at::Tensor& t) {
  return reinterpret_cast<const bc_half*>(t.data_ptr<at::Half>());
}

bc_half* hptr_mut(at::Tensor& t) {
  return reinterpret_cast<bc_half*>(t.data_ptr<at::Half>());
}

// Reference: tree_verify_cuda, bindings/torch_ops.cpp:22-67.
at::Tensor tree_verify_hip(const at::Tensor& q, const at::Tensor& prefix_k,
                           const at::Tensor& prefix_v, const at::Tensor& pages,
                           const at::Tensor& lengths, const at::Tensor& draft_k,
                           const at::Tensor& draft_v, const at::Tensor& parent) {
  check_dev_contig(q, "q", at::kHalf);
  check_dev_contig(prefix_k, "prefix_k", at::kHalf);
  check_dev_contig(prefix_v, "prefix_v", at::kHalf);
  check_dev_contig(draft_k, "draft_k", at::kHalf);
  check_dev_contig(draft_v, "draft_v", at::kHalf);
  check_dev_contig(pages, "pages", at::kInt);
  check_dev_contig(lengths, "lengths", at::kInt);
  check_dev_contig(parent, "parent", at::kInt);
  TORCH_CHECK(q.dim() == 4 && prefix_k.dim() == 4 && prefix_v.dim() == 4 &&
                  draft_k.dim() == 4 && draft_v.dim() == 4 && pages.dim() == 2 &&
                  lengths.dim() == 1 && parent.dim() == 2,
              "invalid tree tensor rank");
  const int64_t b = q.size(0), nodes = q.size(1), hq = q.size(2), d = q.size(3);
  const int64_t hkv = prefix_k.size(2);
  TORCH_CHECK(b > 0 && nodes > 0 && nodes <= BC_MAX_TREE_NODES && hq > 0 &&
                  hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128),
              "unsupported tree shape");
  TORCH_CHECK(prefix_k.size(1) == BC_PAGE_SIZE && prefix_k.size(3) == d &&
                  prefix_v.sizes() == prefix_k.sizes(),
              "prefix K/V shape mismatch");
  TORCH_CHECK(draft_k.sizes() == at::IntArrayRef({b, nodes, hkv, d}) &&
                  draft_v.sizes() == draft_k.sizes(),
              "draft K/V shape mismatch");
  TORCH_CHECK(pages.size(0) == b && lengths.size(0) == b &&
                  parent.sizes() == at::IntArrayRef({b, nodes}),
              "tree metadata shape mismatch");
  TORCH_CHECK(q.device() == prefix_k.device() && q.device() == prefix_v.device() &&
                  q.device() == draft_k.device() && q.device() == draft_v.device() &&
                  q.device() == pages.device() && q.device() == lengths.device() &&
                  q.device() == parent.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(q.device());
  auto output = at::empty(q.sizes(), q.options().dtype(at::kFloat));
  TORCH_CHECK(pages.size(1) >= 1, "pages must have at least one column");
  bc_shape shape{int(b), int(hq), int(hkv), int(d), int(pages.size(1)),
                 int(prefix_k.size(0))};
  bc_inputs prefix{nullptr, hptr(prefix_k), hptr(prefix_v), pages.data_ptr<int>(),
                   lengths.data_ptr<int>(), nullptr};
  bc_tree_inputs in{prefix, hptr(q), hptr(draft_k), hptr(draft_v),
                    parent.data_ptr<int>(), output.data_ptr<float>()};
  const size_t ws_bytes = bc_tree_verify_workspace_size(shape, int(nodes));
  at::Tensor ws;
  if (ws_bytes > 0)
    ws = at::empty({int64_t(ws_bytes)}, q.options().dtype(at::kByte));
  void* const wsp = ws_bytes ? ws.data_ptr() : nullptr;
  check_launch(bc_tree_verify_ws(shape, in, int(nodes), wsp, ws_bytes, current_stream()),
               "tree_verify");
  return output;
}

// Compute units of a device, cached (an immutable attribute).
int device_cus(int device) {
  static std::atomic<int> cache[64];
  if (device >= 0 && device < 64) {
    const int v = cache[device].load(std::memory_order_relaxed);
    if (v > 0) return v;
  }
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess ||
      n < 1)
    n = 256;
  if (device >= 0 && device < 64) cache[device].store(n, std::memory_order_relaxed);
  return n;
}

// Paged GQA decode with FP32 output.  The reference exposes it only as the
// C++ branchcraft::decode / auto_splits (include/branchcraft.hpp:39-41,
// src/paged_gqa.cu:122-142); this op takes the same tensors as Inputs
// (q [B,Hq,D], k/v [P,16,Hkv,D] FP16, pages [B,max_pages] and lengths [B]
// int32).  splits == 0 picks the split count from the shape alone:
// bc_auto_splits with the page table's capacity (max_pages * 16 tokens) as
// the context bound, so the op never reads lengths back to the host and
// can be captured in a HIP graph.  The split scratch comes from the caching
// allocator on the current stream.
at::Tensor paged_decode_hip(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                            const at::Tensor& pages, const at::Tensor& lengths,
                            int64_t splits) {
  check_dev_contig(q, "q", at::kHalf);
  check_dev_contig(k, "k", at::kHalf);
  check_dev_contig(v, "v", at::kHalf);
  check_dev_contig(pages, "pages", at::kInt);
  check_dev_contig(lengths, "lengths", at::kInt);
  TORCH_CHECK(q.dim() == 3 && k.dim() == 4 && pages.dim() == 2 && lengths.dim() == 1,
              "invalid paged decode tensor rank");
  const int64_t b = q.size(0), hq = q.size(1), d = q.size(2), hkv = k.size(2);
  TORCH_CHECK(b > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128),
              "unsupported paged decode shape");
  TORCH_CHECK(k.size(0) > 0 && k.size(1) == BC_PAGE_SIZE && k.size(3) == d &&
                  v.sizes() == k.sizes(),
              "K/V cache shape mismatch");
  TORCH_CHECK(pages.size(0) == b && pages.size(1) >= 1 && lengths.size(0) == b,
              "paged decode metadata mismatch");
  TORCH_CHECK(splits >= 0 && splits <= BC_MAX_SPLITS, "splits must be in [0, ",
              BC_MAX_SPLITS, "]");
  TORCH_CHECK(q.device() == k.device() && q.device() == v.device() &&
                  q.device() == pages.device() && q.device() == lengths.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(q.device());
  bc_shape shape{int(b), int(hq), int(hkv), int(d), int(pages.size(1)), int(k.size(0))};
  if (splits == 0) {
    const int64_t cap = std::min<int64_t>(pages.size(1) * BC_PAGE_SIZE, 1 << 30);
    splits = bc_auto_splits(shape, int(cap), device_cus(q.device().index()));
  }
  auto output = at::empty(q.sizes(), q.options().dtype(at::kFloat));
  at::Tensor scratch;
  bc_scratch scr{nullptr, nullptr};
  if (splits > 1) {
    const int64_t rows = splits * b * hq;
    scratch = at::empty({rows * (d + 2)}, q.options().dtype(at::kFloat));
    scr.partial_a = scratch.data_ptr<float>();
    scr.partial_ml = scr.partial_a + rows * d;
  }
  bc_inputs in{hptr(q), hptr(k), hptr(v), pages.data_ptr<int>(), lengths.data_ptr<int>(),
               output.data_ptr<float>()};
  check_launch(bc_decode(shape, in, scr, int(splits), current_stream()), "paged_decode");
  return output;
}

// Reference: packed_decode_out_cuda, bindings/torch_ops.cpp:69-104.
// packed_kv is either the reference's logical [P, Hkv, 16, 2D] view (V at
// +D, any outer strides) or [P, 2, 16, Hkv, D] (V at stride(1)); the head
// dimension must be contiguous.
at::Tensor packed_decode_out_hip(const at::Tensor& q, const at::Tensor& packed_kv,
                                 const at::Tensor& pages, const at::Tensor& lengths,
                                 at::Tensor& output, double scale) {
  check_dev_contig(q, "q", at::kHalf);
  check_dev_contig(pages, "pages", at::kInt);
  check_dev_contig(lengths, "lengths", at::kInt);
  check_dev_contig(output, "output", at::kHalf);
  TORCH_CHECK(q.dim() == 3 && pages.dim() == 2 && lengths.dim() == 1,
              "invalid packed decode tensor rank");
  const int64_t b = q.size(0), hq = q.size(1), d = q.size(2);
  TORCH_CHECK(packed_kv.is_cuda() && packed_kv.scalar_type() == at::kHalf &&
                  (packed_kv.dim() == 4 || packed_kv.dim() == 5) &&
                  packed_kv.stride(-1) == 1,
              "packed_kv must be a GPU FP16 tensor with contiguous content dim");
  int64_t hkv, bs, hs, ss, kvs;
  if (packed_kv.dim() == 4) {
    hkv = packed_kv.size(1);
    TORCH_CHECK(packed_kv.size(2) == BC_PAGE_SIZE && packed_kv.size(3) == 2 * d,
                "packed KV shape mismatch");
    bs = packed_kv.stride(0);
    hs = packed_kv.stride(1);
    ss = packed_kv.stride(2);
    kvs = d;
  } else {
    hkv = packed_kv.size(3);
    TORCH_CHECK(packed_kv.size(1) == 2 && packed_kv.size(2) == BC_PAGE_SIZE &&
                    packed_kv.size(4) == d,
                "packed KV shape mismatch");
    bs = packed_kv.stride(0);
    kvs = packed_kv.stride(1);
    ss = packed_kv.stride(2);
    hs = packed_kv.stride(3);
  }
  TORCH_CHECK(b > 0 && hq > 0 && hkv > 0 && hq % hkv == 0 && (d == 64 || d == 128),
              "unsupported packed decode shape");
  TORCH_CHECK(pages.size(0) == b && lengths.size(0) == b &&
                  output.numel() == q.numel() && pages.size(1) >= 1,
              "packed decode metadata/output mismatch");
  TORCH_CHECK(q.device() == packed_kv.device() && q.device() == pages.device() &&
                  q.device() == lengths.device() && q.device() == output.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(q.device());
  bc_shape shape{int(b), int(hq), int(hkv), int(d), int(pages.size(1)),
                 int(packed_kv.size(0))};
  const size_t ws_bytes = bc_packed_decode_workspace_size(shape);
  at::Tensor ws;
  if (ws_bytes > 0)
    ws = at::empty({int64_t(ws_bytes)}, q.options().dtype(at::kByte));
  check_launch(bc_packed_decode_ws(shape, hptr(q), hptr(packed_kv),
                                   pages.data_ptr<int>(), lengths.data_ptr<int>(),
                                   hptr_mut(output), bs, hs, ss, kvs, float(scale),
                                   ws_bytes ? ws.data_ptr() : nullptr, ws_bytes,
                                   current_stream()),
               "packed_decode_out");
  return output;
}

// Reference: commit_path_cuda, bindings/torch_ops.cpp:106-140.
void commit_path_hip(at::Tensor& cache_k, at::Tensor& cache_v,
                     const at::Tensor& draft_k, const at::Tensor& draft_v,
                     const at::Tensor& path_nodes, const at::Tensor& dest_pages,
                     const at::Tensor& dest_slots, int64_t request) {
  check_dev_contig(cache_k, "cache_k", at::kHalf);
  check_dev_contig(cache_v, "cache_v", at::kHalf);
  check_dev_contig(draft_k, "draft_k", at::kHalf);
  check_dev_contig(draft_v, "draft_v", at::kHalf);
  check_dev_contig(path_nodes, "path_nodes", at::kInt);
  check_dev_contig(dest_pages, "dest_pages", at::kInt);
  check_dev_contig(dest_slots, "dest_slots", at::kInt);
  TORCH_CHECK(cache_k.dim() == 4 && cache_v.sizes() == cache_k.sizes() &&
                  draft_k.dim() == 4 && draft_v.sizes() == draft_k.sizes() &&
                  path_nodes.dim() == 1 && dest_pages.sizes() == path_nodes.sizes() &&
                  dest_slots.sizes() == path_nodes.sizes(),
              "commit tensor shape mismatch");
  const int64_t b = draft_k.size(0), nodes = draft_k.size(1), hkv = draft_k.size(2);
  const int64_t d = draft_k.size(3);
  TORCH_CHECK(request >= 0 && request < b && path_nodes.numel() > 0 &&
                  path_nodes.numel() <= nodes && cache_k.size(1) == BC_PAGE_SIZE &&
                  cache_k.size(2) == hkv && cache_k.size(3) == d,
              "invalid commit destination");
  TORCH_CHECK(cache_k.device() == draft_k.device() && cache_k.device() == cache_v.device() &&
                  cache_k.device() == draft_v.device() &&
                  cache_k.device() == path_nodes.device() &&
                  cache_k.device() == dest_pages.device() &&
                  cache_k.device() == dest_slots.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(cache_k.device());
  bc_shape shape{int(b), int(hkv), int(hkv), int(d), 1, int(cache_k.size(0))};
  check_launch(bc_commit_path(shape, hptr(draft_k), hptr(draft_v), hptr_mut(cache_k),
                              hptr_mut(cache_v), path_nodes.data_ptr<int>(),
                              dest_pages.data_ptr<int>(), dest_slots.data_ptr<int>(),
                              int(request), int(nodes), int(path_nodes.numel()),
                              current_stream()),
               "commit_path_");
}

// Accepted paths of several requests in one launch (no reference op: it
// batches the per-request commit_path_ calls of a transaction,
// python/branchcraft_torch/transaction.py:144-148).
void commit_paths_hip(at::Tensor& cache_k, at::Tensor& cache_v,
                      const at::Tensor& draft_k, const at::Tensor& draft_v,
                      const at::Tensor& requests, const at::Tensor& path_nodes,
                      const at::Tensor& dest_pages, const at::Tensor& dest_slots) {
  check_dev_contig(cache_k, "cache_k", at::kHalf);
  check_dev_contig(cache_v, "cache_v", at::kHalf);
  check_dev_contig(draft_k, "draft_k", at::kHalf);
  check_dev_contig(draft_v, "draft_v", at::kHalf);
  check_dev_contig(requests, "requests", at::kInt);
  check_dev_contig(path_nodes, "path_nodes", at::kInt);
  check_dev_contig(dest_pages, "dest_pages", at::kInt);
  check_dev_contig(dest_slots, "dest_slots", at::kInt);
  TORCH_CHECK(cache_k.dim() == 4 && cache_v.sizes() == cache_k.sizes() &&
                  draft_k.dim() == 4 && draft_v.sizes() == draft_k.sizes() &&
                  requests.dim() == 1 && path_nodes.sizes() == requests.sizes() &&
                  dest_pages.sizes() == requests.sizes() &&
                  dest_slots.sizes() == requests.sizes(),
              "commit tensor shape mismatch");
  const int64_t b = draft_k.size(0), nodes = draft_k.size(1), hkv = draft_k.size(2);
  const int64_t d = draft_k.size(3);
  TORCH_CHECK(b > 0 && nodes > 0 && cache_k.size(1) == BC_PAGE_SIZE &&
                  cache_k.size(2) == hkv && cache_k.size(3) == d,
              "invalid commit destination");
  TORCH_CHECK(cache_k.device() == draft_k.device() && cache_k.device() == cache_v.device() &&
                  cache_k.device() == draft_v.device() &&
                  cache_k.device() == requests.device() &&
                  cache_k.device() == path_nodes.device() &&
                  cache_k.device() == dest_pages.device() &&
                  cache_k.device() == dest_slots.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(cache_k.device());
  bc_shape shape{int(b), int(hkv), int(hkv), int(d), 1, int(cache_k.size(0))};
  check_launch(bc_commit_paths(shape, hptr(draft_k), hptr(draft_v), hptr_mut(cache_k),
                               hptr_mut(cache_v), requests.data_ptr<int>(),
                               path_nodes.data_ptr<int>(), dest_pages.data_ptr<int>(),
                               dest_slots.data_ptr<int>(), int(nodes),
                               int(requests.numel()), current_stream()),
               "commit_paths_");
}

// Copy-on-write page clone (no reference op: the reference transaction uses
// torch copy_, python/branchcraft_torch/transaction.py:133-134).
void copy_pages_hip(at::Tensor& cache_k, at::Tensor& cache_v,
                    const at::Tensor& src_pages, const at::Tensor& dst_pages) {
  check_dev_contig(cache_k, "cache_k", at::kHalf);
  check_dev_contig(cache_v, "cache_v", at::kHalf);
  check_dev_contig(src_pages, "src_pages", at::kInt);
  check_dev_contig(dst_pages, "dst_pages", at::kInt);
  TORCH_CHECK(cache_k.dim() == 4 && cache_v.sizes() == cache_k.sizes() &&
                  cache_k.size(1) == BC_PAGE_SIZE && src_pages.dim() == 1 &&
                  dst_pages.sizes() == src_pages.sizes(),
              "copy_pages tensor shape mismatch");
  TORCH_CHECK(cache_k.device() == cache_v.device() &&
                  cache_k.device() == src_pages.device() &&
                  cache_k.device() == dst_pages.device(),
              "all tensors must share a device");
  const c10::DeviceGuard guard(cache_k.device());
  bc_shape shape{1, int(cache_k.size(2)), int(cache_k.size(2)), int(cache_k.size(3)), 1,
                 int(cache_k.size(0))};
  check_launch(bc_copy_pages(shape, hptr_mut(cache_k), hptr_mut(cache_v),
                             src_pages.data_ptr<int>(), dst_pages.data_ptr<int>(),
                             int(src_pages.numel()), current_stream()),
               "copy_pages_");
}

}  // namespace

TORCH_LIBRARY(branchcraft, m) {
  m.def("tree_verify(Tensor q, Tensor prefix_k, Tensor prefix_v, Tensor pages, Tensor lengths, Tensor draft_k, Tensor draft_v, Tensor parent) -> Tensor");
  m.def("packed_decode_out(Tensor q, Tensor packed_kv, Tensor pages, Tensor lengths, Tensor(a!) output, float scale) -> Tensor(a!)");
  m.def("commit_path_(Tensor(a!) cache_k, Tensor(b!) cache_v, Tensor draft_k, Tensor draft_v, Tensor path_nodes, Tensor dest_pages, Tensor dest_slots, int request) -> ()");
  m.def("copy_pages_(Tensor(a!) cache_k, Tensor(b!) cache_v, Tensor src_pages, Tensor dst_pages) -> ()");
  m.def("commit_paths_(Tensor(a!) cache_k, Tensor(b!) cache_v, Tensor draft_k, Tensor draft_v, Tensor requests, Tensor path_nodes, Tensor dest_pages, Tensor dest_slots) -> ()");
  m.def("paged_decode(Tensor q, Tensor k, Tensor v, Tensor pages, Tensor lengths, int splits=0) -> Tensor");
}

TORCH_LIBRARY_IMPL(branchcraft, CUDA, m) {
  m.impl("tree_verify", tree_verify_hip);
  m.impl("packed_decode_out", packed_decode_out_hip);
  m.impl("commit_path_", commit_path_hip);
  m.impl("copy_pages_", copy_pages_hip);
  m.impl("commit_paths_", commit_paths_hip);
  m.impl("paged_decode", paged_decode_hip);
}
