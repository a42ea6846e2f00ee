// Accepted-path commit and copy-on-write page clone for gfx950.
//
// Reference: commit_kernel / commit_path (src/tree_attention.cu:73-89,
// 107-122) and the page clone done with cudaMemcpy D2D (src/main.cu:276-281)
// or torch copy_ (python/branchcraft_torch/transaction.py:133-134).
// bc_commit_paths commits the accepted paths of several requests in one
// launch; bc_copy_pages clones any number of pages in one launch.
// Both are bit copies of FP16 rows, moved as 16-byte vectors when every
// tensor pointer is 16-byte aligned and as single halves otherwise (the
// reference accepts any `half*`); every index is range-checked on the device
// and an out-of-range entry is skipped rather than written out of bounds
// (page ids against physical_pages when the caller gives it).
#include "bc_device.h"

namespace {

constexpr int kThreads = 256;

// One workgroup per accepted node; K and V rows of Hkv*D halves each, moved
// as `row_vec` elements of type E (uint4: eight halves, uint16_t: one).  The
// node's request is `requests[i]` when a list is given, else `request`.
template <typename E>
__global__ __launch_bounds__(kThreads) void commit_kernel(
    const E* __restrict__ draft_k, const E* __restrict__ draft_v,
    E* __restrict__ cache_k, E* __restrict__ cache_v,
    const int32_t* __restrict__ requests, const int32_t* __restrict__ path_nodes,
    const int32_t* __restrict__ dest_pages,
    const int32_t* __restrict__ dest_slots, int request, int batch, int nodes,
    int phys_pages, int row_vec) {
  const int i = blockIdx.x;
  if (requests) request = requests[i];
  const int node = path_nodes[i];
  const int page = dest_pages[i];
  const int slot = dest_slots[i];
  if (request < 0 || request >= batch || node < 0 || node >= nodes || page < 0 ||
      page >= phys_pages || slot < 0 || slot >= BC_PAGE_SIZE)
    return;
  const size_t src = ((size_t)request * nodes + node) * row_vec;
  const size_t dst = ((size_t)page * BC_PAGE_SIZE + slot) * row_vec;
  for (int x = threadIdx.x; x < row_vec; x += kThreads) {
    cache_k[dst + x] = draft_k[src + x];
    cache_v[dst + x] = draft_v[src + x];
  }
}

// grid = (count, slices): workgroup (i, s) copies slice s of page pair i,
// in elements of type E as for commit_kernel.
template <typename E>
__global__ __launch_bounds__(kThreads) void copy_pages_kernel(
    E* __restrict__ cache_k, E* __restrict__ cache_v,
    const int32_t* __restrict__ src_pages, const int32_t* __restrict__ dst_pages,
    int phys_pages, int page_vec, int slice_vec) {
  const int i = blockIdx.x;
  const int src = src_pages[i];
  const int dst = dst_pages[i];
  if (src < 0 || src >= phys_pages || dst < 0 || dst >= phys_pages || src == dst)
    return;
  const int lo = blockIdx.y * slice_vec;
  const int hi = min(lo + slice_vec, page_vec);
  const size_t s0 = (size_t)src * page_vec, d0 = (size_t)dst * page_vec;
  for (int x = lo + threadIdx.x; x < hi; x += kThreads) {
    cache_k[d0 + x] = cache_k[s0 + x];
    cache_v[d0 + x] = cache_v[s0 + x];
  }
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

// Upper bound on page ids.  The reference checks no page id
// (src/tree_attention.cu:73-89); a physical_pages below 1 means the pool size
// is not given, and then only negative ids are skipped.
int pool_bound(const bc_shape& s) {
  return s.physical_pages >= 1 ? s.physical_pages : 0x7fffffff;
}

// Launches commit_kernel over `count` entries with 16-byte elements when all
// four tensors allow it, single halves otherwise.
hipError_t launch_commit(const bc_shape& s, const bc_half* draft_k, const bc_half* draft_v,
                         bc_half* cache_k, bc_half* cache_v, const int32_t* requests,
                         const int32_t* path_nodes, const int32_t* dest_pages,
                         const int32_t* dest_slots, int request, int nodes, int count,
                         hipStream_t st) {
  const int row = s.kv_heads * s.dim;  // halves per K (or V) row
  const int phys = pool_bound(s);
  if (aligned16(draft_k) && aligned16(draft_v) && aligned16(cache_k) && aligned16(cache_v))
    commit_kernel<uint4><<<dim3(count), kThreads, 0, st>>>(
        reinterpret_cast<const uint4*>(draft_k), reinterpret_cast<const uint4*>(draft_v),
        reinterpret_cast<uint4*>(cache_k), reinterpret_cast<uint4*>(cache_v), requests,
        path_nodes, dest_pages, dest_slots, request, s.batch, nodes, phys, row / 8);
  else
    commit_kernel<uint16_t><<<dim3(count), kThreads, 0, st>>>(
        draft_k, draft_v, cache_k, cache_v, requests, path_nodes, dest_pages, dest_slots,
        request, s.batch, nodes, phys, row);
  return hipGetLastError();
}

}  // namespace

extern "C" int bc_commit_path(bc_shape s, const bc_half* draft_k,
                              const bc_half* draft_v, bc_half* cache_k,
                              bc_half* cache_v, const int32_t* path_nodes,
                              const int32_t* dest_pages,
                              const int32_t* dest_slots, int request,
                              int nodes, int accepted, bc_stream_t stream) {
  // The reference's rules (src/tree_attention.cu:111-114), nothing more.
  if (!draft_k || !draft_v || !cache_k || !cache_v || !path_nodes ||
      !dest_pages || !dest_slots || request < 0 || request >= s.batch ||
      nodes < 1 || accepted < 1 || accepted > nodes)
    return BC_ERROR_INVALID_VALUE;
  if (s.dim != 64 && s.dim != 128) return BC_ERROR_INVALID_VALUE;
  if (s.kv_heads < 1) return BC_SUCCESS;  // rows of no heads: nothing to copy
  return launch_commit(s, draft_k, draft_v, cache_k, cache_v, nullptr, path_nodes,
                       dest_pages, dest_slots, request, nodes, accepted,
                       reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_commit_paths(bc_shape s, const bc_half* draft_k,
                               const bc_half* draft_v, bc_half* cache_k,
                               bc_half* cache_v, const int32_t* requests,
                               const int32_t* path_nodes,
                               const int32_t* dest_pages,
                               const int32_t* dest_slots, int nodes, int count,
                               bc_stream_t stream) {
  if (!draft_k || !draft_v || !cache_k || !cache_v || !requests || !path_nodes ||
      !dest_pages || !dest_slots || s.batch < 1 || nodes < 1 || count < 0 ||
      (s.dim != 64 && s.dim != 128))
    return BC_ERROR_INVALID_VALUE;
  if (count == 0 || s.kv_heads < 1) return BC_SUCCESS;
  return launch_commit(s, draft_k, draft_v, cache_k, cache_v, requests, path_nodes,
                       dest_pages, dest_slots, 0, nodes, count,
                       reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_copy_pages(bc_shape s, bc_half* cache_k, bc_half* cache_v,
                             const int32_t* src_pages,
                             const int32_t* dst_pages, int count,
                             bc_stream_t stream) {
  if (!cache_k || !cache_v || !src_pages || !dst_pages || count < 0 ||
      (s.dim != 64 && s.dim != 128))
    return BC_ERROR_INVALID_VALUE;
  if (count == 0 || s.kv_heads < 1) return BC_SUCCESS;
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const int page = BC_PAGE_SIZE * s.kv_heads * s.dim;  // halves per page of K (or V)
  const int phys = pool_bound(s);
  if (aligned16(cache_k) && aligned16(cache_v)) {
    const int page_vec = page / 8;
    const int slice_vec = 4 * kThreads;  // 16 KiB of K and of V per workgroup
    const int slices = (page_vec + slice_vec - 1) / slice_vec;
    copy_pages_kernel<uint4><<<dim3(count, slices), kThreads, 0, st>>>(
        reinterpret_cast<uint4*>(cache_k), reinterpret_cast<uint4*>(cache_v), src_pages,
        dst_pages, phys, page_vec, slice_vec);
  } else {
    const int slice = 16 * kThreads;  // 8 KiB of K and of V per workgroup
    copy_pages_kernel<uint16_t><<<dim3(count, (page + slice - 1) / slice), kThreads, 0, st>>>(
        cache_k, cache_v, src_pages, dst_pages, phys, page, slice);
  }
  return hipGetLastError();
}

extern "C" const char* bc_version(void) {
  return "branchcraft-mi355x 0.2 (gfx950)";
}
