// C++ view of the Branchcraft C ABI with the reference's names and types.
//
// Source-compatible with include/branchcraft.hpp:1-76 of
// Haaziq386/branchcraft-cuda: namespace branchcraft with kPageSize,
// kWarpsPerBlock, Shape, Inputs, Scratch, TreeInputs and the functions
// decode, auto_splits, tree_verify, commit_path and packed_decode, taking
// `half` pointers.  A reference caller switches by including this header
// instead of the CUDA one; the differences are that calls return hipError_t
// (hipSuccess / hipErrorInvalidValue) instead of cudaError_t and take a
// hipStream_t.  Every function forwards to the extern "C" entry point of the
// same meaning in branchcraft.h; the structs here are layout-identical to
// their C counterparts.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <cstddef>

#include "branchcraft.h"

namespace branchcraft {

// Reference: include/branchcraft.hpp:8-9.  kWarpsPerBlock is the reference's
// launch geometry (four 32-lane warps per block); it is kept so reference
// code that uses it compiles, and does not describe this build's launches.
constexpr int kPageSize = BC_PAGE_SIZE;
constexpr int kWarpsPerBlock = 4;
// Split counts the reference's decode accepts (src/paged_gqa.cu:126); its
// callers size Scratch for this many splits.
constexpr int kMaxReferenceSplits = 16;

// Reference: include/branchcraft.hpp:11-18, 32-37 (same fields and order).
using Shape = bc_shape;
using Scratch = bc_scratch;

// Reference: include/branchcraft.hpp:20-30.
struct Inputs {
  const half* q;
  const half* k;
  const half* v;
  const int* pages;
  const int* lengths;
  float* output;
};

// Reference: include/branchcraft.hpp:43-53.
struct TreeInputs {
  Inputs prefix;
  const half* draft_q;
  const half* draft_k;
  const half* draft_v;
  const int* parent;
  float* output;
};

static_assert(sizeof(half) == sizeof(bc_half), "half is 16-bit");
static_assert(sizeof(Inputs) == sizeof(bc_inputs) &&
                  offsetof(Inputs, q) == offsetof(bc_inputs, q) &&
                  offsetof(Inputs, k) == offsetof(bc_inputs, k) &&
                  offsetof(Inputs, v) == offsetof(bc_inputs, v) &&
                  offsetof(Inputs, pages) == offsetof(bc_inputs, pages) &&
                  offsetof(Inputs, lengths) == offsetof(bc_inputs, lengths) &&
                  offsetof(Inputs, output) == offsetof(bc_inputs, output),
              "Inputs mirrors bc_inputs");
static_assert(sizeof(TreeInputs) == sizeof(bc_tree_inputs) &&
                  offsetof(TreeInputs, draft_q) == offsetof(bc_tree_inputs, draft_q) &&
                  offsetof(TreeInputs, draft_k) == offsetof(bc_tree_inputs, draft_k) &&
                  offsetof(TreeInputs, draft_v) == offsetof(bc_tree_inputs, draft_v) &&
                  offsetof(TreeInputs, parent) == offsetof(bc_tree_inputs, parent) &&
                  offsetof(TreeInputs, output) == offsetof(bc_tree_inputs, output),
              "TreeInputs mirrors bc_tree_inputs");

namespace detail {

inline const bc_half* bits(const half* p) { return reinterpret_cast<const bc_half*>(p); }
inline bc_half* bits(half* p) { return reinterpret_cast<bc_half*>(p); }
inline bc_stream_t stream(hipStream_t s) { return reinterpret_cast<bc_stream_t>(s); }

inline bc_inputs to_c(const Inputs& in) {
  return bc_inputs{bits(in.q), bits(in.k), bits(in.v), in.pages, in.lengths, in.output};
}

inline bc_tree_inputs to_c(const TreeInputs& in) {
  return bc_tree_inputs{to_c(in.prefix), bits(in.draft_q), bits(in.draft_k),
                        bits(in.draft_v), in.parent, in.output};
}

inline hipError_t err(int e) { return static_cast<hipError_t>(e); }

}  // namespace detail

// Reference: include/branchcraft.hpp:39-40.  Splits above 16 are accepted (up
// to BC_MAX_SPLITS) when Scratch holds splits*B*Hq*D and splits*B*Hq*2 floats.
inline hipError_t decode(Shape shape, Inputs in, Scratch scratch, int splits,
                         hipStream_t stream = nullptr) {
  return detail::err(bc_decode(shape, detail::to_c(in), scratch, splits, detail::stream(stream)));
}

// Reference: include/branchcraft.hpp:41.  Returns at most `max_splits`
// (default 16, the count reference callers size Scratch for); the MI355X
// policy of bc_auto_splits may prefer more, which a caller that sizes Scratch
// for BC_MAX_SPLITS can allow by passing BC_MAX_SPLITS.
inline int auto_splits(Shape shape, int max_length, int sm_count,
                       int max_splits = kMaxReferenceSplits) {
  const int s = bc_auto_splits(shape, max_length, sm_count);
  const int cap = max_splits < 1 ? 1 : max_splits;
  return s < cap ? s : cap;
}

// Reference: include/branchcraft.hpp:55-56.
inline hipError_t tree_verify(Shape shape, TreeInputs in, int nodes,
                              hipStream_t stream = nullptr) {
  return detail::err(bc_tree_verify(shape, detail::to_c(in), nodes, detail::stream(stream)));
}

inline size_t tree_verify_workspace_size(Shape shape, int nodes) {
  return bc_tree_verify_workspace_size(shape, nodes);
}

// tree_verify with a caller-owned workspace (bc_tree_verify_ws).
inline hipError_t tree_verify(Shape shape, TreeInputs in, int nodes, void* workspace,
                              size_t workspace_bytes, hipStream_t stream = nullptr) {
  return detail::err(bc_tree_verify_ws(shape, detail::to_c(in), nodes, workspace,
                                       workspace_bytes, detail::stream(stream)));
}

// Reference: include/branchcraft.hpp:61-65.
inline hipError_t commit_path(Shape shape, const half* draft_k, const half* draft_v,
                              half* cache_k, half* cache_v, const int* path_nodes,
                              const int* dest_pages, const int* dest_slots, int request,
                              int nodes, int accepted, hipStream_t stream = nullptr) {
  using detail::bits;
  return detail::err(bc_commit_path(shape, bits(draft_k), bits(draft_v), bits(cache_k),
                                    bits(cache_v), path_nodes, dest_pages, dest_slots,
                                    request, nodes, accepted, detail::stream(stream)));
}

// Several requests' accepted nodes in one launch (bc_commit_paths).
inline hipError_t commit_paths(Shape shape, const half* draft_k, const half* draft_v,
                               half* cache_k, half* cache_v, const int* requests,
                               const int* path_nodes, const int* dest_pages,
                               const int* dest_slots, int nodes, int count,
                               hipStream_t stream = nullptr) {
  using detail::bits;
  return detail::err(bc_commit_paths(shape, bits(draft_k), bits(draft_v), bits(cache_k),
                                     bits(cache_v), requests, path_nodes, dest_pages,
                                     dest_slots, nodes, count, detail::stream(stream)));
}

// Copy-on-write page clone (bc_copy_pages).
inline hipError_t copy_pages(Shape shape, half* cache_k, half* cache_v, const int* src_pages,
                             const int* dst_pages, int count, hipStream_t stream = nullptr) {
  using detail::bits;
  return detail::err(bc_copy_pages(shape, bits(cache_k), bits(cache_v), src_pages, dst_pages,
                                   count, detail::stream(stream)));
}

// Reference: include/branchcraft.hpp:70-74 (V at +dim inside a logical
// [P, Hkv, 16, 2D] cache).
inline hipError_t packed_decode(Shape shape, const half* q, const half* packed_kv,
                                const int* pages, const int* lengths, half* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, float scale,
                                hipStream_t stream = nullptr) {
  using detail::bits;
  return detail::err(bc_packed_decode(shape, bits(q), bits(packed_kv), pages, lengths,
                                      bits(output), block_stride, head_stride, slot_stride,
                                      shape.dim, scale, detail::stream(stream)));
}

// Extended form (bc_packed_decode_ws): an explicit K->V offset and an
// optional split workspace of packed_decode_workspace_size(shape) bytes.
inline size_t packed_decode_workspace_size(Shape shape) {
  return bc_packed_decode_workspace_size(shape);
}

inline hipError_t packed_decode(Shape shape, const half* q, const half* packed_kv,
                                const int* pages, const int* lengths, half* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, long long kv_stride, float scale,
                                void* workspace, size_t workspace_bytes,
                                hipStream_t stream = nullptr) {
  using detail::bits;
  return detail::err(bc_packed_decode_ws(shape, bits(q), bits(packed_kv), pages, lengths,
                                         bits(output), block_stride, head_stride,
                                         slot_stride, kv_stride, scale, workspace,
                                         workspace_bytes, detail::stream(stream)));
}

}  // namespace branchcraft
