// C++ view of the Branchcraft C ABI with the reference's names.
//
// Mirrors include/branchcraft.hpp:6-76 of Haaziq386/branchcraft-cuda
// (namespace branchcraft: Shape, Inputs, Scratch, TreeInputs, decode,
// auto_splits, tree_verify, commit_path, packed_decode) so C++ callers of
// the reference switch by changing the include and the error type: calls
// return hipError_t instead of cudaError_t.  Every function forwards to the
// extern "C" entry point of the same meaning in branchcraft.h.
#pragma once

#include <hip/hip_runtime_api.h>

#include "branchcraft.h"

namespace branchcraft {

constexpr int kPageSize = BC_PAGE_SIZE;

using Shape = bc_shape;
using Inputs = bc_inputs;
using Scratch = bc_scratch;
using TreeInputs = bc_tree_inputs;
using half_bits = bc_half;

inline bc_stream_t to_bc(hipStream_t s) { return reinterpret_cast<bc_stream_t>(s); }

inline hipError_t decode(Shape shape, Inputs in, Scratch scratch, int splits,
                         hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_decode(shape, in, scratch, splits, to_bc(stream)));
}

inline int auto_splits(Shape shape, int max_length, int cu_count) {
  return bc_auto_splits(shape, max_length, cu_count);
}

inline hipError_t tree_verify(Shape shape, TreeInputs in, int nodes,
                              hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_tree_verify(shape, in, nodes, to_bc(stream)));
}

inline size_t tree_verify_workspace_size(Shape shape, int nodes) {
  return bc_tree_verify_workspace_size(shape, nodes);
}

inline hipError_t tree_verify(Shape shape, TreeInputs in, int nodes, void* workspace,
                              size_t workspace_bytes, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(
      bc_tree_verify_ws(shape, in, nodes, workspace, workspace_bytes, to_bc(stream)));
}

// Requests forked from one prefix: see bc_tree_verify_shared_ws.
inline size_t tree_verify_shared_workspace_size(Shape shape, int nodes) {
  return bc_tree_verify_shared_workspace_size(shape, nodes);
}

inline hipError_t tree_verify_shared(Shape shape, TreeInputs in, int nodes, void* workspace,
                                     size_t workspace_bytes, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_tree_verify_shared_ws(shape, in, nodes, workspace,
                                                          workspace_bytes, to_bc(stream)));
}

inline hipError_t commit_path(Shape shape, const half_bits* draft_k,
                              const half_bits* draft_v, half_bits* cache_k,
                              half_bits* cache_v, const int* path_nodes,
                              const int* dest_pages, const int* dest_slots, int request,
                              int nodes, int accepted, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_commit_path(shape, draft_k, draft_v, cache_k, cache_v,
                                                path_nodes, dest_pages, dest_slots, request,
                                                nodes, accepted, to_bc(stream)));
}

// Several requests' accepted nodes in one launch (no reference counterpart).
inline hipError_t commit_paths(Shape shape, const half_bits* draft_k,
                               const half_bits* draft_v, half_bits* cache_k,
                               half_bits* cache_v, const int* requests, const int* path_nodes,
                               const int* dest_pages, const int* dest_slots, int nodes,
                               int count, hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_commit_paths(shape, draft_k, draft_v, cache_k, cache_v,
                                                 requests, path_nodes, dest_pages, dest_slots,
                                                 nodes, count, to_bc(stream)));
}

inline hipError_t copy_pages(Shape shape, half_bits* cache_k, half_bits* cache_v,
                             const int* src_pages, const int* dst_pages, int count,
                             hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(
      bc_copy_pages(shape, cache_k, cache_v, src_pages, dst_pages, count, to_bc(stream)));
}

// Reference signature (V at +dim inside a [P, Hkv, 16, 2D] logical cache).
inline hipError_t packed_decode(Shape shape, const half_bits* q, const half_bits* packed_kv,
                                const int* pages, const int* lengths, half_bits* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, float scale,
                                hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_packed_decode(shape, q, packed_kv, pages, lengths, output,
                                                  block_stride, head_stride, slot_stride,
                                                  shape.dim, scale, to_bc(stream)));
}

// Extended form: explicit K->V offset and an optional split workspace.
inline size_t packed_decode_workspace_size(Shape shape) {
  return bc_packed_decode_workspace_size(shape);
}

inline hipError_t packed_decode(Shape shape, const half_bits* q, const half_bits* packed_kv,
                                const int* pages, const int* lengths, half_bits* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, long long kv_stride, float scale,
                                void* workspace, size_t workspace_bytes,
                                hipStream_t stream = nullptr) {
  return static_cast<hipError_t>(bc_packed_decode_ws(
      shape, q, packed_kv, pages, lengths, output, block_stride, head_stride, slot_stride,
      kv_stride, scale, workspace, workspace_bytes, to_bc(stream)));
}

}  // namespace branchcraft
