// A C++ host written against the reference's API (include/branchcraft.hpp of
// Haaziq386/branchcraft-cuda): `half` device buffers, brace-initialised
// Inputs/Scratch/TreeInputs, kPageSize/kWarpsPerBlock and the five calls,
// with only the runtime's error and stream types switched to HIP.
// tests/test_cpp_compat.py compiles it with -fsyntax-only; it is never run.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime_api.h>

#include <vector>

#include "branchcraft.hpp"

using branchcraft::Inputs;
using branchcraft::Scratch;
using branchcraft::Shape;
using branchcraft::TreeInputs;
using branchcraft::kPageSize;
using branchcraft::kWarpsPerBlock;

static_assert(kPageSize == 16, "page size is part of the contract");
static_assert(kWarpsPerBlock == 4, "reference launch constant");

struct Buffers {
  half* q;
  half* k;
  half* v;
  int* pages;
  int* lengths;
  float* out;
  float* partial_a;
  float* partial_ml;
  half* draft_q;
  half* draft_k;
  half* draft_v;
  int* parent;
  float* tree_out;
  int* path_nodes;
  int* dest_pages;
  int* dest_slots;
  half* packed;
  half* packed_out;
};

int run_once(const Buffers& d, int sm_count, hipStream_t stream) {
  const Shape s{2, 32, 8, 128, (4096 + kPageSize - 1) / kPageSize, 600};
  const Inputs in{d.q, d.k, d.v, d.pages, d.lengths, d.out};
  const Scratch scratch{d.partial_a, d.partial_ml};

  const int splits = branchcraft::auto_splits(s, 4096, sm_count);
  if (branchcraft::decode(s, in, scratch, splits) != hipSuccess) return 1;
  if (branchcraft::decode(s, in, {nullptr, nullptr}, 2, stream) != hipErrorInvalidValue)
    return 2;

  const TreeInputs tree{in, d.draft_q, d.draft_k, d.draft_v, d.parent, d.tree_out};
  if (branchcraft::tree_verify(s, tree, 7) != hipSuccess) return 3;
  if (branchcraft::tree_verify(s, tree, 7, stream) != hipSuccess) return 3;

  if (branchcraft::commit_path(s, d.draft_k, d.draft_v, const_cast<half*>(in.k),
                               const_cast<half*>(in.v), d.path_nodes, d.dest_pages,
                               d.dest_slots, 0, 7, 3, stream) != hipSuccess)
    return 4;

  const long long block_stride = 8LL * kPageSize * 2 * 128, head_stride = kPageSize * 2 * 128;
  const long long slot_stride = 2 * 128;
  if (branchcraft::packed_decode(s, d.q, d.packed, d.pages, d.lengths, d.packed_out,
                                 block_stride, head_stride, slot_stride, 0.08838834764f,
                                 stream) != hipSuccess)
    return 5;
  return 0;
}

int main() {
  std::vector<half> host(16);
  for (auto& h : host) h = __float2half(0.5f);
  Buffers d{};
  hipDeviceProp_t prop{};
  if (hipGetDeviceProperties(&prop, 0) != hipSuccess) return 1;
  return run_once(d, prop.multiProcessorCount, nullptr);
}
