// Device helpers shared by the Branchcraft gfx950 kernels: FP16 packing,
// packed-FP16 dot products, DPP reductions inside wave64 lane groups and a
// base-2 online-softmax state.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "branchcraft.h"

namespace bcd {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ f16x2 as_f16x2(uint32_t u) {
  return __builtin_bit_cast(f16x2, u);
}

// 8-element FP16 dot product, FP32 accumulate (v_dot2_f32_f16 x4).
__device__ __forceinline__ float dot8(const uint4 a, const uint4 b, float acc) {
  acc = __builtin_amdgcn_fdot2(as_f16x2(a.x), as_f16x2(b.x), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(a.y), as_f16x2(b.y), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(a.z), as_f16x2(b.z), acc, false);
  acc = __builtin_amdgcn_fdot2(as_f16x2(a.w), as_f16x2(b.w), acc, false);
  return acc;
}

// acc[0..7] += p * v[0..7] with v packed FP16 (folds into v_fma_mix_f32).
__device__ __forceinline__ void axpy8(float p, const uint4 v, float* acc) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const f16x2 h = as_f16x2(w[i]);
    acc[2 * i] = __builtin_fmaf(p, (float)h.x, acc[2 * i]);
    acc[2 * i + 1] = __builtin_fmaf(p, (float)h.y, acc[2 * i + 1]);
  }
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);  // v_exp_f32; exp2(-inf) == 0
}

// DPP lane moves inside 16-lane rows (all rows and banks enabled).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                         0xf, 0xf, false));
}

constexpr int kDppRowMirror = 0x140;      // lane i <- lane 15-i (in its row)
constexpr int kDppRowHalfMirror = 0x141;  // lane i <- lane 7-i (in its half)
constexpr int kDppQuadXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppQuadXor1 = 0xb1;        // quad_perm [1,0,3,2]

// Sum over each aligned group of GROUP lanes (GROUP = 8 or 16); every lane
// of the group receives the total.  Each step pairs lanes across the halves
// of the current block, so after log2(GROUP) steps all lanes hold the sum.
template <int GROUP>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(GROUP == 8 || GROUP == 16, "group of 8 or 16 lanes");
  if (GROUP == 16) x += dpp_f<kDppRowMirror>(x);
  x += dpp_f<kDppRowHalfMirror>(x);
  x += dpp_f<kDppQuadXor2>(x);
  x += dpp_f<kDppQuadXor1>(x);
  return x;
}

// group_sum over N independent values, one DPP step at a time across all of
// them, so consecutive DPP reads never depend on the instruction just before.
template <int GROUP, int N>
__device__ __forceinline__ void group_sum_n(float (&x)[N]) {
  static_assert(GROUP == 8 || GROUP == 16, "group of 8 or 16 lanes");
  if (GROUP == 16) {
#pragma unroll
    for (int i = 0; i < N; ++i) x[i] += dpp_f<kDppRowMirror>(x[i]);
  }
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp_f<kDppRowHalfMirror>(x[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp_f<kDppQuadXor2>(x[i]);
#pragma unroll
  for (int i = 0; i < N; ++i) x[i] += dpp_f<kDppQuadXor1>(x[i]);
}

template <int GROUP>
__device__ __forceinline__ float group_max(float x) {
  static_assert(GROUP == 8 || GROUP == 16, "group of 8 or 16 lanes");
  if (GROUP == 16) x = __builtin_fmaxf(x, dpp_f<kDppRowMirror>(x));
  x = __builtin_fmaxf(x, dpp_f<kDppRowHalfMirror>(x));
  x = __builtin_fmaxf(x, dpp_f<kDppQuadXor2>(x));
  x = __builtin_fmaxf(x, dpp_f<kDppQuadXor1>(x));
  return x;
}

__device__ __forceinline__ float shfl_xor_f(float x, int mask) {
  return __shfl_xor(x, mask, 64);
}

// Exponent base used when folding a running max that may still be -inf.
__device__ __forceinline__ float safe_max(float m) {
  return m == kNegInf ? 0.f : m;
}

__device__ __forceinline__ uint4 ldg16(const uint16_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

// 16-byte load marked non-temporal (streaming): for data read once per call,
// such as a decode's K/V pages, so they do not displace reused lines in L2.
__device__ __forceinline__ uint4 ldg16_stream(const uint16_t* p) {
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const u32x4 w = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(w.x, w.y, w.z, w.w);
}

}  // namespace bcd
