// Device helpers shared by the Branchcraft gfx950 kernels: exp2, DPP and
// cross-row reductions over wave64 lanes, and 16-byte loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "branchcraft.h"

namespace bcd {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
// Online softmax: the running max is moved (and the accumulators rescaled)
// only when it would grow by more than this many log2 units.
constexpr float kRescaleSlack = 8.f;

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);  // v_exp_f32; exp2(-inf) == 0
}

// FP16 hi/lo parts of two FP32 values, packed two per register (element 0
// in the low half): hi = p truncated to FP16, lo = p - hi rounded to FP16, so
// hi + lo carries about 21 bits of p.  Three instructions per pair: one
// packed truncating conversion, then one mixed-precision FMA per half, which
// reads hi's half as an FP16 operand, forms p - hi exactly in FP32 and writes
// the FP16 result into its half of lo.
__device__ __forceinline__ void split_hi_lo(float p0, float p1, uint32_t& hi, uint32_t& lo) {
  hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(p0, p1));
  asm("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(lo) : "v"(hi), "v"(p0));
  asm("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "+v"(lo)
      : "v"(hi), "v"(p1));
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

// Whole-wave reductions, every lane receiving the result: DPP inside each
// 16-lane row (no LDS traffic), then two cross-row shuffles.
__device__ __forceinline__ float wave_sum(float x) {
  x = group_sum<16>(x);
  x += shfl_xor_f(x, 16);
  return x + shfl_xor_f(x, 32);
}

__device__ __forceinline__ float wave_max(float x) {
  x = group_max<16>(x);
  x = __builtin_fmaxf(x, shfl_xor_f(x, 16));
  return __builtin_fmaxf(x, shfl_xor_f(x, 32));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int wave_sum_i(int x) {
  x += dpp_i<kDppRowMirror>(x);
  x += dpp_i<kDppRowHalfMirror>(x);
  x += dpp_i<kDppQuadXor2>(x);
  x += dpp_i<kDppQuadXor1>(x);
  x += __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
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

// Eight consecutive FP16 values; VEC selects one 16-byte load, otherwise
// eight 2-byte loads (for tensors or strides that are not 16-byte aligned).
// STREAM marks the 16-byte load non-temporal (data read once per call).
template <bool VEC, bool STREAM = false>
__device__ __forceinline__ uint4 load8(const uint16_t* p) {
  if (VEC) return STREAM ? ldg16_stream(p) : ldg16(p);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Four consecutive floats: one 16-byte store when VEC, else four stores.
template <bool VEC>
__device__ __forceinline__ void store4f(float* p, float a, float b, float c, float d) {
  if (VEC) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  } else {
    p[0] = a;
    p[1] = b;
    p[2] = c;
    p[3] = d;
  }
}

}  // namespace bcd
