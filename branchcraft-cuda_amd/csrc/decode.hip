// Paged GQA decode for gfx950: split-K over the sequence with an FP32 merge
// of partial softmax states, for both the [P,16,Hkv,D] paged cache
// (bc_decode) and the strided packed cache (bc_packed_decode).
//
// Reference kernels replaced: decode_kernel / merge_kernel
// (src/paged_gqa.cu:16-106) and packed_decode_kernel
// (src/packed_decode.cu:15-60).  The reference runs one 32-lane warp per
// query head and walks tokens serially with a shuffle reduction per token.
//
// Here a workgroup owns one (sequence, token range) and holds one wave64
// per KV head (up to eight), so the waves together stream every page of the
// range as whole 16-slot blocks.  Inside a wave, one 16-token page and the
// query heads of one KV head (the GQA group, up to 16) form MFMA tiles:
//
//   S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//       (D/32 x v_mfma_f32_16x16x32_f16; lane = (token, 8-dim slice), so K
//        feeds the A operand with one contiguous 16-byte load per k-step)
//   O^T[D x 16 heads]     += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//       (D/16 x v_mfma_f32_16x16x16_f16 for P's FP16 hi part and again for
//        its lo part, so P keeps ~22 bits; the S^T accumulator is already the
//        P^T B operand, lane for lane)
//
// V is staged row-major in LDS (one 16-byte store per lane and k-step) and
// the V^T A operand is read with ds_read_b64_tr_b16.  The per-head softmax
// statistics (running max over raw scores, sum) use two cross-row lane
// shuffles per page; scale*log2e is folded into the exp2 argument and the
// output rescale is skipped unless a running max grows.  Page ids are scalar
// loads fetched an iteration early, and each page's K/V loads are issued two
// pages ahead of their use.
#include "bc_device.h"

#include <math.h>

namespace {

using namespace bcd;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

constexpr int kMaxWaves = 8;
constexpr int kHeadCols = 16;  // MFMA N: query heads of one KV head per wave

struct AttnParams {
  const uint16_t* q;      // [B, Hq, D]
  const uint16_t* kbase;  // element (page 0, head 0, slot 0, dim 0) of K
  const uint16_t* vbase;  // same for V
  const int32_t* pages;   // [B, max_pages]
  const int32_t* lengths; // [B]
  void* out;              // [B, Hq, D], float or _Float16
  float* part_acc;        // split partials: acc
  float* part_ml;         // split partials: (max, sum), max in log2 units
  long long page_stride;  // elements between physical pages
  long long head_stride;  // elements between KV heads
  long long slot_stride;  // elements between page slots
  int batch, hq, hkv, group, nblk, max_pages, phys_pages;
  int zdim;               // head blocks per sequence = hkv * nblk
  int waves;              // waves per workgroup (head blocks per workgroup)
  float scale_log2;       // softmax scale * log2(e)
  int splits;             // > 0: `splits` equal partitions per sequence
  int chunk_tokens;       // splits == 0: fixed chunks of this many tokens
  int max_chunks;         // chunk rows reserved per (b, h) in chunk mode
};

// Row index of a partial state.  Split mode keeps the reference's scratch
// layout, row = (part*B + b)*Hq + h (src/paged_gqa.cu:141).
__device__ __forceinline__ int partial_row(const AttnParams& P, int part, int b,
                                           int h) {
  return P.splits > 0 ? (part * P.batch + b) * P.hq + h
                      : (b * P.hq + h) * P.max_chunks + part;
}

template <typename OutT>
__device__ __forceinline__ void store4(void* out, size_t idx, float a, float b,
                                       float c, float d) {
  if constexpr (sizeof(OutT) == 4) {
    *reinterpret_cast<float4*>(static_cast<float*>(out) + idx) = make_float4(a, b, c, d);
  } else {
    const f16x4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
    *reinterpret_cast<f16x4*>(static_cast<_Float16*>(out) + idx) = h;
  }
}

template <typename OutT>
__device__ __forceinline__ void store_out(void* out, size_t idx, float x) {
  static_cast<OutT*>(out)[idx] = (OutT)x;
}

// Eight consecutive FP16 values; VEC selects one 16-byte load, otherwise
// eight 2-byte loads (for strides or bases that are not 8-element aligned).
template <bool VEC>
__device__ __forceinline__ uint4 load8(const uint16_t* p) {
  if (VEC) return ldg16(p);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) w[i] = (uint32_t)p[2 * i] | ((uint32_t)p[2 * i + 1] << 16);
  return make_uint4(w[0], w[1], w[2], w[3]);
}

__device__ __forceinline__ f16x4 lds_read_tr(const _Float16* p) {
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(f16x4, r);
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int D, typename OutT, bool VEC>
__global__ __launch_bounds__(64 * kMaxWaves) void paged_attn_kernel(AttnParams P) {
  constexpr int KS = D / 32;  // QK k-steps
  constexpr int DT = D / 16;  // 16-dim output tiles
  constexpr int VP = D + 16;  // halves per staged V row
  __shared__ __attribute__((aligned(16))) _Float16 s_v[kMaxWaves * 16 * VP];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4;   // k-slice group / output row group
  const int c16 = lane & 15;  // token row of A, head column of B and C

  // blockIdx.x = (zg * batch + b) * parts + part; wave -> head block z.
  const int parts = P.splits > 0 ? P.splits : P.max_chunks;
  const int part = blockIdx.x % parts;
  const int zb = blockIdx.x / parts;
  const int b = zb % P.batch;
  const int z = (zb / P.batch) * P.waves + wave;
  if (z >= P.zdim) return;  // no workgroup barrier below
  const int kvh = z / P.nblk;
  const int h0 = kvh * P.group + (z % P.nblk) * kHeadCols;
  const int nh = min(kHeadCols, P.group - (z % P.nblk) * kHeadCols);

  const int len = max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
  int begin, end;
  bool final_out;
  if (P.splits > 0) {
    const int chunk = (len + P.splits - 1) / P.splits;
    begin = min(part * chunk, len);
    end = min(begin + chunk, len);
    final_out = P.splits == 1;
  } else {
    const int nchunks = max(1, (len + P.chunk_tokens - 1) / P.chunk_tokens);
    if (part >= nchunks) return;
    begin = part * P.chunk_tokens;
    end = min(begin + P.chunk_tokens, len);
    final_out = nchunks == 1;
  }

  // Q^T B operand: lane holds Q[head h0+c16][32s + 8*g4 .. +8].
  uint4 qB[KS];
  {
    const uint16_t* qp = P.q + ((size_t)b * P.hq + h0 + c16) * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qB[s] = c16 < nh ? load8<VEC>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
  }

  const float c = P.scale_log2;
  f32x4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;  // head c16; m is the running max of raw scores

  _Float16* vs = s_v + wave * 16 * VP;
  // Transpose-read address: lane (g4, c16) names [token 4*g4 + c16/4][4*(c16%4)].
  const _Float16* vtr = vs + (4 * g4 + (c16 >> 2)) * VP + 4 * (c16 & 3);

  if (end > begin) {
    const int pfirst = begin / BC_PAGE_SIZE;
    const int npg = (end - 1) / BC_PAGE_SIZE - pfirst + 1;
    const int32_t* prow = P.pages + (size_t)b * P.max_pages + pfirst;
    const long long lane_off =
        (long long)kvh * P.head_stride + (long long)c16 * P.slot_stride + 8 * g4;

    // Page ids are scalar loads (counted by lgkmcnt, not vmcnt), fetched one
    // iteration before the K/V loads that use them, so waiting for an id
    // never waits for the K/V prefetches in flight.
    // Issues past the range re-read the range's last page (an L2 hit), so
    // every path through the loop has the same loads in flight and the
    // compiler's vmcnt waits stay two pages deep.
    auto page_id = [&](int r) -> int { return prow[r < npg ? r : npg - 1]; };

    auto issue = [&](int phys, uint4 (&kb)[KS], uint4 (&vb)[KS], bool& valid) {
      valid = phys >= 0 && phys < P.phys_pages;
      const long long base = (valid ? (long long)phys : 0ll) * P.page_stride + lane_off;
#pragma unroll
      for (int s = 0; s < KS; ++s) kb[s] = load8<VEC>(P.kbase + base + 32 * s);
#pragma unroll
      for (int s = 0; s < KS; ++s) vb[s] = load8<VEC>(P.vbase + base + 32 * s);
    };

    auto process = [&](int r, const uint4 (&kb)[KS], uint4 (&vb)[KS], bool valid) {
      const int t0 = (pfirst + r) * BC_PAGE_SIZE;
      const bool full = valid && t0 >= begin && t0 + BC_PAGE_SIZE <= end;
      if (!full) {
        // Slots outside the range may hold any bits (NaN included); their
        // weight is zero, so their V row must be zero too.
        const int t = t0 + c16;
        if (!(valid && t >= begin && t < end)) {
#pragma unroll
          for (int s = 0; s < KS; ++s) vb[s] = make_uint4(0, 0, 0, 0);
        }
      }
      f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, kb[s]),
                                                   __builtin_bit_cast(f16x8, qB[s]),
                                                   sc, 0, 0, 0);
      // Stage V while the MFMAs drain.
#pragma unroll
      for (int s = 0; s < KS; ++s)
        *reinterpret_cast<uint4*>(vs + c16 * VP + 32 * s + 8 * g4) = vb[s];

      float sv[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int t = t0 + 4 * g4 + j;
        sv[j] = (full || (valid && t >= begin && t < end)) ? sc[j] : kNegInf;
      }
      float tmax = __builtin_fmaxf(__builtin_fmaxf(sv[0], sv[1]), __builtin_fmaxf(sv[2], sv[3]));
      tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 16));
      tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 32));
      const float mnew = __builtin_fmaxf(m, tmax);
      if (__builtin_amdgcn_ballot_w64(mnew > m)) {
        const float alpha = fast_exp2((m - safe_max(mnew)) * c);
        l *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t) acc[t] *= alpha;
        m = mnew;
      }
      const float mc = safe_max(m) * c;
      f16x4 ph, pl;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float pr = fast_exp2(__builtin_fmaf(sv[j], c, -mc));
        l += pr;
        ph[j] = (_Float16)pr;
        pl[j] = (_Float16)(pr - (float)ph[j]);
      }
      wave_lds_sync();
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const f16x4 a = lds_read_tr(vtr + 16 * t);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ph, acc[t], 0, 0, 0);
        acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pl, acc[t], 0, 0, 0);
      }
      wave_lds_sync();
    };

    uint4 ka[KS], va[KS], kb2[KS], vb2[KS], kc[KS], vc[KS];
    bool oka = false, okb = false, okc = false;
    issue(page_id(0), ka, va, oka);
    issue(page_id(1), kb2, vb2, okb);
    int nid = page_id(2);  // id of the next page to issue
    for (int r = 0; r < npg; r += 3) {
      issue(nid, kc, vc, okc);
      nid = page_id(r + 3);
      process(r, ka, va, oka);
      if (r + 1 >= npg) break;
      issue(nid, ka, va, oka);
      nid = page_id(r + 4);
      process(r + 1, kb2, vb2, okb);
      if (r + 2 >= npg) break;
      issue(nid, kb2, vb2, okb);
      nid = page_id(r + 5);
      process(r + 2, kc, vc, okc);
    }
  }

  // Each lane summed the weights of its own four token rows; add the groups.
  l += shfl_xor_f(l, 16);
  l += shfl_xor_f(l, 32);
  if (c16 >= nh) return;
  const int h = h0 + c16;
  // acc[t][j] = O^T[dim 16t + 4*g4 + j][head h]
  if (final_out) {
    const float inv = l > 0.f ? 1.f / l : 0.f;
    const size_t o = ((size_t)b * P.hq + h) * D + 4 * g4;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      store4<OutT>(P.out, o + 16 * t, acc[t][0] * inv, acc[t][1] * inv, acc[t][2] * inv,
                   acc[t][3] * inv);
  } else {
    const size_t r = partial_row(P, part, b, h);
    float* pa = P.part_acc + r * D + 4 * g4;
#pragma unroll
    for (int t = 0; t < DT; ++t)
      *reinterpret_cast<float4*>(pa + 16 * t) =
          make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
    if (g4 == 0) {
      P.part_ml[2 * r] = m == kNegInf ? kNegInf : m * c;
      P.part_ml[2 * r + 1] = l;
    }
  }
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x = __builtin_fmaxf(x, shfl_xor_f(x, off));
  return x;
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) x += shfl_xor_f(x, off);
  return x;
}

// out = sum_p 2^(m_p - M) a_p / sum_p 2^(m_p - M) l_p over a sequence's
// partials; all-empty rows give zeros (src/paged_gqa.cu:76-106).  One wave
// per (b, h) output row: lane p reads partial p's (max, sum), the weights are
// formed once, then every lane accumulates its dims over the partials with
// independent loads.
template <int D, typename OutT>
__global__ __launch_bounds__(256) void merge_kernel(AttnParams P) {
  constexpr int PER = D / 64;
  const int lane = threadIdx.x & 63;
  const int rowi = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (rowi >= P.batch * P.hq) return;
  const int b = rowi / P.hq, h = rowi % P.hq;
  int nparts;
  if (P.splits > 0) {
    nparts = P.splits;
  } else {
    const int len = max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
    nparts = (len + P.chunk_tokens - 1) / P.chunk_tokens;
    if (nparts <= 1) return;  // written directly by the attention kernel
  }
  float mm = kNegInf, lsum = 0.f, a[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) a[j] = 0.f;
  for (int p0 = 0; p0 < nparts; p0 += 64) {
    const int cnt = min(64, nparts - p0);
    float mp = kNegInf, lp = 0.f;
    if (lane < cnt) {
      const size_t r = partial_row(P, p0 + lane, b, h);
      mp = P.part_ml[2 * r];
      lp = P.part_ml[2 * r + 1];
    }
    const float bmax = wave_max(mp);
    if (bmax == kNegInf) continue;
    const float mn = __builtin_fmaxf(mm, bmax);
    const float a1 = fast_exp2(mm - mn);
    const float w = fast_exp2(mp - mn);  // 0 for empty partials
    lsum = lsum * a1 + wave_sum(w * lp);
#pragma unroll
    for (int j = 0; j < PER; ++j) a[j] *= a1;
    mm = mn;
    for (int i = 0; i < cnt; ++i) {
      const float wi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                     __builtin_bit_cast(int, w), i));
      const float* src = P.part_acc + (size_t)partial_row(P, p0 + i, b, h) * D + lane;
#pragma unroll
      for (int j = 0; j < PER; ++j) a[j] += wi * src[64 * j];
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    store_out<OutT>(P.out, (size_t)rowi * D + lane + 64 * j, a[j] * inv);
}

bool shape_ok(const bc_shape& s) {
  return s.batch >= 1 && s.query_heads >= 1 && s.kv_heads >= 1 &&
         s.query_heads % s.kv_heads == 0 && (s.dim == 64 || s.dim == 128) &&
         s.max_pages >= 1 && s.physical_pages >= 1;
}

template <int D, typename OutT, bool VEC>
void launch_attn(const AttnParams& P, dim3 grid, hipStream_t st) {
  paged_attn_kernel<D, OutT, VEC><<<grid, dim3(64 * P.waves), 0, st>>>(P);
}

template <int D, typename OutT>
hipError_t launch_dim(const AttnParams& P, int parts, bool vec, hipStream_t st) {
  const int zgroups = (P.zdim + P.waves - 1) / P.waves;
  const dim3 grid((unsigned)((size_t)parts * P.batch * zgroups));
  if (vec) launch_attn<D, OutT, true>(P, grid, st);
  else launch_attn<D, OutT, false>(P, grid, st);
  hipError_t err = hipGetLastError();
  const bool need_merge = P.splits > 0 ? P.splits > 1 : P.max_chunks > 1;
  if (err != hipSuccess || !need_merge) return err;
  const unsigned rows = (unsigned)P.batch * P.hq;
  merge_kernel<D, OutT><<<dim3((rows + 3) / 4), 256, 0, st>>>(P);
  return hipGetLastError();
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename OutT>
hipError_t launch(AttnParams& P, int dim, int parts, hipStream_t st) {
  P.group = P.hq / P.hkv;
  P.nblk = (P.group + kHeadCols - 1) / kHeadCols;
  P.zdim = P.hkv * P.nblk;
  P.waves = P.zdim < kMaxWaves ? P.zdim : kMaxWaves;
  const bool vec = aligned16(P.q) && aligned16(P.kbase) &&
                   aligned16(P.vbase) &&
                   (P.page_stride | P.head_stride | P.slot_stride) % 8 == 0;
  return dim == 64 ? launch_dim<64, OutT>(P, parts, vec, st)
                   : launch_dim<128, OutT>(P, parts, vec, st);
}

// Packed decode splits sequences into chunks of this many tokens when a
// workspace is supplied; a row shorter than one chunk runs unsplit.
#ifndef BC_PACKED_CHUNK_TOKENS
#define BC_PACKED_CHUNK_TOKENS 256
#endif
int packed_chunk_tokens(const bc_shape& s) {
  const int max_tokens = s.max_pages * BC_PAGE_SIZE;
  return max_tokens > BC_PACKED_CHUNK_TOKENS ? BC_PACKED_CHUNK_TOKENS : max_tokens;
}

size_t packed_workspace(const bc_shape& s, int* chunk_tokens, int* max_chunks) {
  const int ct = packed_chunk_tokens(s);
  const int mc = (s.max_pages * BC_PAGE_SIZE + ct - 1) / ct;
  if (chunk_tokens) *chunk_tokens = ct;
  if (max_chunks) *max_chunks = mc;
  if (mc <= 1) return 0;
  const size_t rows = (size_t)s.batch * s.query_heads * mc;
  const size_t acc = rows * s.dim * sizeof(float);
  const size_t ml = rows * 2 * sizeof(float);
  return ((acc + 255) & ~(size_t)255) + ml;
}

}  // namespace

extern "C" int bc_decode(bc_shape s, bc_inputs in, bc_scratch scratch,
                         int splits, bc_stream_t stream) {
  if (!shape_ok(s) || splits < 1 || splits > BC_MAX_SPLITS || !in.q ||
      !in.k || !in.v || !in.pages || !in.lengths || !in.output ||
      (splits > 1 && (!scratch.partial_a || !scratch.partial_ml)))
    return BC_ERROR_INVALID_VALUE;
  AttnParams P{};
  P.q = in.q;
  P.kbase = in.k;
  P.vbase = in.v;
  P.pages = in.pages;
  P.lengths = in.lengths;
  P.out = in.output;
  P.part_acc = scratch.partial_a;
  P.part_ml = scratch.partial_ml;
  P.slot_stride = (long long)s.kv_heads * s.dim;
  P.head_stride = s.dim;
  P.page_stride = (long long)BC_PAGE_SIZE * s.kv_heads * s.dim;
  P.batch = s.batch;
  P.hq = s.query_heads;
  P.hkv = s.kv_heads;
  P.max_pages = s.max_pages;
  P.phys_pages = s.physical_pages;
  P.scale_log2 = (float)(kLog2e / sqrt((double)s.dim));
  P.splits = splits;
  return launch<float>(P, s.dim, splits, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_auto_splits(bc_shape s, int max_length, int cu_count) {
  // One workgroup covers up to eight KV-head blocks of one sequence range.
  // Aim for about two workgroups per CU, keep at least 128 tokens per split
  // and leave contexts under 512 tokens unsplit.
  if (max_length < 512 || s.batch < 1 || s.kv_heads < 1 || s.query_heads < 1 ||
      s.query_heads % s.kv_heads)
    return 1;
  const int group = s.query_heads / s.kv_heads;
  const long long zdim = (long long)s.kv_heads * ((group + kHeadCols - 1) / kHeadCols);
  const long long base = (long long)s.batch * ((zdim + kMaxWaves - 1) / kMaxWaves);
  const long long wanted = (2ll * (cu_count > 0 ? cu_count : 256) + base - 1) / base;
  int splits = 1;
  while (splits < wanted && splits < BC_MAX_SPLITS) splits *= 2;
  while (splits > 1 && max_length / splits < 128) splits /= 2;
  return splits;
}

extern "C" size_t bc_packed_decode_workspace_size(bc_shape s) {
  if (!shape_ok(s)) return 0;
  return packed_workspace(s, nullptr, nullptr);
}

static int packed_common(bc_shape s, const bc_half* q, const bc_half* kv,
                         const int32_t* pages, const int32_t* lengths,
                         bc_half* output, long long bs, long long hs,
                         long long ss, long long kvs, float scale,
                         void* ws, size_t ws_bytes, bc_stream_t stream) {
  if (!shape_ok(s) || !q || !kv || !pages || !lengths || !output || bs < 1 ||
      hs < 1 || ss < 1 || kvs < 1 || !(scale > 0.f))
    return BC_ERROR_INVALID_VALUE;
  AttnParams P{};
  P.q = q;
  P.kbase = kv;
  P.vbase = kv + kvs;
  P.pages = pages;
  P.lengths = lengths;
  P.out = output;
  P.page_stride = bs;
  P.head_stride = hs;
  P.slot_stride = ss;
  P.batch = s.batch;
  P.hq = s.query_heads;
  P.hkv = s.kv_heads;
  P.max_pages = s.max_pages;
  P.phys_pages = s.physical_pages;
  P.scale_log2 = (float)((double)scale * 1.4426950408889634);
  int chunk_tokens = 0, max_chunks = 1;
  const size_t need = packed_workspace(s, &chunk_tokens, &max_chunks);
  if (ws && need > 0 && ws_bytes >= need) {
    P.splits = 0;
    P.chunk_tokens = chunk_tokens;
    P.max_chunks = max_chunks;
    size_t acc_bytes = (size_t)s.batch * s.query_heads * max_chunks * s.dim *
                       sizeof(float);
    acc_bytes = (acc_bytes + 255) & ~(size_t)255;
    P.part_acc = static_cast<float*>(ws);
    P.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + acc_bytes);
    return launch<_Float16>(P, s.dim, max_chunks,
                            reinterpret_cast<hipStream_t>(stream));
  }
  P.splits = 1;
  return launch<_Float16>(P, s.dim, 1, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_packed_decode(bc_shape s, const bc_half* q,
                                const bc_half* packed_kv, const int32_t* pages,
                                const int32_t* lengths, bc_half* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, long long kv_stride,
                                float scale, bc_stream_t stream) {
  return packed_common(s, q, packed_kv, pages, lengths, output, block_stride,
                       head_stride, slot_stride, kv_stride, scale, nullptr, 0,
                       stream);
}

extern "C" int bc_packed_decode_ws(bc_shape s, const bc_half* q,
                                   const bc_half* packed_kv,
                                   const int32_t* pages,
                                   const int32_t* lengths, bc_half* output,
                                   long long block_stride,
                                   long long head_stride,
                                   long long slot_stride, long long kv_stride,
                                   float scale, void* workspace,
                                   size_t workspace_bytes, bc_stream_t stream) {
  return packed_common(s, q, packed_kv, pages, lengths, output, block_stride,
                       head_stride, slot_stride, kv_stride, scale, workspace,
                       workspace_bytes, stream);
}
