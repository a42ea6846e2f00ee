// Paged GQA decode for gfx950: split-K over the sequence with an FP32 merge
// of partial softmax states, for both the [P,16,Hkv,D] paged cache
// (bc_decode) and the strided packed cache (bc_packed_decode).
//
// Reference kernels replaced: decode_kernel / merge_kernel
// (src/paged_gqa.cu:16-106) and packed_decode_kernel
// (src/packed_decode.cu:15-60).  The reference runs one 32-lane warp per
// query head and walks tokens serially; here one workgroup of four wave64s
// owns a (sequence, KV head, token range) and every K/V byte it loads serves
// the whole GQA head group.
//
// Lane layout inside a wave (COLS = D/8 lanes per token row, ROWS = 64/COLS):
//   lane = row*COLS + col; col owns head dims [8*col, 8*col+8);
//   row r handles page slots r, r+ROWS, ... (16/ROWS slots per page).
// Each lane issues one 16-byte load per slot for K and for V, so a page is
// read as fully-used 256-byte (D=128) or 128-byte (D=64) rows.  Q.K is a
// packed-FP16 dot (v_dot2_f32_f16) followed by a DPP sum over the COLS lanes
// of a row; P.V accumulates in FP32 (v_fma_mix_f32).  Every row keeps its own
// online-softmax state (base-2, scale*log2e folded into the score); rows,
// then waves, are merged at the end.
#include "bc_device.h"

#include <math.h>

namespace {

using namespace bcd;

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;

struct AttnParams {
  const uint16_t* q;      // [B, Hq, D]
  const uint16_t* kbase;  // element (page 0, head 0, slot 0, dim 0) of K
  const uint16_t* vbase;  // same for V
  const int32_t* pages;   // [B, max_pages]
  const int32_t* lengths; // [B]
  void* out;              // [B, Hq, D], float or _Float16
  float* part_acc;        // split partials: acc
  float* part_ml;         // split partials: (max, sum)
  long long page_stride;  // elements between physical pages
  long long head_stride;  // elements between KV heads
  long long slot_stride;  // elements between page slots
  int batch, hq, hkv, group, nblk, max_pages, phys_pages;
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

template <int D, int HB, typename OutT, bool VEC>
__global__ __launch_bounds__(kThreads) void paged_attn_kernel(AttnParams P) {
  constexpr int COLS = D / 8;
  constexpr int ROWS = 64 / COLS;
  constexpr int TPL = 16 / ROWS;
  static_assert(COLS == 8 || COLS == 16, "D must be 64 or 128");

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane % COLS;
  const int row = lane / COLS;

  // blockIdx.x = (z * batch + b) * parts + part, z = kvh * nblk + blk.
  const int parts = P.splits > 0 ? P.splits : P.max_chunks;
  const int part = blockIdx.x % parts;
  const int zb = blockIdx.x / parts;
  const int b = zb % P.batch;
  const int z = zb / P.batch;
  const int kvh = z / P.nblk;
  const int blk = z % P.nblk;
  const int h0 = kvh * P.group + blk * HB;
  const int nh = min(HB, P.group - blk * HB);

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
    if (part >= nchunks) return;  // whole workgroup exits together
    begin = part * P.chunk_tokens;
    end = min(begin + P.chunk_tokens, len);
    final_out = nchunks == 1;
  }

  uint4 qv[HB];
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) {
    qv[hh] = make_uint4(0, 0, 0, 0);
    if (hh < nh)
      qv[hh] = load8<VEC>(P.q + ((size_t)b * P.hq + h0 + hh) * D + 8 * col);
  }

  float m[HB], l[HB], acc[HB][8];
#pragma unroll
  for (int hh = 0; hh < HB; ++hh) {
    m[hh] = kNegInf;
    l[hh] = 0.f;
#pragma unroll
    for (int d = 0; d < 8; ++d) acc[hh][d] = 0.f;
  }

  if (end > begin) {
    const int pfirst = begin / BC_PAGE_SIZE;
    const int plast = (end - 1) / BC_PAGE_SIZE;
    const int32_t* prow = P.pages + (size_t)b * P.max_pages;
    const long long lane_off =
        (long long)kvh * P.head_stride + (long long)row * P.slot_stride + 8 * col;
    const long long slot_step = (long long)ROWS * P.slot_stride;

    auto page_base = [&](int p, bool& valid) -> long long {
      const int phys = prow[p];
      valid = phys >= 0 && phys < P.phys_pages;
      return (valid ? (long long)phys : 0ll) * P.page_stride + lane_off;
    };

    uint4 kc[TPL], vc[TPL], kn[TPL], vn[TPL];
    int p = pfirst + wave;
    bool valid_c = false;
    if (p <= plast) {
      const long long base = page_base(p, valid_c);
#pragma unroll
      for (int i = 0; i < TPL; ++i) kc[i] = load8<VEC>(P.kbase + base + i * slot_step);
#pragma unroll
      for (int i = 0; i < TPL; ++i) vc[i] = load8<VEC>(P.vbase + base + i * slot_step);
    }

    for (; p <= plast; p += kWaves) {
      const int pn = p + kWaves;
      bool valid_n = false;
      if (pn <= plast) {
        const long long base = page_base(pn, valid_n);
#pragma unroll
        for (int i = 0; i < TPL; ++i) kn[i] = load8<VEC>(P.kbase + base + i * slot_step);
#pragma unroll
        for (int i = 0; i < TPL; ++i) vn[i] = load8<VEC>(P.vbase + base + i * slot_step);
      }

      // Scores for this lane's TPL slots and HB heads, summed over the row.
      float s[TPL][HB];
#pragma unroll
      for (int i = 0; i < TPL; ++i)
#pragma unroll
        for (int hh = 0; hh < HB; ++hh)
          s[i][hh] = group_sum<COLS>(dot8(qv[hh], kc[i], 0.f)) * P.scale_log2;

      const int t0 = p * BC_PAGE_SIZE;
      const bool full = valid_c && t0 >= begin && t0 + BC_PAGE_SIZE <= end;
      if (!full) {
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
          const int t = t0 + row + ROWS * i;
          const bool ok = valid_c && t >= begin && t < end;
#pragma unroll
          for (int hh = 0; hh < HB; ++hh) s[i][hh] = ok ? s[i][hh] : kNegInf;
          // Slots past the length may hold any bits (NaN included); their
          // weight is zero, so their V row must be zero too.
          if (!ok) vc[i] = make_uint4(0, 0, 0, 0);
        }
      }

      // Lazy rescale: the running max only moves when a score exceeds it.
      float mnew[HB];
      bool grow = false;
#pragma unroll
      for (int hh = 0; hh < HB; ++hh) {
        float mb = s[0][hh];
#pragma unroll
        for (int i = 1; i < TPL; ++i) mb = __builtin_fmaxf(mb, s[i][hh]);
        mnew[hh] = __builtin_fmaxf(m[hh], mb);
        grow |= mnew[hh] > m[hh];
      }
      if (__builtin_amdgcn_ballot_w64(grow)) {
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
          const float alpha = fast_exp2(m[hh] - safe_max(mnew[hh]));
          l[hh] *= alpha;
#pragma unroll
          for (int d = 0; d < 8; ++d) acc[hh][d] *= alpha;
          m[hh] = mnew[hh];
        }
      }

#pragma unroll
      for (int i = 0; i < TPL; ++i) {
#pragma unroll
        for (int hh = 0; hh < HB; ++hh) {
          const float pr = fast_exp2(s[i][hh] - safe_max(m[hh]));
          l[hh] += pr;
          axpy8(pr, vc[i], acc[hh]);
        }
      }

#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        kc[i] = kn[i];
        vc[i] = vn[i];
      }
      valid_c = valid_n;
    }
  }

  // Merge the ROWS row states of this wave (lanes col, col+COLS, ...).
#pragma unroll
  for (int off = COLS; off < 64; off <<= 1) {
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
      const float m2 = shfl_xor_f(m[hh], off);
      const float l2 = shfl_xor_f(l[hh], off);
      const float mm = __builtin_fmaxf(m[hh], m2);
      const float a1 = fast_exp2(m[hh] - safe_max(mm));
      const float a2 = fast_exp2(m2 - safe_max(mm));
      l[hh] = l[hh] * a1 + l2 * a2;
#pragma unroll
      for (int d = 0; d < 8; ++d)
        acc[hh][d] = acc[hh][d] * a1 + shfl_xor_f(acc[hh][d], off) * a2;
      m[hh] = mm;
    }
  }

  // Merge the waves through LDS and write the output or a partial state.
  __shared__ float s_acc[kWaves][HB][D];
  __shared__ float s_m[kWaves][HB];
  __shared__ float s_l[kWaves][HB];
  if (row == 0) {
#pragma unroll
    for (int hh = 0; hh < HB; ++hh) {
#pragma unroll
      for (int d = 0; d < 8; ++d) s_acc[wave][hh][8 * col + d] = acc[hh][d];
      if (col == 0) {
        s_m[wave][hh] = m[hh];
        s_l[wave][hh] = l[hh];
      }
    }
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < nh * D; idx += kThreads) {
    const int hh = idx / D;
    const int d = idx % D;
    float mm = s_m[0][hh];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mm = __builtin_fmaxf(mm, s_m[w][hh]);
    float lsum = 0.f, asum = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float wt = fast_exp2(s_m[w][hh] - safe_max(mm));
      lsum += wt * s_l[w][hh];
      asum += wt * s_acc[w][hh][d];
    }
    const int h = h0 + hh;
    if (final_out) {
      store_out<OutT>(P.out, ((size_t)b * P.hq + h) * D + d,
                      lsum > 0.f ? asum / lsum : 0.f);
    } else {
      const int r = partial_row(P, part, b, h);
      P.part_acc[(size_t)r * D + d] = asum;
      if (d == 0) {
        P.part_ml[2 * (size_t)r] = mm;
        P.part_ml[2 * (size_t)r + 1] = lsum;
      }
    }
  }
}

// out = sum_p 2^(m_p - M) a_p / sum_p 2^(m_p - M) l_p over a sequence's
// partials; all-empty rows give zeros (src/paged_gqa.cu:76-106).
template <int D, typename OutT>
__global__ __launch_bounds__(256) void merge_kernel(AttnParams P) {
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)P.batch * P.hq * D) return;
  const int d = idx % D;
  const int h = (idx / D) % P.hq;
  const int b = idx / ((size_t)D * P.hq);
  int nparts;
  if (P.splits > 0) {
    nparts = P.splits;
  } else {
    const int len = max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
    nparts = (len + P.chunk_tokens - 1) / P.chunk_tokens;
    if (nparts <= 1) return;  // written directly by the attention kernel
  }
  float mm = kNegInf;
  for (int p = 0; p < nparts; ++p)
    mm = __builtin_fmaxf(mm, P.part_ml[2 * (size_t)partial_row(P, p, b, h)]);
  float result = 0.f;
  if (mm != kNegInf) {
    float lsum = 0.f, asum = 0.f;
    for (int p = 0; p < nparts; ++p) {
      const size_t r = partial_row(P, p, b, h);
      const float wt = fast_exp2(P.part_ml[2 * r] - mm);
      lsum += wt * P.part_ml[2 * r + 1];
      asum += wt * P.part_acc[r * D + d];
    }
    result = asum / lsum;
  }
  store_out<OutT>(P.out, idx, result);
}

bool shape_ok(const bc_shape& s) {
  return s.batch >= 1 && s.query_heads >= 1 && s.kv_heads >= 1 &&
         s.query_heads % s.kv_heads == 0 && (s.dim == 64 || s.dim == 128) &&
         s.max_pages >= 1 && s.physical_pages >= 1;
}

// Query heads per workgroup: the GQA group rounded up to a power of two,
// at most 8 (larger groups use several head blocks per KV head).
int head_block(int group) {
  if (group <= 1) return 1;
  if (group <= 2) return 2;
  if (group <= 4) return 4;
  return 8;
}

template <int D, typename OutT, bool VEC>
void launch_attn(const AttnParams& P, int hb, dim3 grid, hipStream_t st) {
  switch (hb) {
    case 1: paged_attn_kernel<D, 1, OutT, VEC><<<grid, kThreads, 0, st>>>(P); break;
    case 2: paged_attn_kernel<D, 2, OutT, VEC><<<grid, kThreads, 0, st>>>(P); break;
    case 4: paged_attn_kernel<D, 4, OutT, VEC><<<grid, kThreads, 0, st>>>(P); break;
    default: paged_attn_kernel<D, 8, OutT, VEC><<<grid, kThreads, 0, st>>>(P); break;
  }
}

template <int D, typename OutT>
hipError_t launch_hb(const AttnParams& P, int hb, int parts, bool vec,
                     hipStream_t st) {
  const dim3 grid((unsigned)((size_t)parts * P.batch * P.hkv * P.nblk));
  if (vec) launch_attn<D, OutT, true>(P, hb, grid, st);
  else launch_attn<D, OutT, false>(P, hb, grid, st);
  hipError_t err = hipGetLastError();
  const bool need_merge = P.splits > 0 ? P.splits > 1 : P.max_chunks > 1;
  if (err != hipSuccess || !need_merge) return err;
  const size_t n = (size_t)P.batch * P.hq * D;
  merge_kernel<D, OutT><<<dim3((unsigned)((n + 255) / 256)), 256, 0, st>>>(P);
  return hipGetLastError();
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename OutT>
hipError_t launch(AttnParams& P, int dim, int parts, hipStream_t st) {
  P.group = P.hq / P.hkv;
  const int hb = head_block(P.group);
  P.nblk = (P.group + hb - 1) / hb;
  const bool vec = aligned16(P.q) && aligned16(P.kbase) &&
                   aligned16(P.vbase) &&
                   (P.page_stride | P.head_stride | P.slot_stride) % 8 == 0;
  return dim == 64 ? launch_hb<64, OutT>(P, hb, parts, vec, st)
                   : launch_hb<128, OutT>(P, hb, parts, vec, st);
}

// Packed decode splits sequences into chunks of this many tokens when a
// workspace is supplied; a row shorter than one chunk runs unsplit.
int packed_chunk_tokens(const bc_shape& s) {
  const int max_tokens = s.max_pages * BC_PAGE_SIZE;
  return max_tokens > 512 ? 512 : max_tokens;
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
  // Aim for about two 4-wave workgroups per CU, keep at least 256 tokens per
  // split and leave contexts under 512 tokens unsplit.
  if (max_length < 512 || s.batch < 1 || s.kv_heads < 1 || s.query_heads < 1)
    return 1;
  const int group = s.query_heads / s.kv_heads;
  const int hb = head_block(group);
  const long long base =
      (long long)s.batch * s.kv_heads * ((group + hb - 1) / hb);
  const long long wanted = (2ll * (cu_count > 0 ? cu_count : 256) + base - 1) / base;
  int splits = 1;
  while (splits < wanted && splits < 64) splits *= 2;
  while (splits > 1 && max_length / splits < 256) splits /= 2;
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
