// Paged GQA decode for gfx950: split-K over the sequence with an FP32 merge
// of partial softmax states, for both the [P,16,Hkv,D] paged cache
// (bc_decode) and the strided packed cache (bc_packed_decode).
//
// Reference kernels replaced: decode_kernel / merge_kernel
// (src/paged_gqa.cu:16-106) and packed_decode_kernel
// (src/packed_decode.cu:15-60).  The reference runs one 32-lane warp per
// query head and walks tokens serially with a shuffle reduction per token.
//
// Two modes.  Split decode (flat ranges): a workgroup holds one wave64 per
// head block (up to four) and walks an equal share of all the batch's
// pages: workgroup w of W takes pages [w*T/W, (w+1)*T/W) of the
// concatenated sequences, crossing sequence boundaries as it goes, so every
// workgroup does the same work however ragged the lengths are; W is at most
// one wave of workgroups (four waves per CU).  A sequence that ends inside
// one workgroup's range is written directly; the others leave an FP32
// partial (max, sum, acc) per workgroup, and a merge kernel combines them,
// finding a sequence's ranges from the lengths or, above 64 sequences, from
// one record per range.  Unsplit decode: one workgroup per (sequence, head block)
// whose eight waves take eighths of the sequence's pages and merge their
// states through LDS.  Inside a wave, one 16-token page and the query heads
// of one KV head (the GQA group, up to 16) form MFMA tiles:
//
//   S^T[16 tok x 16 heads] = K[16 tok x D] . Q^T[D x 16 heads]
//       (D/32 x v_mfma_f32_16x16x32_f16; A operand lane = (token, 8-dim slice))
//   O^T[D x 16 heads]     += V^T[D x 16 tok] . P^T[16 tok x 16 heads]
//       (D/16 x v_mfma_f32_16x16x16_f16 for P's FP16 hi part and again for
//        its lo part, so P keeps ~21 bits; the S^T accumulator is already the
//        P^T B operand, lane for lane)
//
// Pages are fetched as whole token rows (each 16-byte load instruction covers
// complete 128-byte lines) with non-temporal loads: K/V are read once per
// call, and full-line streaming loads run at ~7 TB/s on MI355X where
// partial-line or cached loads stay near 6.  Both K and V are staged
// row-major in LDS: K is read back in the A-operand layout (ds_read_b128),
// V^T through ds_read_b64_tr_b16.  The per-head softmax
// statistics (running max over raw scores, sum) use two cross-row lane
// shuffles per page; scale*log2e is folded into the exp2 argument and the
// output rescale is skipped unless a running max grows.  Each page's K/V
// loads are issued while the previous page is being processed, and page ids
// are read ahead of their pages (two pages ahead with flat ranges).
#include "bc_device.h"
#include "bc_host.h"
#include "bc_slots.h"

#include <math.h>

namespace {

using namespace bcd;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Up to four waves per workgroup at <= 168 VGPRs (three such workgroups fit
// a CU).  Flat ranges launch one wave of workgroups, four waves per CU.
constexpr int kMaxWaves = 4;
// Waves per workgroup without a workspace: one (sequence, head block) per
// workgroup, the pages split kSlices ways and merged through LDS.
constexpr int kSlices = 8;
constexpr int kHeadCols = 16;  // MFMA N: query heads of one KV head per wave

struct AttnParams {
  const uint16_t* q;      // [B, Hq, D]
  const uint16_t* kbase;  // element (page 0, head 0, slot 0, dim 0) of K
  const uint16_t* vbase;  // same for V
  const int32_t* pages;   // [B, max_pages]
  const int32_t* lengths; // [B]
  void* out;              // [B, Hq, D], float or _Float16
  float* part_acc;        // partials [slot][Hq][D] (slot: see pair_slots)
  float* part_ml;         // partials [slot][Hq][2]: (max in log2 units, sum)
  int* range_meta;        // null, or [nwg]: 2 * (range's first sequence) + 1
                          // if the range starts inside it (2 * batch for an
                          // empty range), read by the merge kernel
  long long page_stride;  // elements between physical pages
  long long head_stride;  // elements between KV heads
  long long slot_stride;  // elements between page slots
  int batch, hq, hkv, group, nblk, max_pages, phys_pages;
  int zdim;               // head blocks per sequence = hkv * nblk
  int waves;              // waves per workgroup (head blocks per workgroup)
  float scale_log2;       // softmax scale * log2(e)
  int nwg;                // > 0: flat page ranges over nwg workgroups;
                          // 0: one workgroup per (sequence, head block), its
                          // waves splitting the pages (merged through LDS)
  int pair_slots;         // partial slot of range r cutting sequence b:
                          // 0: r + b (nwg + batch slots); 1: 2r for the
                          // range's first sequence, 2r + 1 for a later one
                          // (2 * nwg slots; packed decode above 64 sequences
                          // under four ranges each, merged per range boundary)
};

// Every kernel argument into scalar registers at the kernel's start, in one
// round of loads.  Otherwise the compiler loads each field where it is first
// used, and a field first used after a branch costs one more serial round
// trip before the kernel's first memory access.
__device__ __forceinline__ void pin_params(const AttnParams& P) {
  asm volatile("" ::"s"(P.q), "s"(P.kbase), "s"(P.vbase), "s"(P.pages), "s"(P.lengths),
               "s"(P.out), "s"(P.part_acc), "s"(P.part_ml), "s"(P.range_meta), "s"(P.page_stride),
               "s"(P.head_stride), "s"(P.slot_stride), "s"(P.batch), "s"(P.hq), "s"(P.hkv),
               "s"(P.group), "s"(P.nblk), "s"(P.max_pages), "s"(P.phys_pages), "s"(P.zdim),
               "s"(P.waves), "s"(P.scale_log2), "s"(P.nwg), "s"(P.pair_slots));
  __builtin_amdgcn_sched_barrier(0);  // nothing that uses them moves above
}

__device__ __forceinline__ int seq_len(const AttnParams& P, int b) {
  return max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
}

__device__ __forceinline__ int seq_pages(const AttnParams& P, int b) {
  return (seq_len(P, b) + BC_PAGE_SIZE - 1) / BC_PAGE_SIZE;
}

__device__ __forceinline__ int wave_incl_scan_i(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off, 64);
    if (lane >= off) x += y;
  }
  return x;
}

__device__ __forceinline__ int pages_of(int len) {
  return (len + BC_PAGE_SIZE - 1) / BC_PAGE_SIZE;
}

// Lengths of 64 consecutive sequences, lane i holding sequence base + i's
// (clamped), so that a cursor stepping into the next sequence reads its
// length from a register instead of waiting for a load queued behind the
// pages in flight.  A step past the window loads the next one.
struct LenWindow {
  int base, len;
  __device__ __forceinline__ int at(const AttnParams& P, int lane, int i) {
    if (i - base >= 64) {
      base = i;
      len = seq_len(P, min(i + lane, P.batch - 1));
    }
    return __builtin_amdgcn_readlane(len, __builtin_amdgcn_readfirstlane(i - base));
  }
};

// Flat mode: workgroup rid's share of the batch's pages, `count` pages of
// the concatenated sequences from local page `plocal` of sequence b, whose
// length is len.  Lane i keeps sequence i's length in a register, so a batch
// of up to 64 sequences costs one round of loads before the first page id.
// Larger batches load the other lengths eight chunks of 64 per round (the
// addresses clamped into the batch, so the loads need no branch): one round
// for the page total per 512 sequences, and as many for the search up to
// the chunk that holds the range's first page.
__device__ void flat_range(const AttnParams& P, int lane, int rid, int& b, int& plocal,
                           int& count, int& len, LenWindow& win) {
  constexpr int U = 8;  // chunks of 64 lengths per round of loads
  const int len0 = lane < P.batch ? seq_len(P, lane) : 0;
  int mine = pages_of(len0);  // this lane's sequences lane, lane + 64, ...
  for (int base = 64; base < P.batch; base += 64 * U) {
    int l[U];
#pragma unroll
    for (int u = 0; u < U; ++u) l[u] = seq_len(P, min(base + 64 * u + lane, P.batch - 1));
#pragma unroll
    for (int u = 0; u < U; ++u) mine += base + 64 * u + lane < P.batch ? pages_of(l[u]) : 0;
  }
  const int total = wave_sum_i(mine);
  const int per = (total + P.nwg - 1) / P.nwg;
  const int f0 = rid * per;
  count = min(total, f0 + per) - f0;
  b = 0;
  plocal = 0;
  len = 0;
  win = LenWindow{0, len0};
  if (count <= 0) return;
  // The chunk of 64 sequences whose pages reach past f0 holds the range's
  // first sequence: the first lane whose inclusive page count exceeds f0.
  int run = 0;  // pages before the chunk
  auto find = [&](int base, int l) -> bool {
    const int n = pages_of(l);
    const int inc = wave_incl_scan_i(n, lane);
    const int tot = __builtin_amdgcn_readlane(inc, 63);
    if (run + tot <= f0) {
      run += tot;
      return false;
    }
    const unsigned long long hit = __builtin_amdgcn_ballot_w64(run + inc > f0);
    const int first = __builtin_ffsll((long long)hit) - 1;
    b = base + first;
    plocal = f0 - run - __builtin_amdgcn_readlane(inc - n, first);
    len = __builtin_amdgcn_readlane(l, first);
    win = LenWindow{base, l};
    return true;
  };
  if (find(0, len0)) return;
  for (int base = 64; base < P.batch; base += 64 * U) {
    int l[U];
#pragma unroll
    for (int u = 0; u < U; ++u) l[u] = seq_len(P, min(base + 64 * u + lane, P.batch - 1));
#pragma unroll
    for (int u = 0; u < U; ++u)
      if (find(base + 64 * u, base + 64 * u + lane < P.batch ? l[u] : 0)) return;
  }
}

// The sequence with the rank-th most pages (ties by index) and its length.
// Workgroups are dispatched in index order, so giving the lowest indices the
// longest sequences balances the rounds of one-workgroup-per-sequence
// launches.  Single sequences and batches above 64 sequences keep index
// order.
__device__ int seq_by_rank(const AttnParams& P, int lane, int rank, int& len) {
  if (P.batch == 1 || P.batch > 64) {
    len = seq_len(P, rank);
    return rank;
  }
  const int l = lane < P.batch ? seq_len(P, lane) : 0;
  const int n = lane < P.batch ? pages_of(l) : -1;
  int r = 0;
  for (int k = 0; k < P.batch; ++k) {
    const int nk = __builtin_amdgcn_readlane(n, k);
    r += (nk > n || (nk == n && k < lane)) ? 1 : 0;
  }
  const unsigned long long hit = __builtin_amdgcn_ballot_w64(lane < P.batch && r == rank);
  const int b = __builtin_ffsll((long long)hit) - 1;
  len = __builtin_amdgcn_readlane(l, b);
  return b;
}

// Four consecutive outputs: one vector store when the launch checked the
// buffer's 16-byte alignment (VEC), else four element stores.
template <typename OutT, bool VEC>
__device__ __forceinline__ void store4(void* out, size_t idx, float a, float b,
                                       float c, float d) {
  OutT* p = static_cast<OutT*>(out) + idx;
  if constexpr (!VEC) {
    p[0] = (OutT)a;
    p[1] = (OutT)b;
    p[2] = (OutT)c;
    p[3] = (OutT)d;
  } else if constexpr (sizeof(OutT) == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(a, b, c, d);
  } else {
    const f16x4 h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
    *reinterpret_cast<f16x4*>(p) = h;
  }
}

template <typename OutT>
__device__ __forceinline__ void store_out(void* out, size_t idx, float x) {
  static_cast<OutT*>(out)[idx] = (OutT)x;
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

// WAVES: waves per workgroup (4 in flat mode, kSlices in sliced mode).
template <int D, typename OutT, bool VEC, int WAVES>
__global__ __launch_bounds__(64 * WAVES, WAVES == kMaxWaves ? 3 : 2) void paged_attn_kernel(
    AttnParams P) {
  pin_params(P);
  constexpr int KS = D / 32;   // QK k-steps (and 16-byte loads per page row set)
  constexpr int DT = D / 16;   // 16-dim output tiles
  constexpr int VP = D + 16;   // halves per staged V row
  constexpr int KP = D + 8;    // halves per staged K row
  constexpr int LPR = D / 8;   // lanes per token row in a page load
  constexpr int RPI = 64 / LPR;  // token rows per load instruction
  static_assert(RPI * KS == BC_PAGE_SIZE, "one page = KS loads per lane");
  // Per-wave K/V staging, one contiguous area per wave (V rows, then K
  // rows); after the page loop the sliced mode's merge puts each wave's
  // [head][D + 4] FP32 state, then its (max, sum) per head, in that wave's
  // own area.
  constexpr int XP = D + 4;
  constexpr int kWaveStage = 16 * (VP + KP) * 2;  // bytes per wave
  static_assert(16 * (XP + 2) * 4 <= kWaveStage, "a wave's merge state fits its area");
  __shared__ __attribute__((aligned(16))) char s_mem[(size_t)WAVES * kWaveStage];

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g4 = lane >> 4;   // k-slice group / output row group
  const int c16 = lane & 15;  // token row of A, head column of B and C

  // Flat mode: blockIdx.x = range * zgroups + zg, wave -> head block z.
  // Sliced mode (nwg == 0): blockIdx.x = sequence * zdim + z, every wave on
  // head block z, wave w on the w-th of WAVES shares of the sequence's pages.
  const bool sliced = P.nwg == 0;
  const int zgroups = (P.zdim + P.waves - 1) / P.waves;
  const int rid = sliced ? blockIdx.x / P.zdim : blockIdx.x / zgroups;
  const int z = sliced ? blockIdx.x % P.zdim : (blockIdx.x % zgroups) * P.waves + wave;
  if (z >= P.zdim) return;  // flat mode only: no workgroup barrier there
  const int kvh = z / P.nblk;
  const int h0 = kvh * P.group + (z % P.nblk) * kHeadCols;
  const int nh = min(kHeadCols, P.group - (z % P.nblk) * kHeadCols);
  const float c = P.scale_log2;
  const float slack_raw = kRescaleSlack / c;  // the slack in raw score units

  // This workgroup's pages: sequence pb from local page `plocal`, `count`
  // pages in all (crossing into later sequences in flat mode).
  int pb, plocal, count, plen;
  LenWindow iwin{0, 0}, cwin{0, 0};  // lengths for the issue and compute cursors
  if (sliced) {
    pb = seq_by_rank(P, lane, rid, plen);
    const int np = pages_of(plen);
    plocal = wave * np / WAVES;
    count = (wave + 1) * np / WAVES - plocal;  // may be 0 (an empty slice)
  } else {
    flat_range(P, lane, rid, pb, plocal, count, plen, iwin);
    cwin = iwin;
    if (P.range_meta && z == 0 && lane == 0)
      P.range_meta[rid] = count > 0 ? 2 * pb + (plocal > 0 ? 1 : 0) : 2 * P.batch;
    if (count <= 0) return;
  }
  int ppages = pages_of(plen);
  int seg0 = plocal;  // first local page of pb in this range
  const int pb_first = pb;  // the range's first sequence

  // Q^T B operand: lane holds Q[head h0+c16][32s + 8*g4 .. +8].
  uint4 qB[KS];
  auto load_q = [&](int b) {
    const uint16_t* qp = P.q + ((size_t)b * P.hq + h0 + c16) * D + 8 * g4;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qB[s] = c16 < nh ? load8<VEC>(qp + 32 * s) : make_uint4(0, 0, 0, 0);
  };
  load_q(pb);

  f32x4 acc[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = kNegInf, l = 0.f;  // head c16; m is the running max of raw scores

  // acc[t][j] = O^T[dim 16t + 4*g4 + j][head h0 + c16]
  auto finalize = [&](bool complete) {
    float lt = l + shfl_xor_f(l, 16);  // each lane summed its own 4 token rows
    lt += shfl_xor_f(lt, 32);
    if (c16 >= nh) return;
    const int h = h0 + c16;
    if (complete) {
      const float inv = lt > 0.f ? 1.f / lt : 0.f;
      const size_t o = ((size_t)pb * P.hq + h) * D + 4 * g4;
#pragma unroll
      for (int t = 0; t < DT; ++t)
        store4<OutT, VEC>(P.out, o + 16 * t, acc[t][0] * inv, acc[t][1] * inv,
                          acc[t][2] * inv, acc[t][3] * inv);
    } else {
      // A range cuts at most two sequences: its first (which started in an
      // earlier range) and its last (which goes on in the next one).  Plain
      // arithmetic: a select on pair_slots becomes a branch.
      const int slot = rid + pb + P.pair_slots * (rid + (pb != pb_first) - pb);
      const size_t r = (size_t)slot * P.hq + h;
      float* pa = P.part_acc + r * D + 4 * g4;
#pragma unroll
      for (int t = 0; t < DT; ++t)
        store4<float, VEC>(pa, 16 * t, acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
      if (g4 == 0) {
        P.part_ml[2 * r] = m == kNegInf ? kNegInf : m * c;
        P.part_ml[2 * r + 1] = lt;
      }
    }
  };

  _Float16* vs = reinterpret_cast<_Float16*>(s_mem + (size_t)wave * kWaveStage);
  _Float16* ks = vs + 16 * VP;
  // Transpose-read address: lane (g4, c16) names [token 4*g4 + c16/4][4*(c16%4)].
  const _Float16* vtr = vs + (4 * g4 + (c16 >> 2)) * VP + 4 * (c16 & 3);
  // Page loads read whole token rows: load s of a lane covers token
  // s*RPI + lane/LPR, dims 8*(lane%LPR) .. +8, so every instruction fetches
  // complete 128-byte lines (streaming loads then stay at full rate).
  const int lrow = lane / LPR, lcol = 8 * (lane % LPR);
  const long long lane_off =
      (long long)kvh * P.head_stride + (long long)lrow * P.slot_stride + lcol;
  const long long row_step = (long long)RPI * P.slot_stride;

  // Issue cursor: walks the same pages ahead of the compute cursor.  The
  // cursor is the same in every lane, but the compiler keeps it in vector
  // registers, so page ids are vector loads counted by vmcnt like the K/V
  // loads; the loops below order them accordingly.  Issues past the range still load
  // (every path keeps the same loads in flight), but from page 0 of the pool
  // like an out-of-pool id: all of them share that one L2-resident page,
  // whereas repeating the range's last page would fetch it from HBM again,
  // since the page loads are non-temporal (about 25 MB per call at C5).
  int ib = pb, ilocal = plocal, ipages = ppages, issued = 0;
  auto next_id = [&]() -> int {
    if (issued >= count) return -1;
    const int phys = P.pages[(size_t)ib * P.max_pages + ilocal];
    ++issued;
    if (++ilocal == ipages && issued < count) {
      do {
        ++ib;
        ipages = pages_of(iwin.at(P, lane, ib));
      } while (ipages == 0);
      ilocal = 0;
    }
    return phys;
  };

  auto issue = [&](int phys, uint4 (&kb)[KS], uint4 (&vb)[KS], bool& valid) {
    valid = phys >= 0 && phys < P.phys_pages;
    const long long base = (valid ? (long long)phys : 0ll) * P.page_stride + lane_off;
#pragma unroll
    for (int s = 0; s < KS; ++s) kb[s] = load8<VEC, true>(P.kbase + base + s * row_step);
#pragma unroll
    for (int s = 0; s < KS; ++s) vb[s] = load8<VEC, true>(P.vbase + base + s * row_step);
  };

  auto process = [&](int idx, const uint4 (&kb)[KS], uint4 (&vb)[KS], bool valid) {
    if (idx >= count) return;  // padding step: loop bodies never exit early
    const int t0 = plocal * BC_PAGE_SIZE;
    const bool full = valid && t0 + BC_PAGE_SIZE <= plen;
    if (!full) {
      // Slots past the length may hold any bits (NaN included); their weight
      // is zero, so their V row must be zero too.
#pragma unroll
      for (int s = 0; s < KS; ++s)
        if (!(valid && t0 + s * RPI + lrow < plen)) vb[s] = make_uint4(0, 0, 0, 0);
    }
    // Stage the page's K and V rows; K comes back in the A-operand layout
    // (lane = token c16, dims 32s + 8*g4), V through transpose reads.
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      *reinterpret_cast<uint4*>(ks + (s * RPI + lrow) * KP + lcol) = kb[s];
      *reinterpret_cast<uint4*>(vs + (s * RPI + lrow) * VP + lcol) = vb[s];
    }
    wave_lds_sync();
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 ka = *reinterpret_cast<const uint4*>(ks + c16 * KP + 32 * s + 8 * g4);
      sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, ka),
                                                 __builtin_bit_cast(f16x8, qB[s]),
                                                 sc, 0, 0, 0);
    }

    float sv[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sv[j] = (full || (valid && t0 + 4 * g4 + j < plen)) ? sc[j] : kNegInf;
    float tmax = __builtin_fmaxf(__builtin_fmaxf(sv[0], sv[1]), __builtin_fmaxf(sv[2], sv[3]));
    tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 16));
    tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 32));
    // The running max moves only when it would grow by more than
    // kRescaleSlack in log2 units (weights stay below 2^kRescaleSlack), so
    // most pages skip rescaling the accumulators.
    const float mnew = __builtin_fmaxf(m, tmax);
    if (__builtin_amdgcn_ballot_w64(mnew > m + slack_raw)) {
      const float alpha = fast_exp2((m - safe_max(mnew)) * c);
      l *= alpha;
#pragma unroll
      for (int t = 0; t < DT; ++t) acc[t] *= alpha;
      m = mnew;
    }
    const float mc = safe_max(m) * c;
    // P as an FP16 hi/lo pair (hi truncated, lo = p - hi rounded): P.V
    // carries ~21 bits of P.
    float pr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pr[j] = fast_exp2(__builtin_fmaf(sv[j], c, -mc));
      l += pr[j];
    }
    uint32_t wh[2], wl[2];
    split_hi_lo(pr[0], pr[1], wh[0], wl[0]);
    split_hi_lo(pr[2], pr[3], wh[1], wl[1]);
    const f16x4 ph = __builtin_bit_cast(f16x4, u32x2{wh[0], wh[1]});
    const f16x4 pl = __builtin_bit_cast(f16x4, u32x2{wl[0], wl[1]});
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const f16x4 a = lds_read_tr(vtr + 16 * t);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ph, acc[t], 0, 0, 0);
      acc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, pl, acc[t], 0, 0, 0);
    }
    wave_lds_sync();

    if (++plocal == ppages) {
      // Sequence pb ends inside this range.
      if (!sliced) finalize(seg0 == 0);
      if (idx + 1 < count) {
        do {
          ++pb;
          plen = cwin.at(P, lane, pb);
          ppages = pages_of(plen);
        } while (ppages == 0);
        plocal = 0;
        seg0 = 0;
        load_q(pb);
#pragma unroll
        for (int t = 0; t < DT; ++t) acc[t] = f32x4{0.f, 0.f, 0.f, 0.f};
        m = kNegInf;
        l = 0.f;
      }
    }
  };

  uint4 ka[KS], va[KS], kb2[KS], vb2[KS];
  bool oka = false, okb = false;
  if constexpr (WAVES == kSlices) {
    // Sliced mode (eight waves per CU or more): a page id is requested
    // after the K/V loads of the page before it, so waiting for the id also
    // waits for that page, and each wave has one page in flight while it
    // computes; the two-ahead order below measured slower here (C1 8.7 ->
    // 8.8 us, packed C5 without a workspace 92.8 -> 94.2 us).
    issue(next_id(), ka, va, oka);
    int nid = next_id();
    for (int idx = 0; idx < count; idx += 2) {
      issue(nid, kb2, vb2, okb);
      nid = next_id();
      process(idx, ka, va, oka);
      issue(nid, ka, va, oka);
      nid = next_id();
      process(idx + 1, kb2, vb2, okb);
    }
  } else {
    // Flat mode (one four-wave workgroup per CU): page ids run two pages
    // ahead of the K/V loads and are requested before the loads of the page
    // in between, so the wait for an id never waits for a page still in
    // flight (loads complete in issue order) and each wave keeps two pages
    // in flight.
    const int id0 = next_id();
    int nid = next_id();
    issue(id0, ka, va, oka);
    for (int idx = 0; idx < count; idx += 2) {
      const int nid2 = next_id();  // page idx + 2
      issue(nid, kb2, vb2, okb);   // page idx + 1
      process(idx, ka, va, oka);
      nid = next_id();             // page idx + 3
      issue(nid2, ka, va, oka);
      process(idx + 1, kb2, vb2, okb);
    }
  }
  // The range ended inside sequence pb: leave a partial.
  if (!sliced) {
    if (plocal != ppages) finalize(false);
    return;
  }

  // Sliced mode: combine the waves' states.  Each wave stores (m, l, acc) of
  // its 16 head columns; wave w then merges CPW = 16/WAVES of the columns,
  // lane = (column CPW*w + lane/LPC, dims (lane%LPC)*DL ..).  Empty sequences
  // and empty slices carry m = -inf, l = 0 and give weight 0 (all-empty:
  // zeros, src/paged_gqa.cu:63).
  // The state goes to the wave's own staging area, which no other wave
  // uses: the stores need no barrier and overlap the waves still walking
  // their pages.
  float lt = l + shfl_xor_f(l, 16);
  lt += shfl_xor_f(lt, 32);
  auto xw = [&](int w) { return reinterpret_cast<float*>(s_mem + (size_t)w * kWaveStage); };
#pragma unroll
  for (int t = 0; t < DT; ++t)
    *reinterpret_cast<float4*>(xw(wave) + c16 * XP + 16 * t + 4 * g4) =
        make_float4(acc[t][0], acc[t][1], acc[t][2], acc[t][3]);
  if (g4 == 0)
    *reinterpret_cast<float2*>(xw(wave) + 16 * XP + 2 * c16) =
        make_float2(m == kNegInf ? kNegInf : m * c, lt);
  __syncthreads();
  constexpr int CPW = 16 / WAVES;  // head columns merged per wave
  constexpr int LPC = 64 / CPW;    // lanes per column
  constexpr int DL = D / LPC;      // dims per lane
  static_assert(DL % 2 == 0, "at least float2 merge steps");
  const int col = CPW * wave + lane / LPC, d0 = (lane % LPC) * DL;
  float mx = kNegInf;
  for (int w = 0; w < WAVES; ++w) mx = __builtin_fmaxf(mx, xw(w)[16 * XP + 2 * col]);
  float o[DL], lsum = 0.f;
#pragma unroll
  for (int j = 0; j < DL; ++j) o[j] = 0.f;
  for (int w = 0; w < WAVES; ++w) {
    const float mw = xw(w)[16 * XP + 2 * col];
    const float wt = mw == kNegInf ? 0.f : fast_exp2(mw - mx);
    lsum += wt * xw(w)[16 * XP + 2 * col + 1];
    const float* src = xw(w) + col * XP + d0;
#pragma unroll
    for (int j = 0; j < DL; j += 2) {
      const float2 v2 = *reinterpret_cast<const float2*>(src + j);
      o[j] += wt * v2.x;
      o[j + 1] += wt * v2.y;
    }
  }
  if (col < nh) {
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    const size_t off = ((size_t)pb * P.hq + h0 + col) * D + d0;
#pragma unroll
    for (int j = 0; j < DL; ++j) store_out<OutT>(P.out, off + j, o[j] * inv);
  }
}

// Flat mode: out = sum_w 2^(m_w - M) a_w / sum_w 2^(m_w - M) l_w over the
// workgroups whose ranges cut sequence b (src/paged_gqa.cu:76-106); empty
// sequences give zeros.  Lane i holds partial i's weight and every lane
// accumulates its dims.  Three row forms:
//  - per (b, h) row (META false), RW waves each (1 or 4): two dependent
//    memory rounds, the lengths (page geometry), then every partial's (max,
//    sum) together with the first eight partials' accumulators.  With RW = 4
//    each wave combines a contiguous quarter of the row's partials and wave
//    0 merges the four states through LDS: rows of a few long sequences have
//    hundreds of partials, too many for one wave.
//  - per (range boundary, h) row with range records (META) and pair slots
//    (PAIR): one round, records and partials together.
//  - the same rows with slot = range + sequence (META only, bc_decode above
//    64 sequences): the records, then the partials.
template <int D, typename OutT, int RW, bool PAIR, bool META>
__global__ __launch_bounds__(256) void merge_kernel(AttnParams P) {
  pin_params(P);
  static_assert(RW == 1 || RW == 4, "one or four waves per row");
  static_assert(META || !PAIR, "pair slots come with range records");
  constexpr int PER = D / 64;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = wave % RW;  // this wave's share of the row's partials
  // Row (b, h) of the output and the ranges w0..w1 whose pages include
  // sequence b's (slot w + b each).
  int b, h, np, w0, w1;
  if constexpr (META) {
    // One row per (range boundary r, head): the sequence that range r starts
    // inside, merged at the first boundary that cuts it.  Every other
    // sequence either ends inside one range (written directly) or is empty;
    // the workgroups past the rows give the empty ones zeros.
    static_assert(RW == 1, "one wave per boundary row");
    const int nrw = ((P.nwg - 1) * P.hq + 3) / 4;
    if ((int)blockIdx.x >= nrw) {
      const int base = ((int)blockIdx.x - nrw) * 256 + wave * 64;
      const int i = base + lane;
      unsigned long long empty =
          __builtin_amdgcn_ballot_w64(i < P.batch && seq_pages(P, min(i, P.batch - 1)) == 0);
      while (empty) {
        const int e = base + __builtin_ffsll((long long)empty) - 1;
        empty &= empty - 1;
        for (int hh = 0; hh < P.hq; ++hh) {
#pragma unroll
          for (int j = 0; j < PER; ++j)
            store_out<OutT>(P.out, ((size_t)e * P.hq + hh) * D + lane + 64 * j, 0.f);
        }
      }
      return;
    }
    const int rowi = blockIdx.x * 4 + wave;
    const int r = 1 + rowi / P.hq;
    h = rowi % P.hq;
    if (r >= P.nwg) return;
    if constexpr (PAIR) {
      // Pair slots: boundary r's parts are ranges r - 1 + p.  Part p >= 1
      // starts inside the row's sequence (slot 2(r - 1 + p)); part 0 holds it
      // as its first sequence (slot 2(r - 1)) or a later one (2(r - 1) + 1).
      // No slot depends on which sequence that is, so the records, every
      // part's (max, sum), both part-0 candidates and the first KP parts'
      // accumulators go out in one memory round, before the row knows
      // whether it merges at all.
      constexpr int KP = 4;
      auto srow = [&](int slot) { return (size_t)slot * P.hq + h; };
      const int m1 = P.range_meta[r], m0 = P.range_meta[r - 1];
      const int mv = P.range_meta[min(r + 1 + lane, P.nwg - 1)];  // range r + 1 + lane
      const size_t rl = srow(2 * min(r - 1 + lane, P.nwg - 1));
      const float mpa = P.part_ml[2 * rl], lpa = P.part_ml[2 * rl + 1];
      const size_t rb = srow(2 * (r - 1) + 1);
      const float mpb = P.part_ml[2 * rb], lpb = P.part_ml[2 * rb + 1];
      float va[KP][PER], vb[PER];
#pragma unroll
      for (int k = 0; k < KP; ++k) {
        const float* src = P.part_acc + srow(2 * min(r - 1 + k, P.nwg - 1)) * D + lane;
#pragma unroll
        for (int j = 0; j < PER; ++j) va[k][j] = src[64 * j];
      }
#pragma unroll
      for (int j = 0; j < PER; ++j) vb[j] = P.part_acc[rb * D + lane + 64 * j];
      // Every load above is issued before the first use (otherwise the
      // compiler sinks the accumulator loads below the branches).
      asm volatile("" ::"v"(mv), "v"(mpa), "v"(lpa), "v"(mpb), "v"(lpb));
#pragma unroll
      for (int j = 0; j < PER; ++j) {
        asm volatile("" ::"v"(vb[j]));
#pragma unroll
        for (int k = 0; k < KP; ++k) asm volatile("" ::"v"(va[k][j]));
      }
      b = m1 >> 1;
      if (!(m1 & 1)) return;                 // r starts on a sequence's first page
      if (m0 >> 1 == b && (m0 & 1)) return;  // an earlier boundary cuts b too
      const bool later = m0 >> 1 != b;       // part 0 in slot 2(r - 1) + 1
      // The ranges after r whose first sequence is b follow r: count them.
      w1 = r;
      {
        const unsigned long long hit =
            __builtin_amdgcn_ballot_w64(r + 1 + lane < P.nwg && mv >> 1 == b);
        const int n = ~hit ? __builtin_ffsll((long long)~hit) - 1 : 64;
        w1 += n;
        for (int base = r + 65; n == 64 && base < P.nwg; base += 64) {
          const int rr = base + lane;
          const int mw = P.range_meta[min(rr, P.nwg - 1)];
          const unsigned long long more = __builtin_amdgcn_ballot_w64(rr < P.nwg && mw >> 1 == b);
          const int k = ~more ? __builtin_ffsll((long long)~more) - 1 : 64;
          w1 += k;
          if (k < 64) break;
        }
      }
      const int nparts = w1 - r + 2;
      float mm = kNegInf, lsum = 0.f, a[PER];
#pragma unroll
      for (int j = 0; j < PER; ++j) a[j] = 0.f;
      for (int c0 = 0; c0 < nparts; c0 += 64) {
        const int cnt = min(64, nparts - c0);
        float mp, lp;
        if (c0 == 0) {
          mp = lane == 0 && later ? mpb : mpa;
          lp = lane == 0 && later ? lpb : lpa;
        } else {
          const size_t rr = srow(2 * min(r - 1 + c0 + lane, P.nwg - 1));
          mp = P.part_ml[2 * rr];
          lp = P.part_ml[2 * rr + 1];
        }
        mp = lane < cnt ? mp : kNegInf;
        lp = lane < cnt ? lp : 0.f;
        const float mn = __builtin_fmaxf(mm, wave_max(mp));
        const float ms = safe_max(mn);
        const float a1 = fast_exp2(mm - ms);
        const float w = fast_exp2(mp - ms);  // 0 past the parts
        lsum = lsum * a1 + wave_sum(w * lp);
#pragma unroll
        for (int j = 0; j < PER; ++j) a[j] *= a1;
        mm = mn;
        auto wt = [&](int p) {
          return __builtin_bit_cast(
              float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), p));
        };
        int i0 = 0;
        if (c0 == 0) {
#pragma unroll
          for (int k = 0; k < KP; ++k)
            if (k < cnt) {
              const float wk = wt(k);
#pragma unroll
              for (int j = 0; j < PER; ++j) a[j] += wk * (k == 0 && later ? vb[j] : va[k][j]);
            }
          i0 = KP;
        }
        // The rest eight parts per step (slots past cnt re-read the last
        // part, with weight 0).
        for (int i = i0; i < cnt; i += 8) {
          float v[8][PER];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int p = min(i + u, cnt - 1);
            const float* src = P.part_acc + srow(2 * (r - 1 + c0 + p)) * D + lane;
#pragma unroll
            for (int j = 0; j < PER; ++j) v[u][j] = src[64 * j];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const float wu = i + u < cnt ? wt(i + u) : 0.f;
#pragma unroll
            for (int j = 0; j < PER; ++j) a[j] += wu * v[u][j];
          }
        }
      }
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
      for (int j = 0; j < PER; ++j)
        store_out<OutT>(P.out, ((size_t)b * P.hq + h) * D + lane + 64 * j, a[j] * inv);
      return;
    }
    const int m1 = P.range_meta[r], m0 = P.range_meta[r - 1];
    b = m1 >> 1;
    if (!(m1 & 1)) return;                       // r starts on a sequence's first page
    if (m0 >> 1 == b && (m0 & 1)) return;        // an earlier boundary cuts b too
    w0 = r - 1;
    // The ranges after r that start inside b follow r: count them.
    w1 = r;
    for (int base = r + 1; base < P.nwg; base += 64) {
      const int rr = base + lane;
      const int mv = P.range_meta[min(rr, P.nwg - 1)];
      const unsigned long long hit = __builtin_amdgcn_ballot_w64(rr < P.nwg && mv >> 1 == b);
      const int n = ~hit ? __builtin_ffsll((long long)~hit) - 1 : 64;
      w1 += n;
      if (n < 64) break;
    }
    np = 1;
  } else {
    const int rowi = blockIdx.x * (4 / RW) + wave / RW;
    // Every exit before the LDS merge below is uniform over a row, so with
    // RW = 4 the whole workgroup leaves together.
    if (rowi >= P.batch * P.hq) return;
    b = rowi / P.hq;
    h = rowi % P.hq;
    // Lengths of the whole batch, 64 per round: the page total (as
    // flat_range), the pages before sequence b and b's own page count.
    int total = 0, before = 0;
    np = 0;
    for (int base = 0; base < P.batch; base += 64) {
      const int i = base + lane;
      const int n = i < P.batch ? seq_pages(P, i) : 0;
      total += wave_sum_i(n);
      before += wave_sum_i(i < b ? n : 0);
      if (b >= base && b < base + 64) np = __builtin_amdgcn_readlane(n, b - base);
    }
    const int per = max(1, (total + P.nwg - 1) / P.nwg);
    w0 = before / per;
    w1 = np > 0 ? (before + np - 1) / per : w0;
  }
  if (np == 0) {
    if (sub == 0) {
#pragma unroll
      for (int j = 0; j < PER; ++j)
        store_out<OutT>(P.out, ((size_t)b * P.hq + h) * D + lane + 64 * j, 0.f);
    }
    return;
  }
  if (w0 == w1) return;  // the sequence ended inside one range: written directly
  auto slot_of = [&](int w) { return w + b; };  // range w's partial slot
  // This wave's partials: [r0, r1] (empty when r1 < r0).
  const int nparts = w1 - w0 + 1;
  const int r0 = w0 + sub * nparts / RW, r1 = w0 + (sub + 1) * nparts / RW - 1;
  float mm = kNegInf, lsum = 0.f, a[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) a[j] = 0.f;
  // Eight partials per step, all loads issued before the first use; parts
  // past cnt re-read the last valid partial (finite) with weight 0.
  auto load8p = [&](int wb, int cnt, int i0, float (&v)[8][PER]) {
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int i = min(i0 + u, cnt - 1);
      const float* src = P.part_acc + ((size_t)slot_of(wb + i) * P.hq + h) * D + lane;
#pragma unroll
      for (int j = 0; j < PER; ++j) v[u][j] = src[64 * j];
    }
  };
  for (int wb = r0; wb <= r1; wb += 64) {
    const int cnt = min(64, r1 - wb + 1);
    // The (max, sum) loads and the first step's partials go out together:
    // the partial loads do not depend on the weights.
    const size_t r = (size_t)slot_of(wb + min(lane, cnt - 1)) * P.hq + h;
    const float mp0 = P.part_ml[2 * r], lp0 = P.part_ml[2 * r + 1];
    // Up to S steps of eight partials load together with them (a wave of
    // a four-wave row over one long sequence combines 32).
    constexpr int S = 4;
    float v[S][8][PER];
    load8p(wb, cnt, 0, v[0]);
#pragma unroll
    for (int k = 1; k < S; ++k)
      if (8 * k < cnt) load8p(wb, cnt, 8 * k, v[k]);
    // One wait for all the load sets here; left alone, the compiler sinks
    // the partial loads below the reductions and pays a round trip each.
#pragma unroll
    for (int k = 0; k < S; ++k)
      if (k == 0 || 8 * k < cnt) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int j = 0; j < PER; ++j) asm volatile("" ::"v"(v[k][u][j]));
      }
    const float mp = lane < cnt ? mp0 : kNegInf;
    const float lp = lane < cnt ? lp0 : 0.f;
    const float mn = __builtin_fmaxf(mm, wave_max(mp));
    const float ms = safe_max(mn);   // all-empty so far: every weight is 0
    const float a1 = fast_exp2(mm - ms);
    const float w = fast_exp2(mp - ms);  // 0 for empty partials
    lsum = lsum * a1 + wave_sum(w * lp);
#pragma unroll
    for (int j = 0; j < PER; ++j) a[j] *= a1;
    mm = mn;
    auto add8 = [&](int i0, const float (&vs)[8][PER]) {
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float wi = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), min(i0 + u, 63)));
#pragma unroll
        for (int j = 0; j < PER; ++j) a[j] += wi * vs[u][j];
      }
    };
#pragma unroll
    for (int k = 0; k < S; ++k)
      if (8 * k < cnt) add8(8 * k, v[k]);
    for (int i0 = 8 * S; i0 < cnt; i0 += 8) {
      load8p(wb, cnt, i0, v[0]);
      add8(i0, v[0]);
    }
  }
  if constexpr (RW > 1) {
    __shared__ float xa[RW][D];
    __shared__ float xml[RW][2];
#pragma unroll
    for (int j = 0; j < PER; ++j) xa[sub][lane + 64 * j] = a[j];
    if (lane == 0) {
      xml[sub][0] = mm;
      xml[sub][1] = lsum;
    }
    __syncthreads();
    if (sub != 0) return;
    float mx = kNegInf;
#pragma unroll
    for (int q = 0; q < RW; ++q) mx = __builtin_fmaxf(mx, xml[q][0]);
    const float ms = safe_max(mx);
    lsum = 0.f;
#pragma unroll
    for (int j = 0; j < PER; ++j) a[j] = 0.f;
#pragma unroll
    for (int q = 0; q < RW; ++q) {
      const float wq = fast_exp2(xml[q][0] - ms);  // 0 for a wave without partials
      lsum += wq * xml[q][1];
#pragma unroll
      for (int j = 0; j < PER; ++j) a[j] += wq * xa[q][lane + 64 * j];
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
#pragma unroll
  for (int j = 0; j < PER; ++j)
    store_out<OutT>(P.out, ((size_t)b * P.hq + h) * D + lane + 64 * j, a[j] * inv);
}

}  // namespace

namespace {

bool shape_ok(const bc_shape& s) {
  return s.batch >= 1 && s.query_heads >= 1 && s.kv_heads >= 1 &&
         s.query_heads % s.kv_heads == 0 && (s.dim == 64 || s.dim == 128) &&
         s.max_pages >= 1 && s.physical_pages >= 1;
}

template <int D, typename OutT, bool VEC>
void launch_attn(const AttnParams& P, dim3 grid, hipStream_t st) {
  if (P.nwg == 0)
    paged_attn_kernel<D, OutT, VEC, kSlices><<<grid, dim3(64 * kSlices), 0, st>>>(P);
  else
    paged_attn_kernel<D, OutT, VEC, kMaxWaves><<<grid, dim3(64 * P.waves), 0, st>>>(P);
}

template <int D, typename OutT>
hipError_t launch_dim(const AttnParams& P, bool vec, hipStream_t st) {
  const int zgroups = (P.zdim + P.waves - 1) / P.waves;
  const dim3 grid((unsigned)(P.nwg > 0 ? (size_t)P.nwg * zgroups : (size_t)P.batch * P.zdim));
  if (vec) launch_attn<D, OutT, true>(P, grid, st);
  else launch_attn<D, OutT, false>(P, grid, st);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || P.nwg == 0) return err;
  const unsigned rows = (unsigned)P.batch * P.hq;
  // Four waves per row once the ranges outnumber the sequences 16 to 1
  // (never with pair slots, which need more sequences than ranges).
  // Range records come with more than 64 sequences (below, RW = 1): a row
  // per (range boundary, head), then a workgroup per 256 sequences for the
  // empty ones.
  const dim3 g1((rows + 3) / 4);
  const dim3 gm((unsigned)((((size_t)P.nwg - 1) * P.hq + 3) / 4 + ((size_t)P.batch + 255) / 256));
  if (P.nwg >= 16 * P.batch)
    merge_kernel<D, OutT, 4, false, false><<<dim3(rows), 256, 0, st>>>(P);
  else if (P.range_meta && P.pair_slots)
    merge_kernel<D, OutT, 1, true, true><<<gm, 256, 0, st>>>(P);
  else if (P.range_meta)
    merge_kernel<D, OutT, 1, false, true><<<gm, 256, 0, st>>>(P);
  else
    merge_kernel<D, OutT, 1, false, false><<<g1, 256, 0, st>>>(P);
  return hipGetLastError();
}

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

template <typename OutT>
hipError_t launch(AttnParams& P, int dim, hipStream_t st) {
  P.group = P.hq / P.hkv;
  P.nblk = (P.group + kHeadCols - 1) / kHeadCols;
  P.zdim = P.hkv * P.nblk;
  // Flat mode: one wave per head block, up to four per workgroup.  Sliced
  // mode: kSlices waves on one head block, each on a share of the pages.
  P.waves = P.nwg == 0 ? kSlices : P.zdim >= kMaxWaves ? kMaxWaves : P.zdim;
  // 16-byte loads and stores need every buffer they touch aligned: a
  // caller's output or split scratch that is only element-aligned takes the
  // element-wise path too.
  const bool vec = aligned16(P.q) && aligned16(P.kbase) &&
                   aligned16(P.vbase) && aligned16(P.out) &&
                   (P.nwg == 0 || aligned16(P.part_acc)) &&
                   (P.page_stride | P.head_stride | P.slot_stride) % 8 == 0;
  return dim == 64 ? launch_dim<64, OutT>(P, vec, st)
                   : launch_dim<128, OutT>(P, vec, st);
}

using bch::device_cus;

long long zdim_of(const bc_shape& s) {
  const int group = s.query_heads / s.kv_heads;
  return (long long)s.kv_heads * ((group + kHeadCols - 1) / kHeadCols);
}

// Flat ranges for one wave of workgroups: each range runs one wave per head
// block (zdim waves), and kMaxWaves waves per CU keep the most bytes in
// flight (same box, 32/8 heads: one wave more per SIMD measured 5 % slower
// at 64 sequences; at 1-2 head blocks, one workgroup per CU left the CUs
// 16-45 % slower than four waves each).  D = 64 pages carry half the bytes,
// so twice the ranges (eight waves per CU) keep as many in flight: 64
// sequences of up to 4096 tokens 67.1 -> 50.8 us, 128 of them 121.1 -> 92.4.
int flat_ranges(const bc_shape& s, int cus) {
  const long long n =
      (long long)(cus > 0 ? cus : 256) * kMaxWaves * (s.dim == 64 ? 2 : 1) / zdim_of(s);
  return n < 1 ? 1 : n > (1 << 20) ? (1 << 20) : (int)n;
}

// The ranges a launch uses: flat_ranges, but at least two pages per range
// on a full page table (one 4096-token sequence over 256 ranges of one page
// merged 256 partials per row: 11.96 against 10.40 us at 128 ranges).
int launch_ranges(const bc_shape& s, int cus) {
  const long long cap = (long long)s.batch * s.max_pages / 2;
  const int r = flat_ranges(s, cus);
  return cap < 1 ? 1 : cap < r ? (int)cap : r;
}

// Flat-mode workgroup count for bc_decode's `slots` partial slots per head:
// slot = workgroup + sequence must stay below `slots`, and more ranges than
// one wave of workgroups only add partials (one wave: 85.9 us against 103.8
// us for 64 sequences of up to 4096 tokens at 16 splits).
int flat_workgroups(int batch, long long slots, int ranges) {
  long long nwg = slots - batch + 1;
  if (nwg > ranges) nwg = ranges;
  if (nwg < 1) nwg = 1;
  return (int)nwg;
}

// Packed decode with a workspace: one wave of flat ranges.
int packed_nwg(const bc_shape& s) { return launch_ranges(s, device_cus()); }

// Packed decode's partial slots: above 64 sequences, while the ranges number
// under four per sequence, pair slots (AttnParams::pair_slots, 2 * nwg
// slots): the merge then takes one wave per range boundary and loads a row's
// records and first partials in one round, their addresses not depending on
// the sequence (same box, 32/8 heads, against records then partials: 512 x
// U[16, 512] 101.3 -> 100.7-101.1 us, 2048 x U[16, 128] 140.4 -> 139.9-140.3
// us).  Otherwise slot = range + sequence (nwg + batch slots), merged per
// (sequence, head) row: up to 64 sequences it finds the ranges from one round
// of lengths (C5 timed level either way), and with many ranges per sequence
// the boundary rows' first round covers too few of a row's partials (16 x
// U[128, 4096]: 30.9 against 31.5 us).
bool packed_pairs(const bc_shape& s, int nwg) {
  return s.batch > 64 && nwg < 4LL * s.batch;
}

size_t packed_slots(const bc_shape& s, int nwg) {
  return packed_pairs(s, nwg) ? 2 * (size_t)nwg : (size_t)nwg + s.batch;
}

// Workspace: partial accumulators (256-byte aligned), then their (max, sum)
// pairs, then one record per range for the merge kernel.
size_t packed_workspace(const bc_shape& s, int nwg) {
  const size_t slots = packed_slots(s, nwg);
  const size_t acc = (slots * s.query_heads * s.dim * sizeof(float) + 255) & ~(size_t)255;
  return acc + slots * s.query_heads * 2 * sizeof(float) + (size_t)nwg * sizeof(int);
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
  // splits == 1: one workgroup per sequence.  splits > 1: flat ranges whose
  // partial slots fit the caller's splits*B*Hq rows.
  P.nwg = splits == 1 ? 0
                      : flat_workgroups(s.batch, (long long)splits * s.batch,
                                        launch_ranges(s, device_cus()));
  // Above 64 sequences the range records go to the (max, sum) scratch past
  // the slots in use where it has room for them; otherwise the merge kernel
  // finds the ranges from the lengths.
  if (P.nwg > 0 && s.batch > 64) {
    const long long used = (long long)P.nwg + s.batch - 1;
    const long long spare = ((long long)splits * s.batch - used) * s.query_heads * 2;
    if (spare >= P.nwg)
      P.range_meta = reinterpret_cast<int*>(scratch.partial_ml + used * s.query_heads * 2);
  }
  return launch<float>(P, s.dim, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_auto_splits(bc_shape s, int max_length, int cu_count) {
  // splits == 1 runs one workgroup per (sequence, head block) with the pages
  // split kSlices ways inside it and no merge kernel.  splits > 1 runs flat
  // page ranges, min((splits - 1) * batch + 1, R) of them, R = flat_ranges
  // (one wave of workgroups at four waves per CU, eight at D = 64).
  //  - With one or two head blocks, batches whose (sequence, head block)
  //    workgroups fill the CUs stay whole: eight waves per CU beat the
  //    ranges' four there (same box, 1024 tokens: 8/1 heads, 512 sequences
  //    30.5 against 35.5 us at three splits; 16/2 heads, 256 sequences 31.9
  //    against 35.6 us; 1024 sequences of up to 400 tokens, where two
  //    splits are 3 % faster, are the exception measured).
  //  - Batches of R sequences or more take two splits, so R ranges, whatever
  //    the context length: one wave of workgroups streaming many sequences
  //    each beats a launch of one workgroup per (sequence, head block) in
  //    rounds (same box, 32/8 heads, R = 128: 384 sequences of up to 1024
  //    tokens 151.5 against 161.3 us, 512 of up to 256 tokens 68.5 against
  //    86.9 us, 2048 of up to 128 tokens 246.8 against 276.8 us).
  //  - Smaller batches keep the reference's rule that contexts below 512
  //    tokens stay whole (src/paged_gqa.cu:135), and stay whole up to 768
  //    tokens (1024 where their workgroups fill half the CUs or more) while
  //    those workgroups fit the CUs at once.
  //  - Otherwise the smallest split count whose ranges fill the wave, so
  //    that no CU idles: at batch 64 two splits would leave 65 of 128 ranges
  //    (55 % of HBM bandwidth), three fill them (76 %).
  if (s.batch < 1 || s.kv_heads < 1 || s.query_heads < 1 || s.query_heads % s.kv_heads)
    return 1;
  const int cus = cu_count > 0 ? cu_count : 256;
  const int ranges = flat_ranges(s, cus);
  if (ranges <= 1) return 1;
  const long long wgs = (long long)s.batch * zdim_of(s);
  if (zdim_of(s) <= 2 && wgs >= cus) return 1;
  if (s.batch >= ranges) return 2;
  if (max_length < 512) return 1;
  // Unsplit up to 768 tokens; up to 1024 only where the batch's workgroups
  // already fill half the CUs or more (1024 tokens, 32/8 heads, same box:
  // one sequence 12.3 us unsplit against 9.7 us split, 8 sequences 14.4
  // against 12.7, 12 sequences 16.0 against 16.0, 16 sequences 17.0 against
  // 18.0, 32 sequences 23.5 against 24.9 at the best split count).
  if (wgs <= cus && (max_length <= 768 || (max_length <= 1024 && 2 * wgs >= cus))) return 1;
  long long splits = ((long long)ranges + 2LL * s.batch - 2) / s.batch;
  if (splits > BC_MAX_SPLITS) splits = BC_MAX_SPLITS;
  return (int)splits;
}

// Packed decode splits the pages over flat ranges (workspace + merge) unless
// the page table is short enough for the unsplit mode, by the same rule as
// bc_auto_splits with the table's capacity as the context bound; the choice
// needs only the shape, so callers never read lengths back to the host.
static bool packed_split(const bc_shape& s) {
  const long long cap = (long long)s.max_pages * BC_PAGE_SIZE;
  return bc_auto_splits(s, cap > (1 << 30) ? (1 << 30) : (int)cap, device_cus()) > 1;
}

extern "C" size_t bc_packed_decode_workspace_size(bc_shape s) {
  if (!shape_ok(s) || !packed_split(s)) return 0;
  return packed_workspace(s, packed_nwg(s));
}

// The reference's packed_decode rules (src/packed_decode.cu:64-73) plus
// kv_stride >= 1.
static bool packed_args_ok(const bc_shape& s, const bc_half* q, const bc_half* kv,
                           const int32_t* pages, const int32_t* lengths,
                           const bc_half* output, long long bs, long long hs, long long ss,
                           long long kvs, float scale) {
  return shape_ok(s) && q && kv && pages && lengths && output && bs >= 1 && hs >= 1 &&
         ss >= 1 && kvs >= 1 && scale > 0.f;
}

static int packed_common(bc_shape s, const bc_half* q, const bc_half* kv,
                         const int32_t* pages, const int32_t* lengths,
                         bc_half* output, long long bs, long long hs,
                         long long ss, long long kvs, float scale,
                         void* ws, size_t ws_bytes, bc_stream_t stream) {
  if (!packed_args_ok(s, q, kv, pages, lengths, output, bs, hs, ss, kvs, scale))
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
  const int nwg = packed_nwg(s);
  const size_t need = packed_workspace(s, nwg);
  if (ws && ws_bytes >= need && aligned16(ws) && packed_split(s)) {
    P.nwg = nwg;
    P.pair_slots = packed_pairs(s, nwg) ? 1 : 0;
    const size_t slots = packed_slots(s, nwg);
    const size_t acc_bytes =
        (slots * s.query_heads * s.dim * sizeof(float) + 255) & ~(size_t)255;
    P.part_acc = static_cast<float*>(ws);
    P.part_ml = reinterpret_cast<float*>(static_cast<char*>(ws) + acc_bytes);
    // Range records: with pair slots (the merge's boundary rows), and above
    // 64 sequences, where the per-row merge would scan the lengths 64 per
    // round.
    if (P.pair_slots || s.batch > 64)
      P.range_meta = reinterpret_cast<int*>(P.part_ml + slots * s.query_heads * 2);
  }
  return launch<_Float16>(P, s.dim, reinterpret_cast<hipStream_t>(stream));
}

extern "C" int bc_packed_decode(bc_shape s, const bc_half* q,
                                const bc_half* packed_kv, const int32_t* pages,
                                const int32_t* lengths, bc_half* output,
                                long long block_stride, long long head_stride,
                                long long slot_stride, long long kv_stride,
                                float scale, bc_stream_t stream) {
  if (!packed_args_ok(s, q, packed_kv, pages, lengths, output, block_stride, head_stride,
                      slot_stride, kv_stride, scale))
    return BC_ERROR_INVALID_VALUE;
  // The reference's signature has no workspace: a shape that splits borrows
  // a slot of the library's scratch pool for the call (none under graph
  // capture or when the slot is too small: the single pass then runs).
  const size_t need = bc_packed_decode_workspace_size(s);
  const bch::ScratchLease lease(reinterpret_cast<hipStream_t>(stream), need);
  return packed_common(s, q, packed_kv, pages, lengths, output, block_stride,
                       head_stride, slot_stride, kv_stride, scale, lease.get(),
                       lease.get() ? need : 0, stream);
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
  // A workspace that cannot serve the split (null, too small, not 16-byte
  // aligned) is ignored: the call is bc_packed_decode's.
  if (!workspace || !aligned16(workspace) ||
      (shape_ok(s) && workspace_bytes < bc_packed_decode_workspace_size(s)))
    return bc_packed_decode(s, q, packed_kv, pages, lengths, output, block_stride,
                            head_stride, slot_stride, kv_stride, scale, stream);
  return packed_common(s, q, packed_kv, pages, lengths, output, block_stride,
                       head_stride, slot_stride, kv_stride, scale, workspace,
                       workspace_bytes, stream);
}

// ---- bc_packed_decode_noalloc: the split workspace in a static array ----

namespace {

// File-scope device scratch for bc_packed_decode_noalloc: every device the
// library runs on holds its own copy until the process ends.  Host code
// never passes `scratch` itself to a kernel (in host code the name is a
// host-side stand-in, not a device address); it uses the address
// hipGetSymbolAddress returns for the current device.
constexpr size_t kStaticScratchBytes = BC_STATIC_SCRATCH_BYTES;
__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and cached; null if the lookup fails.
void* static_scratch() {
  static std::atomic<void*> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
  void* p = cache[dev].load(std::memory_order_acquire);
  if (p) return p;
  void* addr = nullptr;
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr) return nullptr;
  cache[dev].store(addr, std::memory_order_release);  // the same address if two threads race
  return addr;
}

}  // namespace

extern "C" int bc_packed_decode_noalloc(bc_shape s, const bc_half* q,
                                        const bc_half* packed_kv, const int32_t* pages,
                                        const int32_t* lengths, bc_half* output,
                                        long long block_stride, long long head_stride,
                                        long long slot_stride, long long kv_stride,
                                        float scale, bc_stream_t stream) {
  if (!shape_ok(s)) return BC_ERROR_INVALID_VALUE;
  const size_t need = bc_packed_decode_workspace_size(s);
  if (need > kStaticScratchBytes) return BC_ERROR_OUT_OF_MEMORY;
  void* ws = nullptr;
  if (need > 0) {
    ws = static_scratch();
    if (!ws) return BC_ERROR_INVALID_VALUE;
  }
  return packed_common(s, q, packed_kv, pages, lengths, output, block_stride, head_stride,
                       slot_stride, kv_stride, scale, ws, need, stream);
}
