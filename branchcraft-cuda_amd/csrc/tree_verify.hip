// Ancestor-only tree verification over a shared paged prefix for gfx950.
//
// Reference: tree_kernel / tree_verify (src/tree_attention.cu:14-71,
// 93-105).  The reference gives every (request, node, query head) one warp
// that walks the whole prefix token by token.  Here the query rows of one KV
// head -- nodes x GQA group, e.g. 7 x 4 = 28 -- fill the 32 columns of a
// v_mfma_f32_32x32x16_f16 tile, so each K/V token is read once per request
// and KV head and serves every candidate:
//
//   S^T[32 tok x 32 rows] = K[32 tok x D] . Q^T[D x 32 rows]   (D/16 MFMAs)
//   O^T[D x 32 rows]     += V^T[D x 32 tok] . P^T[32 tok x 32 rows]
//
// P enters the second product as an FP16 hi/lo pair (two MFMAs), so the
// only rounding left is the FP32 accumulation.  The S^T accumulator layout
// is, lane for lane, the B operand of the P.V product once the token order
// inside a 16-token step is permuted, so P never leaves registers; V^T is
// read from LDS with ds_read_b64_tr_b16.  The draft nodes form extra 32-token
// tiles whose scores are masked by the row's ancestor set, walked from the
// parent array (at most N steps, stopping at a parent outside [0, N)).
//
// Kernels:
//  - tree_split_kernel (16-byte aligned tensors, the common path): unit =
//    (request, KV head, row tile); each of a unit's `parts` workgroups takes
//    a range of 32-token tiles (draft tiles first, then prefix tiles), its
//    waves take the range's tiles round-robin with whole-row 16-byte loads
//    staged through per-wave LDS, and merge through LDS; with parts > 1
//    merge_split_kernel combines the FP32 partials.  A single pass over
//    more units than CUs may give one eight-wave workgroup two requests,
//    four waves each on the same tiles.  Workgroup ids put
//    (KV head, row tile) in the low bits, so requests that share prefix
//    pages run on the same XCD and reuse its L2.
//  - tree_rows_kernel: trees of many row tiles per (request, KV head), whose
//    units already fill the CUs: four waves take four row tiles and walk the
//    same K/V tiles, loaded once per workgroup.
//  - tree_kernel: the single pass for tensors that are not 16-byte aligned
//    (element-wise loads and stores).
#include <type_traits>

#include "bc_device.h"
#include "bc_host.h"
#include "bc_slots.h"

namespace {

using namespace bcd;

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 32;       // tokens per MFMA tile (two pages)
// Halves per staged V row: D + 32 spaces the four token rows a 16-lane
// transpose read touches 16 banks apart.
template <int D>
constexpr int v_pitch() { return D + 32; }

struct TreeParams {
  const uint16_t* k;        // prefix K [P,16,Hkv,D]
  const uint16_t* v;        // prefix V
  const int32_t* pages;     // [B, max_pages]
  const int32_t* lengths;   // [B]
  const uint16_t* dq;       // draft Q [B,N,Hq,D]
  const uint16_t* dk;       // draft K [B,N,Hkv,D]
  const uint16_t* dv;       // draft V
  const int32_t* parent;    // [B,N]
  float* out;               // [B,N,Hq,D]
  float* part_acc;          // split-kernel partials (null: one part per unit)
  float* part_ml;
  int batch, nodes, hq, hkv, group, max_pages, phys_pages;
  int rows, row_tiles;      // rows = nodes * group per (request, KV head)
  float scale_log2;
  // tree_split_kernel: parts per unit and tiles per part; with parts > 1,
  // part_acc/part_ml hold P.parts slots per output row.
  int parts, tiles_per_part;
  // ceil(2^32 / d) for d = group and d = row_tiles (0: divide plainly), and
  // whether the launch is a (KV head x row tile, request group, part) grid.
  unsigned long long group_mul, rt_mul;
  int grid3d;
};

// Every kernel argument into scalar registers at the kernel's start, in one
// round of loads.  Otherwise the compiler loads each field where it is first
// used, and a field first used after a branch costs one more serial round
// trip before the kernel's first memory access.
__device__ __forceinline__ void pin_params(const TreeParams& P) {
  asm volatile("" ::"s"(P.k), "s"(P.v), "s"(P.pages), "s"(P.lengths), "s"(P.dq), "s"(P.dk),
               "s"(P.dv), "s"(P.parent), "s"(P.out), "s"(P.part_acc), "s"(P.part_ml),
               "s"(P.batch), "s"(P.nodes), "s"(P.hq), "s"(P.hkv), "s"(P.group),
               "s"(P.max_pages), "s"(P.phys_pages), "s"(P.rows), "s"(P.row_tiles),
               "s"(P.scale_log2), "s"(P.parts), "s"(P.tiles_per_part), "s"(P.group_mul),
               "s"(P.rt_mul), "s"(P.grid3d));
  __builtin_amdgcn_sched_barrier(0);  // nothing that uses them moves above
}

// n / d, as a multiply-high when the host passed mul = ceil(2^32 / d) (exact
// for n * d < 2^32, which the host checks), else a plain division.
__device__ __forceinline__ int div_by(int n, int d, unsigned long long mul) {
  return mul ? (int)(((unsigned long long)(unsigned)n * mul) >> 32) : n / d;
}

__device__ __forceinline__ f16x8 as_f16x8(const uint4 u) {
  return __builtin_bit_cast(f16x8, u);
}

typedef short i16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f16x4 lds_read_tr(const _Float16* p) {
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) i16x4*)(p));
  return __builtin_bit_cast(f16x4, r);
}

template <int D, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void tree_kernel(TreeParams P) {
  pin_params(P);
  constexpr int KS = D / 16;  // MFMA k-steps over the head dimension
  constexpr int DT = D / 32;  // 32-row output tiles over the head dimension
  constexpr int VP = v_pitch<D>();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;   // lane half
  const int lr = lane & 31;  // tile column (query row) / token slot

  const int zdim = P.hkv * P.row_tiles;
  const int z = blockIdx.x % zdim;
  const int b = blockIdx.x / zdim;
  const int kvh = z / P.row_tiles;
  const int rt = z % P.row_tiles;

  // Page ids of this wave's first prefix tile, requested together with the
  // length (they do not depend on it) so the first K/V loads wait for one
  // memory round trip instead of two.
  int ida[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const int pg = wave * (kTile / BC_PAGE_SIZE) + q;
    ida[q] = pg < P.max_pages ? P.pages[(size_t)b * P.max_pages + pg] : -1;
  }
  const int len = max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
  const int ntile_p = (len + kTile - 1) / kTile;
  const int ntile_d = (P.nodes + kTile - 1) / kTile;

  // This lane's query row (tile column lr).
  const int r = rt * 32 + lr;
  const bool rvalid = r < P.rows;
  const int node = rvalid ? r / P.group : 0;
  const int h = kvh * P.group + (rvalid ? r % P.group : 0);
  // Q^T B operand fragments, the same for every wave of the workgroup: wave
  // 0 stages them in LDS (lane-major per k-step), all waves read them back.
  __shared__ uint4 s_q[KS][64];
  __shared__ int s_parent[BC_MAX_TREE_NODES];
  __shared__ __attribute__((aligned(16))) char s_mem[kWaves * kTile * VP * 2];
  __shared__ float s_m[2][32], s_l[2][32];
  // The loads before the first barrier go out together and on one path, so
  // the waits before the LDS stores cover Q and the parents only: the parent
  // array (one entry per thread, the index clamped so every lane loads),
  // each wave's quarter of the Q^T fragments and, further down, the first
  // tile's K.  Rows past the tile's query rows read row (node 0, head h) and
  // store zeros.
  static_assert(BC_MAX_TREE_NODES <= kThreads, "one parent entry per thread");
  constexpr int QS = KS / kWaves;  // Q^T k-steps staged per wave
  static_assert(QS * kWaves == KS, "Q^T k-steps split evenly over the waves");
  const bool has_parent = (int)threadIdx.x < P.nodes;
  const int par = P.parent[(size_t)b * P.nodes + min((int)threadIdx.x, P.nodes - 1)];
  uint4 qf[QS];
  {
    const uint16_t* qp = P.dq + (((size_t)b * P.nodes + node) * P.hq + h) * D + 8 * g;
#pragma unroll
    for (int j = 0; j < QS; ++j) qf[j] = load8<VEC>(qp + 16 * (wave * QS + j));
  }

  _Float16* vs = reinterpret_cast<_Float16*>(s_mem) + wave * kTile * VP;
  // Transpose-read address of this lane: group G = lane/16, j = lane%16.
  const int trG = lane >> 4, trj = lane & 15;
  const _Float16* vtr = vs + (4 * (trG >> 1) + (trj >> 2)) * VP + 16 * (trG & 1) + 4 * (trj & 3);
  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[dt][j] = 0.f;
  float m = kNegInf, l = 0.f;

  const size_t tok_stride = (size_t)P.hkv * D;  // elements between slots
  const int ntile = ntile_p + ntile_d;
  const int nmine = ntile > wave ? (ntile - wave + kWaves - 1) / kWaves : 0;

  // Tile `idx` of this wave is tile wave + kWaves*idx of the workgroup.  The
  // loads of a tile are issued one tile ahead of its MFMAs; issues past the
  // wave's last tile repeat that tile (L2 hits), so every iteration has the
  // same loads in flight and the loop body never exits early.
  auto tile_of = [&](int idx) { return wave + kWaves * min(idx, max(nmine - 1, 0)); };
  // Physical ids of a prefix tile's two pages: uniform scalar loads, fetched
  // one tile before the K/V loads that use them.
  auto ids_of = [&](int idx, int (&ph)[2]) {
    const int it = tile_of(idx);
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pg = it * (kTile / BC_PAGE_SIZE) + q;
      ph[q] = it < ntile_p && pg < P.max_pages ? P.pages[(size_t)b * P.max_pages + pg] : -1;
    }
  };
  // K is loaded one tile ahead; V is requested when its tile starts and is
  // consumed after the scores and softmax.
  auto issue = [&](int idx, const int (&ph)[2], uint4 (&kr)[KS], const uint16_t*& vp, bool& tv,
                   bool (&pok)[2]) {
    const int it = tile_of(idx);
    const uint16_t* kp;
    if (it < ntile_p) {
      const int tbase = it * kTile;
#pragma unroll
      for (int q = 0; q < 2; ++q) pok[q] = ph[q] >= 0 && ph[q] < P.phys_pages;
      const int t = tbase + lr;
      tv = t < len && pok[lr >> 4];
      const size_t phys = (size_t)(tv ? (lr >> 4 ? ph[1] : ph[0]) : 0);
      const size_t off =
          tv ? (phys * BC_PAGE_SIZE + t % BC_PAGE_SIZE) * tok_stride + (size_t)kvh * D : 0;
      // Rows that are not tokens read draft row 0 (always present): with the
      // pool size not given, page 0 of the pool may not exist.
      kp = tv ? P.k + off : P.dk;
      vp = tv ? P.v + off : P.dv;
    } else {
      pok[0] = pok[1] = true;
      const int dn = (it - ntile_p) * kTile + lr;
      tv = dn < P.nodes;
      const size_t off = tv ? (((size_t)b * P.nodes + dn) * P.hkv + kvh) * D : 0;
      kp = P.dk + off;
      vp = P.dv + off;
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) kr[s] = load8<VEC>(kp + 16 * s + 8 * g);
  };

  auto process = [&](int idx, const uint4 (&kr)[KS], const uint16_t* vp, bool tv,
                     const bool (&pok)[2]) {
    if (idx >= nmine) return;  // padding step
    uint4 vr[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) vr[s] = load8<VEC>(vp + 16 * s + 8 * g);
    const int it = wave + kWaves * idx;
    const bool is_draft = it >= ntile_p;
    const int tbase = (is_draft ? it - ntile_p : it) * kTile;
    // Valid token rows of the tile as a bit mask (bit i = token tbase + i):
    // prefix tiles stop at the length and drop pages outside the pool
    // (uniform over the wave); draft tiles take this row's ancestor-or-self
    // set.
    uint32_t okbits;
    if (!is_draft) {
      const int hi = min(max(len - tbase, 0), kTile);
      okbits = (hi >= kTile ? ~0u : (1u << hi) - 1u) &
               ((pok[0] ? 0x0000ffffu : 0u) | (pok[1] ? 0xffff0000u : 0u));
    } else {
      okbits = 0;
      int cur = node;
      for (int steps = 0; steps < P.nodes && cur >= 0 && cur < P.nodes; ++steps) {
        if (cur >= tbase && cur < tbase + kTile) okbits |= 1u << (cur - tbase);
        cur = s_parent[cur];
      }
    }
    // Rows past the prefix or the node count may hold any bits (NaN
    // included); their weight is zero, so their V row must be zero too.
    if (is_draft || okbits != ~0u) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        vr[s].x = tv ? vr[s].x : 0u;
        vr[s].y = tv ? vr[s].y : 0u;
        vr[s].z = tv ? vr[s].z : 0u;
        vr[s].w = tv ? vr[s].w : 0u;
      }
    }

    // ---- S^T = K Q^T ----
    f32x16 sc;
#pragma unroll
    for (int j = 0; j < 16; ++j) sc[j] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s)
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(kr[s]),
                                                  as_f16x8(s_q[s][lane]), sc, 0, 0, 0);

    // ---- stage V row-major while the MFMAs drain ----
#pragma unroll
    for (int s = 0; s < KS; ++s)
      *reinterpret_cast<uint4*>(vs + lr * VP + 16 * s + 8 * g) = vr[s];

    // ---- mask and online softmax (column lr = query row) ----
    // sc[j] holds token row 8*(j/4) + 4*g + j%4.
    const uint32_t ob = okbits >> (4 * g);
    float sv[16];
    float tmax = kNegInf;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const bool ok = (ob >> (8 * (j >> 2) + (j & 3))) & 1u;
      sv[j] = ok ? sc[j] * P.scale_log2 : kNegInf;
      tmax = __builtin_fmaxf(tmax, sv[j]);
    }
    tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 32));
    // The running max moves only when it would grow by more than
    // kRescaleSlack (log2 units): weights then stay below 2^kRescaleSlack and
    // most tiles skip rescaling the accumulators.
    const float mnew = __builtin_fmaxf(m, tmax);
    if (__builtin_amdgcn_ballot_w64(mnew > m + kRescaleSlack)) {
      const float alpha = fast_exp2(m - safe_max(mnew));
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[dt][j] *= alpha;
      m = mnew;
    }
    // P is split into FP16 hi + lo parts (two MFMAs each) so the P.V product
    // carries ~21 bits of P instead of FP16's 11.
    const float mb = safe_max(m);
    f16x8 pb[2], pl[2];
    float pr[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pr[j] = fast_exp2(sv[j] - mb);
      l += pr[j];
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      uint32_t wh[4], wl[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        split_hi_lo(pr[8 * hh + 2 * q], pr[8 * hh + 2 * q + 1], wh[q], wl[q]);
      pb[hh] = __builtin_bit_cast(f16x8, u32x4{wh[0], wh[1], wh[2], wh[3]});
      pl[hh] = __builtin_bit_cast(f16x8, u32x4{wl[0], wl[1], wl[2], wl[3]});
    }

    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    // ---- O^T += V^T P^T; A operand tokens 16st + 8hf + 4g + k, dim lr ----
    // The MFMAs go round the DT accumulators, so consecutive ones are
    // independent: one accumulator's chain of four would wait out each
    // MFMA's latency in turn.
    f16x8 av[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const f16x4 lo = lds_read_tr(vtr + (16 * st) * VP + 32 * dt);
        const f16x4 hi = lds_read_tr(vtr + (16 * st + 8) * VP + 32 * dt);
        av[dt][st] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pb[st], acc[dt], 0, 0, 0);
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pl[st], acc[dt], 0, 0, 0);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  uint4 ka[KS], kb[KS];
  const uint16_t* va = P.v;
  const uint16_t* vb = P.v;
  bool ta = false, tb = false;
  bool pa[2] = {true, true}, pbk[2] = {true, true};
  int idb[2];
  // The first tile's loads go out before Q and the parent array are stored
  // and published by the barrier.  A wave without tiles issues them too
  // (tile_of clamps, and every address stays inside its tensor) so that all
  // waves run the same code up to the barrier.
  issue(0, ida, ka, va, ta, pa);
#pragma unroll
  for (int j = 0; j < QS; ++j)
    s_q[wave * QS + j][lane] = rvalid ? qf[j] : make_uint4(0, 0, 0, 0);
  if (has_parent) s_parent[threadIdx.x] = par;
  ids_of(1, idb);
  __syncthreads();
  if (nmine > 0) {
    for (int idx = 0; idx < nmine; idx += 2) {
      issue(idx + 1, idb, kb, vb, tb, pbk);
      ids_of(idx + 2, ida);
      process(idx, ka, va, ta, pa);
      issue(idx + 2, ida, ka, va, ta, pa);
      ids_of(idx + 3, idb);
      process(idx + 1, kb, vb, tb, pbk);
    }
  }
  // Both lane halves share m; combine their partial sums.
  l += shfl_xor_f(l, 32);

  // ---- merge the four waves: 3,2 -> 1,0 then 1 -> 0 through LDS ----
  // Rows are padded to D + 4 floats so the 32 rows a float4 access touches
  // fall in different LDS banks.
  constexpr int XP = D + 4;
  static_assert(kWaves * kTile * VP * 2 >= 2 * 32 * XP * 4, "merge buffer fits");
  float* xacc = reinterpret_cast<float*>(s_mem);  // [2][32 rows][XP]
  auto put = [&](int slot) {
    float* dst = xacc + (size_t)slot * 32 * XP + (size_t)lr * XP;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        float4 v4 = make_float4(acc[dt][4 * jq], acc[dt][4 * jq + 1],
                                acc[dt][4 * jq + 2], acc[dt][4 * jq + 3]);
        *reinterpret_cast<float4*>(dst + 32 * dt + 8 * jq + 4 * g) = v4;
      }
    if (g == 0) {
      s_m[slot][lr] = m;
      s_l[slot][lr] = l;
    }
  };
  auto take = [&](int slot) {
    const float* src = xacc + (size_t)slot * 32 * XP + (size_t)lr * XP;
    const float m2 = s_m[slot][lr], l2 = s_l[slot][lr];
    const float mm = __builtin_fmaxf(m, m2);
    const float a1 = fast_exp2(m - safe_max(mm)), a2 = fast_exp2(m2 - safe_max(mm));
    l = l * a1 + l2 * a2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq) {
        const float4 v4 = *reinterpret_cast<const float4*>(src + 32 * dt + 8 * jq + 4 * g);
        acc[dt][4 * jq] = acc[dt][4 * jq] * a1 + v4.x * a2;
        acc[dt][4 * jq + 1] = acc[dt][4 * jq + 1] * a1 + v4.y * a2;
        acc[dt][4 * jq + 2] = acc[dt][4 * jq + 2] * a1 + v4.z * a2;
        acc[dt][4 * jq + 3] = acc[dt][4 * jq + 3] * a1 + v4.w * a2;
      }
    m = mm;
  };
  __syncthreads();  // V^T staging area is reused below
  if (wave >= 2) put(wave - 2);
  __syncthreads();
  if (wave < 2) take(wave);
  __syncthreads();
  if (wave == 1) put(0);
  __syncthreads();
  if (wave != 0) return;
  take(0);
  if (!rvalid) return;

  // ---- write: lane holds O^T[32dt + 8jq + 4g + e][row r] ----
  float* dst = P.out + (((size_t)b * P.nodes + node) * P.hq + h) * D;
  const float inv = 1.f / l;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq)
      store4f<VEC>(dst + 32 * dt + 8 * jq + 4 * g, acc[dt][4 * jq] * inv,
                   acc[dt][4 * jq + 1] * inv, acc[dt][4 * jq + 2] * inv,
                   acc[dt][4 * jq + 3] * inv);
}

// ---- per-tile pieces of tree_split_kernel ----

// Valid tokens of a prefix tile: the first `valid` rows (clipped to
// [0, 32]), minus the 16-row halves whose page id lies outside the pool.
__device__ __forceinline__ uint32_t prefix_bits(int valid, int id0, int id1, int phys) {
  const int hi = min(max(valid, 0), kTile);
  return (hi >= kTile ? ~0u : (1u << hi) - 1u) &
         ((id0 >= 0 && id0 < phys ? 0x0000ffffu : 0u) |
          (id1 >= 0 && id1 < phys ? 0xffff0000u : 0u));
}

// parent[i] for i in [0, nodes) from the parent registers (lane i of
// register c holds parent[i + 64c]).
__device__ __forceinline__ int parent_at(const int (&parr)[4], int nodes, int i) {
  if (nodes <= 64) return __shfl(parr[0], i, 64);
  const int c0 = __shfl(parr[0], i & 63, 64), c1 = __shfl(parr[1], i & 63, 64);
  const int c2 = __shfl(parr[2], i & 63, 64), c3 = __shfl(parr[3], i & 63, 64);
  const int c = i >> 6;
  return c == 0 ? c0 : c == 1 ? c1 : c == 2 ? c2 : c3;
}

// Valid tokens of the draft tile starting at node tbase for the lane's
// query row: its node and that node's ancestors.  Lanes walk different
// chains, so the loop runs until every lane's walk has ended (a parent
// outside [0, nodes) ends it; at most `nodes` steps).
__device__ __forceinline__ uint32_t ancestor_bits(const int (&parr)[4], int nodes, int node,
                                                  int tbase) {
  uint32_t okbits = 0;
  int cur = node;
  for (int steps = 0; steps < nodes; ++steps) {
    const bool live = cur >= 0 && cur < nodes;
    if (!__builtin_amdgcn_ballot_w64(live)) break;
    if (live && cur >= tbase && cur < tbase + kTile) okbits |= 1u << (cur - tbase);
    const int nx = parent_at(parr, nodes, live ? cur : 0);
    cur = live ? nx : -1;
  }
  return okbits;
}

// One 32-token tile staged in LDS (K rows at a pitch of D + 8 halves, V
// rows at D + 16), in two steps.  tile_scores: S^T = K Q^T as one MFMA
// chain over the k-steps and the masked online-softmax update of (m, l,
// acc), leaving P as an FP16 hi/lo pair; tile_pv: O^T += V^T P^T.  kr is
// this lane's K row (token lr), vtr its transpose-read address in the V
// rows, qf this lane's Q^T B-operand fragments (k-step s at qf[QS s]: in
// LDS, QS = 64; in registers, QS = 1) and okbits the valid tokens of the
// lane's query row.
// FIRST: the wave's first tile; its running max starts at -inf and acc is
// not yet defined, so the rescale is skipped (tile_pv then starts acc from
// zero).
template <int D, int QS, bool FIRST>
__device__ __forceinline__ void tile_scores(const _Float16* kr, const uint4* qf,
                                            uint32_t okbits, float scale_log2, int g,
                                            f32x16 (&acc)[D / 32], float& m, float& l,
                                            f16x8 (&pb)[2], f16x8 (&pl)[2]) {
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  f32x16 sc;
#pragma unroll
  for (int j = 0; j < 16; ++j) sc[j] = 0.f;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    const uint4 k0 = *reinterpret_cast<const uint4*>(kr + 16 * s + 8 * g);
    sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(k0), as_f16x8(qf[QS * s]), sc, 0, 0, 0);
  }
  // sc[j] holds token row 8*(j/4) + 4*g + j%4.  Scores stay unscaled here;
  // the scale enters the running max once and the exp2 argument as an FMA.
  float sv[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) sv[j] = sc[j];
  if (__builtin_amdgcn_ballot_w64(okbits != ~0u)) {  // masked tokens in the tile
    const uint32_t ob = okbits >> (4 * g);
#pragma unroll
    for (int j = 0; j < 16; ++j)
      sv[j] = (ob >> (8 * (j >> 2) + (j & 3))) & 1u ? sv[j] : kNegInf;
  }
  float tmax = kNegInf;
#pragma unroll
  for (int j = 0; j < 16; ++j) tmax = __builtin_fmaxf(tmax, sv[j]);
  tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 32)) * scale_log2;
  if constexpr (FIRST) {
    m = tmax;  // l is still 0
  } else {
    const float mnew = __builtin_fmaxf(m, tmax);
    if (__builtin_amdgcn_ballot_w64(mnew > m + kRescaleSlack)) {
      const float alpha = fast_exp2(m - safe_max(mnew));
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[dt][j] *= alpha;
      m = mnew;
    }
  }
  // P splits into an FP16 hi part (p truncated to FP16, exact for p in
  // [2^-14, 2^8]) and lo = p - hi rounded to FP16, so P.V carries ~21 bits
  // of P.
  const float mb = safe_max(m);
  float pr[16];
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    pr[j] = fast_exp2(__builtin_fmaf(sv[j], scale_log2, -mb));
    l += pr[j];
  }
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    uint32_t wh[4], wl[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) split_hi_lo(pr[8 * h + 2 * q], pr[8 * h + 2 * q + 1], wh[q], wl[q]);
    pb[h] = __builtin_bit_cast(f16x8, u32x4{wh[0], wh[1], wh[2], wh[3]});
    pl[h] = __builtin_bit_cast(f16x8, u32x4{wl[0], wl[1], wl[2], wl[3]});
  }
}

// FIRST: acc starts from zero (the first MFMA of each accumulator takes a
// zero C operand).
template <int D, bool FIRST>
__device__ __forceinline__ void tile_pv(const _Float16* vtr, const f16x8 (&pb)[2],
                                        const f16x8 (&pl)[2], f32x16 (&acc)[D / 32]) {
  constexpr int DT = D / 32;
  constexpr int VP = D + 16;
  // ---- O^T += V^T P^T; A operand tokens 16st + 8hf + 4g + k, dim lr ----
  // The MFMAs go round the DT accumulators, so consecutive ones are
  // independent.
  f16x8 av[DT][2];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const f16x4 lo = lds_read_tr(vtr + (16 * st) * VP + 32 * dt);
      const f16x4 hi = lds_read_tr(vtr + (16 * st + 8) * VP + 32 * dt);
      av[dt][st] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  const f32x16 zero = {};
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pb[st],
                                                       FIRST && st == 0 ? zero : acc[dt], 0, 0,
                                                       0);
#pragma unroll
  for (int st = 0; st < 2; ++st)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pl[st], acc[dt], 0, 0, 0);
}

// Wave-local LDS handoff: this wave's LDS writes are visible to its own
// later reads (and its reads done before its later writes).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Split tree verification.  Unit = (request, KV head, row tile); its work is
// one tile space: the draft tiles [0, ntd) followed by the prefix tiles (32
// tokens each, up to the request's length).  Workgroup `part` of a unit
// takes tiles [part*T, part*T + T), T = P.tiles_per_part, and its W waves
// take those tiles round-robin.  The row tile's Q^T fragments are fetched
// once per workgroup into LDS, where the score MFMAs read them.  A wave
// loads a tile's K and V as whole token rows (each 16-byte load instruction
// covers complete 128-byte lines: measured 2x the tile rate of loading K in
// the MFMA operand layout, where an instruction touches 32 rows), stages
// them in its own LDS area -- K rows at a pitch for conflict-free A-operand
// reads, V rows at a pitch for transpose reads -- and issues the next tile's
// loads as soon as the rows are staged, so they are in flight during the
// current tile's MFMAs.  Masks, softmax and the hi/lo P.V product are
// tree_kernel's.  The waves merge through LDS, each thread combining the
// waves' states for its share of a row; with one part per unit (no
// workspace) that share goes to the output, otherwise every part with tiles
// writes an FP32 partial per row, slot (row, part), and merge_split_kernel
// combines them.
template <int D, int W, int RQ>
__global__ __launch_bounds__(64 * W, 2) void tree_split_kernel(TreeParams P) {
  constexpr int KS = D / 16;      // MFMA k-steps; also load instructions per tile
  constexpr int DT = D / 32;      // 32-row output tiles over the head dimension
  constexpr int KP = D + 8;       // halves per staged K row
  constexpr int VP = D + 16;      // halves per staged V row
  constexpr int LPR = D / 8;      // lanes per token row in a whole-row load
  constexpr int RPI = 64 / LPR;   // token rows per load instruction
  static_assert(RPI * KS == kTile, "KS whole-row loads cover a tile");
  constexpr int STAGE = kTile * (KP + VP);  // halves per wave
  constexpr int LN = W / RQ;      // waves per request

  pin_params(P);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;   // lane half
  const int lr = lane & 31;  // tile column (query row) / token slot

  // RQ requests per workgroup: wave w serves request RQ*group + w/LN and
  // takes every LN-th tile from w%LN, so the RQ requests walk the same
  // tiles at the same time (their shared pages then meet in the CU's L1).
  const int rq = wave / LN;
  const int ln = wave % LN;
  // Workgroup ids put (KV head, row tile) in the low bits, then the request
  // group, then the part (a 3-D grid, or the same order flattened).
  int z, b0, part;
  if (P.grid3d) {
    z = blockIdx.x;
    b0 = blockIdx.y * RQ;
    part = blockIdx.z;
  } else {
    const int zdim = P.hkv * P.row_tiles;
    const int units = zdim * ((P.batch + RQ - 1) / RQ);
    const int unit = blockIdx.x % units;
    part = blockIdx.x / units;
    z = unit % zdim;
    b0 = (unit / zdim) * RQ;
  }
  const bool present = b0 + rq < P.batch;  // uniform per wave
  const int b = present ? b0 + rq : b0;    // absent waves read request b0, unused
  const int kvh = div_by(z, P.row_tiles, P.rt_mul);
  const int rt = z - kvh * P.row_tiles;
  const int T = P.tiles_per_part;
  const int tbeg = part * T;

  // Page ids of this wave's tiles as vector loads (lane j: page j%2 of the
  // wave's tile j/2, 32 tiles per register, the next 32 fetched a chunk
  // ahead).  Scalar loads would share lgkmcnt with the LDS reads of every
  // tile, whose waits would then also wait for the prefetched ids.
  //
  // Every load of the start is unconditional, from an address inside the
  // request's table row (the page index clamped), and what the entry means
  // is decided where it is used: a load under a condition is a branch, and
  // after one the compiler's wait for the kernel arguments also waits for
  // every scalar load in flight, which made the first two ids and the length
  // three serial round trips ahead of the first Q and K/V loads.  The values
  // that depend on the length are formed after those loads are issued.
  const int ntd = (P.nodes + kTile - 1) / kTile;  // draft tiles come first
  const size_t prow = (size_t)b * P.max_pages;
  auto table_entry = [&](int pg) { return P.pages[prow + min(max(pg, 0), P.max_pages - 1)]; };
  // Raw entries of chunk `chunk` (ids_of keeps those that are ids).
  auto load_ids = [&](int chunk) {
    const int it = tbeg + ln + LN * (chunk * 32 + (lane >> 1));
    return table_entry((it - ntd) * (kTile / BC_PAGE_SIZE) + (lane & 1));
  };
  int idv = load_ids(0);
  int idv_next = load_ids(1);

  const int r = rt * 32 + lr;
  const bool rvalid = r < P.rows;
  const int rnode = div_by(r, P.group, P.group_mul);
  const int node = rvalid ? rnode : 0;
  const int h = kvh * P.group + (rvalid ? r - rnode * P.group : 0);

  // Q stays in LDS (see s_q below) except in the D = 64 two-request
  // workgroups.
  constexpr bool QL = !(D == 64 && RQ == 2);
  // Q^T fragments: with Q in LDS, the LN waves of a request load KS / LN of
  // them each into s_q, so the workgroup fetches each fragment once instead
  // of once per wave (every wave of a request reads the same rows).  Q and
  // the parents load without selects (a select right after a load would wait
  // for it there): lanes past the tile's query rows read row (node 0, head
  // h), whose scores land in columns that are never written out, and parent
  // entries past the node count repeat the last one and are never read
  // (walks visit nodes in [0, nodes) only).
  constexpr int QPW = QL ? (KS + LN - 1) / LN : KS;  // fragments loaded per wave
  uint4 qown[QPW];
  {
    const uint16_t* qp = P.dq + (((size_t)b * P.nodes + node) * P.hq + h) * D + 8 * g;
#pragma unroll
    for (int j = 0; j < QPW; ++j)
      qown[j] = ldg16(qp + 16 * (QL ? min(ln + LN * j, KS - 1) : j));
  }

  // A wave whose first tile is a draft tile (part 0's first waves: draft
  // tiles come first) needs neither a page id nor the length for it, which
  // the launch geometry alone tells; the other waves load tile 0's two
  // entries and the length as scalar loads, together, after the vector loads
  // above.  Only scalar loads sit under this condition: vector loads under a
  // condition would leave the compiler's wait counts after it assuming the
  // fewest either side issued.
  const bool early = tbeg + ln < ntd;  // uniform
  const int pg0 = (tbeg + ln - ntd) * (kTile / BC_PAGE_SIZE);
  int raw0 = -1, raw1 = -1, len_raw = 0;
  if (!early) {
    raw0 = table_entry(pg0);
    raw1 = table_entry(pg0 + 1);
    len_raw = P.lengths[b];
  }
  int cur[2] = {-1, -1};
  int len = 0, ntot = 0, nmine = 0;
  auto set_lengths = [&]() {
    len = max(0, min(len_raw, P.max_pages * BC_PAGE_SIZE));
    ntot = ntd + (len + kTile - 1) / kTile;
    const int tend = min(tbeg + T, ntot);
    nmine = present && tend > tbeg + ln ? (tend - tbeg - ln + LN - 1) / LN : 0;
  };

  __shared__ __attribute__((aligned(16))) _Float16 s_stage[W * STAGE];
  // Q^T B operand of each request's row tile: lane (g, lr) of k-step s
  // holds Q[row lr][16s + 8g .. +8] (rows past the tile's query rows: row
  // (node 0, head h), unused).  It stays in LDS for the whole kernel (read
  // back per tile, which keeps 32 registers free), except in the D = 64
  // two-request workgroups, where it would leave room for one workgroup per
  // CU instead of two: there every wave holds it in registers.  The parent
  // array in registers: lane i holds parent[i + 64c] (c < 4), so a wave
  // walks ancestor chains with lane shuffles.
  __shared__ uint4 s_q[QL ? RQ * KS * 64 : 1];
  uint4 qreg[QL ? 1 : KS];
  static_assert(BC_MAX_TREE_NODES <= 256, "four parent registers per lane");
  int parr[4];

  _Float16* const ks = s_stage + wave * STAGE;
  _Float16* const vs = ks + kTile * KP;
  const int trG = lane >> 4, trj = lane & 15;
  const _Float16* vtr = vs + (4 * (trG >> 1) + (trj >> 2)) * VP + 16 * (trG & 1) + 4 * (trj & 3);
  // Whole-row load geometry: load s of a lane covers token row
  // s*RPI + lane/LPR, dims 8*(lane%LPR) .. +8.
  const int lrow = lane / LPR, lcol = 8 * (lane % LPR);
  const size_t tok_stride = (size_t)P.hkv * D;

  f32x16 acc[DT];  // defined by the first tile, or zeroed for a wave without tiles
  float m = kNegInf, l = 0.f;

  uint4 kreg[KS], vreg[KS];
  uint32_t rowok = 0;  // bit s: this lane's row of load s is a valid token
  constexpr uint32_t kAllRows = (1u << KS) - 1;
  // Byte offset of this lane's 16 bytes in whole-row load j of a page (j <
  // KS/2 loads per page: token row j*RPI + lrow, dims lcol .. +8); a prefix
  // tile's loads are then a uniform page base plus these offsets.
  constexpr int LPP = KS / 2;
  unsigned loff[LPP];
#pragma unroll
  for (int j = 0; j < LPP; ++j)
    loff[j] = (unsigned)((((size_t)(j * RPI + lrow)) * tok_stride + lcol) * sizeof(uint16_t));
  const size_t page_elems = (size_t)BC_PAGE_SIZE * tok_stride;
  // Issue the loads of this wave's tile `idx` from page ids ph.  Pages
  // outside the pool read page 0 and rows past the length read their page's
  // rows (all in bounds); both are masked.
  // K and V are issued apart (K first), so a wave can wait for K alone;
  // draft_tag (std::true_type: a draft tile) picks the address form at
  // compile time.
  auto issue_half = [&](int idx, const int (&ph)[2], bool is_v, auto draft_tag) {
    const int it = tbeg + ln + LN * idx - ntd;  // prefix tile index when >= 0
    uint4 (&dst)[KS] = is_v ? vreg : kreg;
    if constexpr (!decltype(draft_tag)::value) {
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const bool okp = ph[q] >= 0 && ph[q] < P.phys_pages;
        const size_t base = (size_t)(okp ? ph[q] : 0) * page_elems + (size_t)kvh * D;
        const char* src = reinterpret_cast<const char*>((is_v ? P.v : P.k) + base);
#pragma unroll
        for (int j = 0; j < LPP; ++j) dst[q * LPP + j] = *reinterpret_cast<const uint4*>(src + loff[j]);
      }
    } else {
      // Rows past the node count read the last node's row (masked); the
      // clamp, unlike a select of addresses, keeps the loads branch-free.
      const uint16_t* src = is_v ? P.dv : P.dk;
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const int dn = min((it + ntd) * kTile + s * RPI + lrow, P.nodes - 1);
        dst[s] = ldg16(src + (((size_t)b * P.nodes + dn) * P.hkv + kvh) * D + lcol);
      }
    }
  };
  // Rows of the wave's tile `idx` that hold valid tokens (bit s: this
  // lane's row of load s).
  auto rows_of = [&](int idx, const int (&ph)[2]) {
    const int it = tbeg + ln + LN * idx - ntd;
    uint32_t ok = 0;
    if (it >= 0) {
      const int tb = it * kTile;
      const bool okp0 = ph[0] >= 0 && ph[0] < P.phys_pages;
      const bool okp1 = ph[1] >= 0 && ph[1] < P.phys_pages;
      if (okp0 && okp1 && tb + kTile <= len) return kAllRows;  // uniform: every row valid
#pragma unroll
      for (int s = 0; s < KS; ++s)
        ok |= (s < LPP ? okp0 : okp1) && tb + s * RPI + lrow < len ? 1u << s : 0u;
    } else {
#pragma unroll
      for (int s = 0; s < KS; ++s)
        ok |= (it + ntd) * kTile + s * RPI + lrow < P.nodes ? 1u << s : 0u;
    }
    return ok;
  };
  // One tile's loads: K (is_v false), V (true), or both.
  auto issue_part = [&](int idx, const int (&ph)[2], bool k, bool v) {
    if (tbeg + ln + LN * idx < ntd) {
      if (k) issue_half(idx, ph, false, std::true_type{});
      if (v) issue_half(idx, ph, true, std::true_type{});
    } else {
      if (k) issue_half(idx, ph, false, std::false_type{});
      if (v) issue_half(idx, ph, true, std::false_type{});
    }
    if (v) rowok = rows_of(idx, ph);
  };
  auto issue = [&](int idx, const int (&ph)[2]) { issue_part(idx, ph, true, true); };

  // first_tag: std::true_type for the wave's first tile (a separate copy
  // of the tile code), std::false_type for the rest.
  // Valid token rows of tile idx as a bit mask (bit i = token tbase + i):
  // prefix tiles clip at the length and drop pages outside the pool; draft
  // tiles take this row's ancestor-or-self set.
  auto okbits_of = [&](int idx, const int (&ph)[2], bool is_draft) {
    const int it = tbeg + ln + LN * idx;
    const int tbase = (is_draft ? it : it - ntd) * kTile;
    return is_draft ? ancestor_bits(parr, P.nodes, node, tbase)
                    : prefix_bits(len - tbase, ph[0], ph[1], P.phys_pages);
  };
  // staged: the tile's rows are in the staging area already (an early
  // wave's first tile, see below).
  auto process = [&](int idx, uint32_t okbits, const int (&next_ids)[2], auto first_tag,
                     bool staged = false) {
    // Stage K and V rows; rows that are not valid tokens may hold any bits
    // (NaN included): their weight is zero, so their V row must be zero.
    auto stage_v = [&]() {
#pragma unroll
      for (int s = 0; s < KS; ++s)
        *reinterpret_cast<uint4*>(vs + (s * RPI + lrow) * VP + lcol) = vreg[s];
      if (__builtin_amdgcn_ballot_w64(rowok != kAllRows)) {  // rows past the data: zero V
#pragma unroll
        for (int s = 0; s < KS; ++s)
          if (!((rowok >> s) & 1u))
            *reinterpret_cast<uint4*>(vs + (s * RPI + lrow) * VP + lcol) = make_uint4(0, 0, 0, 0);
      }
    };
    constexpr bool first = decltype(first_tag)::value;
    if (!staged) {
#pragma unroll
      for (int s = 0; s < KS; ++s)
        *reinterpret_cast<uint4*>(ks + (s * RPI + lrow) * KP + lcol) = kreg[s];
      // The first tile's scores start as soon as its K is staged (its V was
      // issued after K and Q); later tiles stage both, then issue the next
      // tile's loads, which are then in flight during this tile's MFMAs.
      if (!first) stage_v();
    }
    wave_lds_sync();
    if (!first && idx + 1 < nmine) issue(idx + 1, next_ids);
    // The first tile's K registers are free once K is staged: the next
    // tile's K loads go out now, its V loads once this tile's V is staged.
    if (first && idx + 1 < nmine) issue_part(idx + 1, next_ids, true, false);
    f16x8 pb[2], pl[2];
    if constexpr (QL)
      tile_scores<D, 64, first>(ks + lr * KP, s_q + (size_t)rq * KS * 64 + lane, okbits,
                                P.scale_log2, g, acc, m, l, pb, pl);
    else
      tile_scores<D, 1, first>(ks + lr * KP, qreg, okbits, P.scale_log2, g, acc, m, l, pb, pl);
    if constexpr (first) {
      stage_v();
      wave_lds_sync();
      if (idx + 1 < nmine) issue_part(idx + 1, next_ids, false, true);
    }
    tile_pv<D, first>(vtr, pb, pl, acc);
    // The staging area is rewritten by the next tile.
    wave_lds_sync();
  };

  // Ids of the wave's tile idx < nmine: entries past the page table read as
  // -1 (a draft tile's entries are never used).
  auto ids_of = [&](int idx, int (&ph)[2]) {
    if ((idx & 31) == 0 && idx > 0) {  // uniform: move to the next chunk of ids
      idv = idv_next;
      if (T > 32 * LN * ((idx >> 5) + 1)) idv_next = load_ids((idx >> 5) + 1);
    }
    const int pg = (tbeg + ln + LN * idx - ntd) * (kTile / BC_PAGE_SIZE);
    const int r0 = __builtin_amdgcn_readlane(idv, 2 * (idx & 31));
    const int r1 = __builtin_amdgcn_readlane(idv, 2 * (idx & 31) + 1);
    ph[0] = pg >= 0 && pg < P.max_pages ? r0 : -1;
    ph[1] = pg >= 0 && pg + 1 < P.max_pages ? r1 : -1;
  };
  auto load_parents = [&]() {
#pragma unroll
    for (int c = 0; c < 4; ++c)
      parr[c] = P.parent[(size_t)b * P.nodes + min(lane + 64 * c, P.nodes - 1)];
  };
  // This wave's Q fragments into s_q.  Each path below writes them itself:
  // the compiler's wait for Q at a point both paths reach is the stricter of
  // the two, and it would make the later path wait for its whole first tile.
  auto publish_q = [&]() {
    if constexpr (QL) {
#pragma unroll
      for (int j = 0; j < QPW; ++j)
        if (ln + LN * j < KS) s_q[((size_t)rq * KS + ln + LN * j) * 64 + lane] = qown[j];
    }
  };
  // Tile 0's loads, one straight-line sequence for draft and prefix tiles
  // alike (each address selected per wave): K, the parents, then V, so a
  // prefix tile's scores wait for Q and K only.  A wave without tiles issues
  // them too (pages outside the pool read page 0, draft rows past the node
  // count the last node's row, all in bounds), so every wave runs the same
  // loads and barriers.  Only a prefix tile's addresses wait for the scalar
  // loads above; an early wave issues its draft tile's loads at once and
  // stages the tile before the Q barrier, and after the barrier its first
  // step issues the second tile's loads (in single passes over short
  // prefixes this is the wave with the extra tile: one request over 256
  // tokens has 9 tiles for 8 waves).
  auto issue_first = [&](bool is_v) {
    uint4 (&dst)[KS] = is_v ? vreg : kreg;
    const uint16_t* pbase = is_v ? P.v : P.k;
    const uint16_t* dbase = is_v ? P.dv : P.dk;
    const int dn0 = (tbeg + ln) * kTile + lrow;  // draft row of load 0 (early waves)
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const bool okp = cur[q] >= 0 && cur[q] < P.phys_pages;
      const char* pg = reinterpret_cast<const char*>(
          pbase + (size_t)(okp ? cur[q] : 0) * page_elems + (size_t)kvh * D);
#pragma unroll
      for (int j = 0; j < LPP; ++j) {
        const int s = q * LPP + j;
        const int dn = min(dn0 + s * RPI, P.nodes - 1);
        const uint16_t* da = dbase + (((size_t)b * P.nodes + dn) * P.hkv + kvh) * D + lcol;
        dst[s] = *(early ? reinterpret_cast<const uint4*>(da)
                         : reinterpret_cast<const uint4*>(pg + loff[j]));
      }
    }
  };
  __builtin_amdgcn_sched_barrier(0);  // Q's loads go out before the id wait
  if (!early) {
    cur[0] = pg0 >= 0 && pg0 < P.max_pages ? raw0 : -1;
    cur[1] = pg0 >= 0 && pg0 + 1 < P.max_pages ? raw1 : -1;
  }
  issue_first(false);
  load_parents();
  issue_first(true);
  publish_q();
  if (early) {
    // The draft tile's rows into the staging area (V rows that are not
    // tokens zeroed by a mask), then the length.  No vector load is issued
    // here: the waits after this block are then exactly the other path's
    // (issuing the second tile here made that path's first K wait also
    // cover most of its V).
    rowok = rows_of(0, cur);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const unsigned keep = 0u - ((rowok >> s) & 1u);
      *reinterpret_cast<uint4*>(ks + (s * RPI + lrow) * KP + lcol) = kreg[s];
      *reinterpret_cast<uint4*>(vs + (s * RPI + lrow) * VP + lcol) =
          make_uint4(vreg[s].x & keep, vreg[s].y & keep, vreg[s].z & keep, vreg[s].w & keep);
    }
    len_raw = P.lengths[b];
  }
  set_lengths();
  rowok = rows_of(0, cur);
  if constexpr (QL) {
    __syncthreads();  // every wave's Q fragments are in s_q
  } else {
#pragma unroll
    for (int j = 0; j < KS; ++j) qreg[j] = qown[j];
  }
  if (nmine > 0 && !early) {
    int nxt[2] = {-1, -1};
    if (1 < nmine) ids_of(1, nxt);
    process(0, okbits_of(0, cur, false), nxt, std::true_type{});
    cur[0] = nxt[0];
    cur[1] = nxt[1];
  } else {
    // No tile yet, or an early wave's staged first tile, which the loop
    // below takes with the later tiles' code from acc = 0, m = -inf, l = 0:
    // the rescale then multiplies zeros by 0, and the result is the
    // first-tile code's bit for bit.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 16; ++j) acc[dt][j] = 0.f;
  }
  // The loads run one tile ahead of the MFMAs: while tile idx is processed,
  // tile idx+1's rows are loading.
  for (int idx = early ? 0 : 1; idx < nmine; ++idx) {
    int nxt[2] = {-1, -1};
    if (idx + 1 < nmine) ids_of(idx + 1, nxt);
    process(idx, okbits_of(idx, cur, tbeg + ln + LN * idx < ntd), nxt, std::false_type{},
            early && idx == 0);
    cur[0] = nxt[0];
    cur[1] = nxt[1];
  }
  l += shfl_xor_f(l, 32);  // both lane halves share m

  // ---- merge each request's LN waves through LDS in one step ----
  // Every wave stores its state in its own staging area as soon as its
  // tiles are done: no other wave uses that area, so the stores need no
  // barrier and overlap the waves still computing.  After one barrier each
  // thread combines the LN states of its request's share of the tile (row
  // mrow, DPT dims) and writes it.
  constexpr int XP = D + 4;      // padded rows: a float4 access spreads over banks
  constexpr int XW = STAGE / 2;  // floats in a wave's staging area
  static_assert(32 * XP + 64 <= XW, "a wave's state fits its staging area");
  // Wave w's state: [32 rows][XP] accumulators, then (max, sum) per row.
  auto xw = [&](int w) { return reinterpret_cast<float*>(s_stage) + (size_t)w * XW; };
  {
    float* dst = xw(wave) + (size_t)lr * XP;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int jq = 0; jq < 4; ++jq)
        *reinterpret_cast<float4*>(dst + 32 * dt + 8 * jq + 4 * g) =
            make_float4(acc[dt][4 * jq], acc[dt][4 * jq + 1], acc[dt][4 * jq + 2],
                        acc[dt][4 * jq + 3]);
    if (g == 0) *reinterpret_cast<float2*>(xw(wave) + 32 * XP + 2 * lr) = make_float2(m, l);
  }
  __syncthreads();
  constexpr int TPR = 2 * LN;   // threads per row
  constexpr int DPT = D / TPR;  // dims per thread
  static_assert(DPT % 4 == 0, "float4 steps");
  const int t = threadIdx.x % (64 * LN);  // the request's waves hold its rows
  const int mrow = t / TPR;
  const int md0 = (t % TPR) * DPT;
  const int rr = rt * 32 + mrow;
  if (!present || rr >= P.rows) return;
  const int w0 = rq * LN;
  float mw[LN], mm = kNegInf;
#pragma unroll
  for (int w = 0; w < LN; ++w) {
    mw[w] = xw(w0 + w)[32 * XP + 2 * mrow];
    mm = __builtin_fmaxf(mm, mw[w]);
  }
  const float ms = safe_max(mm);  // all waves empty: every weight is 0
  float ll = 0.f, o[DPT];
#pragma unroll
  for (int j = 0; j < DPT; ++j) o[j] = 0.f;
#pragma unroll
  for (int w = 0; w < LN; ++w) {
    const float wt = fast_exp2(mw[w] - ms);  // 0 for a wave without tiles
    ll += wt * xw(w0 + w)[32 * XP + 2 * mrow + 1];
    const float* src = xw(w0 + w) + (size_t)mrow * XP + md0;
#pragma unroll
    for (int j = 0; j < DPT; j += 4) {
      const float4 v4 = *reinterpret_cast<const float4*>(src + j);
      o[j] += wt * v4.x;
      o[j + 1] += wt * v4.y;
      o[j + 2] += wt * v4.z;
      o[j + 3] += wt * v4.w;
    }
  }
  const int rrn = div_by(rr, P.group, P.group_mul);
  const size_t orow =
      ((size_t)b * P.nodes + rrn) * P.hq + kvh * P.group + (rr - rrn * P.group);
  if (P.parts == 1) {
    const float inv = 1.f / ll;  // every row sees its own node: ll > 0
    float* dst = P.out + orow * D + md0;
#pragma unroll
    for (int j = 0; j < DPT; j += 4)
      *reinterpret_cast<float4*>(dst + j) =
          make_float4(o[j] * inv, o[j + 1] * inv, o[j + 2] * inv, o[j + 3] * inv);
  } else if (tbeg < ntot) {
    const size_t slot = orow * P.parts + part;
    float* dst = P.part_acc + slot * D + md0;
#pragma unroll
    for (int j = 0; j < DPT; j += 4)
      *reinterpret_cast<float4*>(dst + j) = make_float4(o[j], o[j + 1], o[j + 2], o[j + 3]);
    if (md0 == 0) *reinterpret_cast<float2*>(P.part_ml + 2 * slot) = make_float2(mm, ll);
  }
}

// Combines tree_split_kernel's partials: one wave per output row (b, node,
// h); the parts that held tiles, [0, nparts) with nparts from the request's
// length, wrote slots (row, part).  Lane p holds slot p's (max, sum); the
// weights are formed once and every lane accumulates its dims from the
// slots.  The (max, sum) loads and the first 8 * NB slots' accumulators go
// out together with the length, in one memory round (NB = ceil(parts / 8),
// at most 4); slots past nparts are masked afterwards (their contents are
// whatever the workspace held).  Rows of more than 8 * NB parts load the
// rest eight slots at a time.
template <int D, int NB>
__global__ __launch_bounds__(256) void merge_split_kernel(TreeParams P) {
  pin_params(P);
  constexpr int PER = D / 64;
  constexpr int NS = 8 * NB;  // slots loaded in the first round
  const int lane = threadIdx.x & 63;
  const size_t row = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // (b*N+node)*Hq+h
  if (row >= (size_t)P.batch * P.nodes * P.hq) return;
  const int b = row / ((size_t)P.nodes * P.hq);
  const int lraw = P.lengths[b];
  const size_t base = row * P.parts;  // P.parts <= 64
  auto load_slot = [&](int sidx, float (&v)[PER]) {
    const float* src = P.part_acc + (base + sidx) * D + lane;
#pragma unroll
    for (int j = 0; j < PER; ++j) v[j] = src[64 * j];
  };
  const float2 ml0 = *reinterpret_cast<const float2*>(P.part_ml + 2 * (base + min(lane, P.parts - 1)));
  float v[NS][PER];
#pragma unroll
  for (int u = 0; u < NS; ++u) load_slot(min(u, P.parts - 1), v[u]);
  // Nothing that waits for the length moves above the last slot load.
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < PER; ++j)
#pragma unroll
    for (int u = 0; u < NS; ++u) asm volatile("" ::"v"(v[u][j]));
  const int len = max(0, min(lraw, P.max_pages * BC_PAGE_SIZE));
  const int ntot = (len + kTile - 1) / kTile + (P.nodes + kTile - 1) / kTile;
  const int nparts = (ntot + P.tiles_per_part - 1) / P.tiles_per_part;  // >= 1
  const bool written = lane < nparts;
  const float mp = written ? ml0.x : kNegInf;
  const float lp = written ? ml0.y : 0.f;
  const float mm = wave_max(mp);
  const float w = fast_exp2(mp - mm);  // every row sees its own node: mm finite
  const float lsum = wave_sum(w * lp);
  auto weight = [&](int i) {
    return __builtin_bit_cast(float,
                              __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), i));
  };
  float a[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) a[j] = 0.f;
#pragma unroll
  for (int u = 0; u < NS; ++u) {
    if (u < nparts) {  // uniform
      const float wi = weight(u);
#pragma unroll
      for (int j = 0; j < PER; ++j) a[j] += wi * v[u][j];
    }
  }
  for (int i0 = NS; i0 < nparts; i0 += 8) {
    float x[8][PER];
#pragma unroll
    for (int u = 0; u < 8; ++u) load_slot(min(i0 + u, nparts - 1), x[u]);
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (i0 + u < nparts) {  // uniform
        const float wi = weight(i0 + u);
#pragma unroll
        for (int j = 0; j < PER; ++j) a[j] += wi * x[u][j];
      }
    }
  }
  const float inv = 1.f / lsum;
#pragma unroll
  for (int j = 0; j < PER; ++j) P.out[row * D + lane + 64 * j] = a[j] * inv;
}

template <int D>
void launch_merge_split(const TreeParams& P, dim3 grid, hipStream_t st) {
  if (P.parts <= 8) merge_split_kernel<D, 1><<<grid, 256, 0, st>>>(P);
  else if (P.parts <= 16) merge_split_kernel<D, 2><<<grid, 256, 0, st>>>(P);
  else if (P.parts <= 24) merge_split_kernel<D, 3><<<grid, 256, 0, st>>>(P);
  else merge_split_kernel<D, 4><<<grid, 256, 0, st>>>(P);
}

// Row-sharing variant for trees of four or more row tiles per (request, KV
// head), where tree_kernel would read the prefix once per row tile: the four
// waves take four row tiles and walk the same 32-token tiles, which the
// workgroup loads once (two 16-byte chunks of K and of V per thread) into a
// double-buffered LDS tile, one barrier per tile.  Each wave reads K back in
// the A-operand layout and V through transpose reads, and owns its rows to
// the end: no merge between waves.  Masks, softmax and the P.V product are
// those of tree_kernel.
template <int D, bool VEC>
__global__ __launch_bounds__(kThreads, 2) void tree_rows_kernel(TreeParams P) {
  // No pin_params here: this kernel's loop runs tens to hundreds of us, and
  // holding every argument in registers from the start measured 0.4-2%
  // slower on it (8 x 2048 x 256 nodes: 161.9 -> 164.0 us; 32 x 512 x 64:
  // 48.3 -> 49.3 us) against about 0.5 us saved at the start.
  constexpr int KS = D / 16;
  constexpr int DT = D / 32;
  constexpr int VP = v_pitch<D>();
  constexpr int KP = D + 8;            // halves per staged K row
  constexpr int CPR = D / 8;           // 16-byte chunks per token row
  constexpr int CPT = kTile * CPR / kThreads;  // chunks per thread, K and V each
  static_assert(CPT * kThreads == kTile * CPR, "tile chunks split evenly");
  constexpr int BUF = kTile * (KP + VP);       // halves per staged tile

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 5;
  const int lr = lane & 31;

  const int rgroups = (P.row_tiles + kWaves - 1) / kWaves;
  const int zdim = P.hkv * rgroups;
  const int z = blockIdx.x % zdim;
  const int b = blockIdx.x / zdim;
  const int kvh = z / rgroups;
  const int rt = (z % rgroups) * kWaves + wave;  // row tile; idle when >= row_tiles

  const int len = max(0, min(P.lengths[b], P.max_pages * BC_PAGE_SIZE));
  const int ntile_p = (len + kTile - 1) / kTile;
  const int ntile = ntile_p + (P.nodes + kTile - 1) / kTile;

  const int r = rt * 32 + lr;
  const bool rvalid = rt < P.row_tiles && r < P.rows;
  const int node = rvalid ? r / P.group : 0;
  const int h = kvh * P.group + (rvalid ? r % P.group : 0);

  __shared__ int s_parent[BC_MAX_TREE_NODES];
  __shared__ __attribute__((aligned(16))) _Float16 s_kv[2 * BUF];
  __shared__ bool s_pok[2][2];

  // Q^T B operand of this wave's row tile; parent entries (one per thread).
  uint4 qB[KS];
  {
    const uint16_t* qp = P.dq + (((size_t)b * P.nodes + node) * P.hq + h) * D + 8 * g;
#pragma unroll
    for (int s = 0; s < KS; ++s) qB[s] = rvalid ? load8<VEC>(qp + 16 * s) : make_uint4(0, 0, 0, 0);
  }
  static_assert(BC_MAX_TREE_NODES <= kThreads, "one parent entry per thread");
  const bool has_parent = (int)threadIdx.x < P.nodes;
  const int par = P.parent[(size_t)b * P.nodes + min((int)threadIdx.x, P.nodes - 1)];

  const size_t tok_stride = (size_t)P.hkv * D;
  // Tile i's chunk c of this thread: token row c / CPR, dims 8 * (c % CPR).
  // Every address stays inside its tensor: rows of invalid pages read page
  // 0, draft rows past the node count read the last node; their V is staged
  // as zeros and their scores are masked.
  uint4 kreg[2][CPT], vreg[2][CPT];
  bool vok[2][CPT];
  int ph[2][2] = {{-1, -1}, {-1, -1}};
  auto page_ids = [&](int i, int (&pg)[2]) {
#pragma unroll
    for (int q = 0; q < 2; ++q) {
      const int pi = i * (kTile / BC_PAGE_SIZE) + q;
      pg[q] = i < ntile_p && pi < P.max_pages ? P.pages[(size_t)b * P.max_pages + pi] : -1;
    }
  };
  auto load_tile = [&](int i, int set) {
    const int (&pg)[2] = ph[set];
    const bool is_draft = i >= ntile_p;
    const int tbase = (is_draft ? i - ntile_p : i) * kTile;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int chunk = (int)threadIdx.x + kThreads * c;
      const int row = chunk / CPR, col = 8 * (chunk % CPR);
      size_t off;
      bool ok;
      if (!is_draft) {
        const int pgq = pg[row / BC_PAGE_SIZE];
        const bool pok = pgq >= 0 && pgq < P.phys_pages;
        const int t = tbase + row;
        ok = pok && t < len;
        off = (pok ? ((size_t)pgq * BC_PAGE_SIZE + row % BC_PAGE_SIZE) * tok_stride : 0) +
              (size_t)kvh * D + col;
        kreg[set][c] = load8<VEC>(P.k + off);
        vreg[set][c] = load8<VEC>(P.v + off);
      } else {
        const int dn = tbase + row;
        ok = dn < P.nodes;
        off = (((size_t)b * P.nodes + min(dn, P.nodes - 1)) * P.hkv + kvh) * D + col;
        kreg[set][c] = load8<VEC>(P.dk + off);
        vreg[set][c] = load8<VEC>(P.dv + off);
      }
      vok[set][c] = ok;
    }
  };
  auto store_tile = [&](int i, int set) {
    const int buf = i & 1;
    const int (&pg)[2] = ph[set];
    _Float16* sk = s_kv + buf * BUF;
    _Float16* sv = sk + kTile * KP;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
      const int chunk = (int)threadIdx.x + kThreads * c;
      const int row = chunk / CPR, col = 8 * (chunk % CPR);
      *reinterpret_cast<uint4*>(sk + row * KP + col) = kreg[set][c];
      *reinterpret_cast<uint4*>(sv + row * VP + col) =
          vok[set][c] ? vreg[set][c] : make_uint4(0, 0, 0, 0);
    }
    if (threadIdx.x < 2) {
      const int pgq = pg[threadIdx.x];
      s_pok[buf][threadIdx.x] = i >= ntile_p || (pgq >= 0 && pgq < P.phys_pages);
    }
  };

  f32x16 acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[dt][j] = 0.f;
  float m = kNegInf, l = 0.f;
  // Transpose-read address of this lane in a staged V tile.
  const int trG = lane >> 4, trj = lane & 15;
  const int vtr_off = (4 * (trG >> 1) + (trj >> 2)) * VP + 16 * (trG & 1) + 4 * (trj & 3);

  auto compute = [&](int i, int buf) {
    const _Float16* sk = s_kv + buf * BUF;
    const _Float16* sv = sk + kTile * KP;
    const bool is_draft = i >= ntile_p;
    const int tbase = (is_draft ? i - ntile_p : i) * kTile;
    uint32_t okbits;
    if (!is_draft) {
      const int hi = min(max(len - tbase, 0), kTile);
      okbits = (hi >= kTile ? ~0u : (1u << hi) - 1u) &
               ((s_pok[buf][0] ? 0x0000ffffu : 0u) | (s_pok[buf][1] ? 0xffff0000u : 0u));
    } else {
      okbits = 0;
      int cur = node;
      for (int steps = 0; steps < P.nodes && cur >= 0 && cur < P.nodes; ++steps) {
        if (cur >= tbase && cur < tbase + kTile) okbits |= 1u << (cur - tbase);
        cur = s_parent[cur];
      }
    }
    // ---- S^T = K Q^T, K from the staged tile in the A-operand layout ----
    f32x16 sc;
#pragma unroll
    for (int j = 0; j < 16; ++j) sc[j] = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const uint4 ka = *reinterpret_cast<const uint4*>(sk + lr * KP + 16 * s + 8 * g);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_f16(as_f16x8(ka), as_f16x8(qB[s]), sc, 0, 0, 0);
    }
    // ---- mask and online softmax (column lr = query row) ----
    // Scores stay unscaled: the scale enters the running max once and the
    // exp2 argument as an FMA; fully valid tiles skip the mask.
    float svv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) svv[j] = sc[j];
    if (__builtin_amdgcn_ballot_w64(okbits != ~0u)) {
      const uint32_t ob = okbits >> (4 * g);
#pragma unroll
      for (int j = 0; j < 16; ++j)
        svv[j] = (ob >> (8 * (j >> 2) + (j & 3))) & 1u ? svv[j] : kNegInf;
    }
    float tmax = kNegInf;
#pragma unroll
    for (int j = 0; j < 16; ++j) tmax = __builtin_fmaxf(tmax, svv[j]);
    tmax = __builtin_fmaxf(tmax, shfl_xor_f(tmax, 32)) * P.scale_log2;
    const float mnew = __builtin_fmaxf(m, tmax);
    if (__builtin_amdgcn_ballot_w64(mnew > m + kRescaleSlack)) {
      const float alpha = fast_exp2(m - safe_max(mnew));
      l *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[dt][j] *= alpha;
      m = mnew;
    }
    const float mb = safe_max(m);
    f16x8 pb[2], pl[2];
    float pr[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      pr[j] = fast_exp2(__builtin_fmaf(svv[j], P.scale_log2, -mb));
      l += pr[j];
    }
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      uint32_t wh[4], wl[4];
#pragma unroll
      for (int q = 0; q < 4; ++q)
        split_hi_lo(pr[8 * hh + 2 * q], pr[8 * hh + 2 * q + 1], wh[q], wl[q]);
      pb[hh] = __builtin_bit_cast(f16x8, u32x4{wh[0], wh[1], wh[2], wh[3]});
      pl[hh] = __builtin_bit_cast(f16x8, u32x4{wl[0], wl[1], wl[2], wl[3]});
    }
    // ---- O^T += V^T P^T from the staged tile ----
    const _Float16* vtr = sv + vtr_off;
    f16x8 av[DT][2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const f16x4 lo = lds_read_tr(vtr + (16 * st) * VP + 32 * dt);
        const f16x4 hi = lds_read_tr(vtr + (16 * st + 8) * VP + 32 * dt);
        av[dt][st] = f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pb[st], acc[dt], 0, 0, 0);
#pragma unroll
    for (int st = 0; st < 2; ++st)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[dt][st], pl[st], acc[dt], 0, 0, 0);
  };

  // Loads run two tiles ahead in two register sets (set = tile & 1); LDS
  // holds two staged tiles (buffer = tile & 1).  Tiles 0 and 1 are loaded
  // and tile 0 staged before the first barrier, together with the parent
  // array.  Step i loads tile i + 2, computes tile i and stages tile i + 1,
  // then the barrier publishes tile i + 1 and frees tile i's buffer.
  if (ntile > 0) {
    page_ids(0, ph[0]);
    load_tile(0, 0);
  }
  if (ntile > 1) {
    page_ids(1, ph[1]);
    load_tile(1, 1);
  }
  if (ntile > 0) store_tile(0, 0);
  if (has_parent) s_parent[threadIdx.x] = par;
  __syncthreads();
  auto step = [&](int i, int set) {  // set = i & 1, a compile-time constant
    if (i >= ntile) return;
    if (i + 2 < ntile) {
      page_ids(i + 2, ph[set]);
      load_tile(i + 2, set);
    }
    if (rt < P.row_tiles) compute(i, set);
    if (i + 1 < ntile) store_tile(i + 1, set ^ 1);
    __syncthreads();
  };
  for (int i = 0; i < ntile; i += 2) {
    step(i, 0);
    step(i + 1, 1);
  }
  if (!rvalid) return;
  l += shfl_xor_f(l, 32);

  // ---- write: lane holds O^T[32dt + 8jq + 4g + e][row r] ----
  float* dst = P.out + (((size_t)b * P.nodes + node) * P.hq + h) * D;
  const float inv = 1.f / l;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq)
      store4f<VEC>(dst + 32 * dt + 8 * jq + 4 * g, acc[dt][4 * jq] * inv,
                   acc[dt][4 * jq + 1] * inv, acc[dt][4 * jq + 2] * inv,
                   acc[dt][4 * jq + 3] * inv);
}

// The reference's rules (src/tree_attention.cu:94-99): physical_pages is not
// among them, and a value below 1 means the pool size is not given.
bool tree_args_ok(const bc_shape& s, const bc_tree_inputs& in, int nodes) {
  return s.batch >= 1 && s.query_heads >= 1 && s.kv_heads >= 1 &&
         s.query_heads % s.kv_heads == 0 && (s.dim == 64 || s.dim == 128) &&
         s.max_pages >= 1 && nodes >= 1 && nodes <= BC_MAX_TREE_NODES && in.prefix.k &&
         in.prefix.v && in.prefix.pages && in.prefix.lengths && in.draft_q && in.draft_k &&
         in.draft_v && in.parent && in.output;
}

// With the pool size given, ids outside [0, physical_pages) are masked and
// every padding load may read page 0.  Without it (physical_pages < 1, as an
// empty pool gives), the page-table entries inside a length are trusted as in
// the reference, and only tree_kernel runs: it reads pages for tokens inside
// the length only and points every other row at the draft tensors.
bool pool_known(const bc_shape& s) { return s.physical_pages >= 1; }

bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15) == 0;
}

TreeParams make_params(const bc_shape& s, const bc_tree_inputs& in, int nodes) {
  TreeParams P{};
  P.k = in.prefix.k;
  P.v = in.prefix.v;
  P.pages = in.prefix.pages;
  P.lengths = in.prefix.lengths;
  P.dq = in.draft_q;
  P.dk = in.draft_k;
  P.dv = in.draft_v;
  P.parent = in.parent;
  P.out = in.output;
  P.batch = s.batch;
  P.nodes = nodes;
  P.hq = s.query_heads;
  P.hkv = s.kv_heads;
  P.group = s.query_heads / s.kv_heads;
  P.max_pages = s.max_pages;
  // physical_pages is not part of the reference tree contract
  // (bindings/torch_ops.cpp:54 passes prefix_k.size(0)); below 1 the ids
  // are not range-checked (tree_kernel only, see pool_known).
  P.phys_pages = pool_known(s) ? s.physical_pages : 0x7fffffff;
  P.rows = nodes * P.group;
  P.row_tiles = (P.rows + 31) / 32;
  P.scale_log2 = (float)(1.4426950408889634 / __builtin_sqrt((double)s.dim));
  // Multiply-high division needs n * d < 2^32 for every n it divides: row
  // indices stay below 32 * row_tiles, (KV head, row tile) indices below
  // hkv * row_tiles.
  const unsigned long long lim = 1ull << 32;
  if ((unsigned long long)P.row_tiles * 32 * P.group < lim)
    P.group_mul = (lim + P.group - 1) / P.group;
  if ((unsigned long long)P.hkv * P.row_tiles * P.row_tiles < lim)
    P.rt_mul = (lim + P.row_tiles - 1) / P.row_tiles;
  return P;
}

// tree_rows_kernel (one K/V tile shared by four row tiles) pays once its
// row groups fill the CUs: the split kernel would then run several rounds
// of workgroups that each read the prefix for one row tile (8 requests x
// 2048 tokens x 256 nodes: 153 against 206 us; 32 x 512 x 64 nodes: 48
// against 78 us).  With fewer row groups the split kernel wins (8 x 2048 x
// 64 nodes: 50 against 59 us; 4 x 2048 x 128: 52 against 58 us), and with
// fewer than four row tiles the rows kernel's serial walk lost outright
// (one request, 32 nodes: 101 against 36 us).
bool rows_kernel_for(int batch, int hkv, int row_tiles, int cus) {
  return row_tiles >= kWaves &&
         (long long)batch * hkv * ((row_tiles + kWaves - 1) / kWaves) >= cus;
}

// Workgroups per (request, KV head).
int row_units(int row_tiles, bool rows_kernel) {
  return rows_kernel ? (row_tiles + kWaves - 1) / kWaves : row_tiles;
}

template <int D, bool VEC>
void launch_tree_kernel(const TreeParams& P, bool rows_kernel, dim3 grid, hipStream_t st) {
  if (rows_kernel)
    tree_rows_kernel<D, VEC><<<grid, kThreads, 0, st>>>(P);
  else  // unaligned tensors or an unknown pool size: the split kernel takes the rest
    tree_kernel<D, false><<<grid, kThreads, 0, st>>>(P);
}

// vec: every FP16 tensor and the output are 16-byte aligned (16-byte loads
// and stores); otherwise the kernels move single halves and floats.
// known_pool: false sends every shape to tree_kernel (see pool_known).
hipError_t launch_tree(const TreeParams& P, int dim, bool vec, bool known_pool,
                       hipStream_t st) {
  const bool rows_kernel =
      known_pool && rows_kernel_for(P.batch, P.hkv, P.row_tiles, bch::device_cus());
  const dim3 grid((unsigned)((size_t)P.batch * P.hkv * row_units(P.row_tiles, rows_kernel)));
  if (dim == 64) {
    if (vec) launch_tree_kernel<64, true>(P, rows_kernel, grid, st);
    else launch_tree_kernel<64, false>(P, rows_kernel, grid, st);
  } else {
    if (vec) launch_tree_kernel<128, true>(P, rows_kernel, grid, st);
    else launch_tree_kernel<128, false>(P, rows_kernel, grid, st);
  }
  return hipGetLastError();
}

bool tree_ptrs_aligned(const bc_tree_inputs& in) {
  return aligned16(in.prefix.k) && aligned16(in.prefix.v) &&
         aligned16(in.draft_q) && aligned16(in.draft_k) &&
         aligned16(in.draft_v) && aligned16(in.output);
}

// ---- tree_split_kernel: plan, workspace and launch ----

struct SplitPlan {
  int parts;  // workgroups per (request group, KV head, row tile), <= 64
  int tiles;  // 32-token tiles per workgroup and request (draft then prefix tiles)
  int waves;  // waves per workgroup: 4 or 8
  int rq = 1;  // requests per workgroup (waves / rq per request)
};

// A single pass of more (request, KV head, row tile) units than CUs runs
// its eight-wave workgroups (one per CU) in rounds.  Two requests per
// workgroup, four waves each on the same tiles, halve the workgroups and
// double each wave's tiles, so they pay where they at least halve the
// rounds; requests that share pages then also share them in the CU's L1.
// Measured against one request per workgroup (32 / 8 heads, D = 128, 7
// nodes, shared prefix): 33 x 2048 tokens 48.9 -> 45.3 us, 40 x 1024 31.6
// -> 28.2, 64 x 1024 32.4 -> 30.1, 128 x 512 46.3 -> 39.2; 96 x 512 (three
// rounds against two) 35.5 -> 37.9 and 32 x 2048 (one round) 27.9 -> 45.7,
// so neither of those pairs.
SplitPlan pair_requests(int batch, long long units, SplitPlan p, int cus) {
  if (p.parts != 1 || p.waves != 8 || batch < 2) return p;
  const long long per_request = units / batch;  // KV heads x row tiles
  const long long rounds1 = (units + cus - 1) / cus;
  const long long rounds2 = ((batch + 1) / 2 * per_request + cus - 1) / cus;
  if (2 * rounds2 <= rounds1) p.rq = 2;
  return p;
}

// Parts per unit and tiles per part for `cus` compute units, sized from the
// page table's capacity (lengths stay on the device).  A CU holds one
// eight-wave or two four-wave workgroups (LDS), so both shapes offer eight
// wave slots per CU: eight-wave workgroups take about cus/units parts, four-
// wave ones about 2*cus/units.  The plan with more waves that have a tile
// wins (12 requests x 2048 tokens, 96 units: four waves x 5 parts 20.2 us
// against eight waves x 2 parts 20.8 and four waves x 2 parts 24.5); at about
// equal counts, the one spread over more CUs (one request x 2048 tokens:
// four waves x 17 parts, 10.4 against 11.8 us), else eight waves, which
// merge more tiles in LDS (8 and 16 requests), or run single-pass (24 and 32
// requests: one part, 28.6 against 31.7 us with two); see pair_requests for
// single passes of more units than CUs.
SplitPlan split_plan(const bc_shape& s, int nodes, int cus) {
  const int group = s.query_heads / s.kv_heads;
  const int row_tiles = (nodes * group + 31) / 32;
  const long long units = (long long)s.batch * s.kv_heads * row_tiles;
  const int max_tiles =
      (s.max_pages * BC_PAGE_SIZE + kTile - 1) / kTile + (nodes + kTile - 1) / kTile;
  auto plan_for = [&](int waves, long long want) {
    if (want > 64) want = 64;
    SplitPlan p{1, max_tiles, waves};
    if (want < 2) return p;
    int tiles = (int)((max_tiles + want - 1) / want);
    if (tiles < waves) tiles = waves;
    const int parts = (max_tiles + tiles - 1) / tiles;
    return parts < 2 ? p : SplitPlan{parts, tiles, waves};
  };
  const long long u = units > 0 ? units : 1;
  // A single pass whose eight waves take two tiles or fewer each beats a
  // split, which adds the merge launch (one request over 256 tokens: 8.2
  // against 9.6 us, over 384: 8.4 against 9.3 us; 2 x 256: 8.5 against
  // 9.6 us; 16 x 256: 10.3 against 13.2 us).  Up to five tiles per wave it
  // still wins once its units fill (tiles per wave - 1) eighths of the CUs
  // (12 x 512 tokens: 9.5 against 12.1 us; 16 x 512: 9.4 against 12.1 us;
  // 12 x 768: 11.2 against 13.7 us; 8 x 1024 with 16 nodes: 13.3 against
  // 15.0 us); below that the split wins (one request over 512 tokens: 9.1
  // against 9.7 us).
  const int rounds = (max_tiles + 7) / 8;  // tiles per wave in a single pass
  if (max_tiles <= 2 * 8 || (rounds <= 5 && 8 * u >= (long long)cus * (rounds - 1)))
    return pair_requests(s.batch, u, SplitPlan{1, max_tiles, 8}, cus);
  const SplitPlan eight = plan_for(8, cus / u);
  const SplitPlan four = plan_for(4, 2LL * cus / u);
  // Waves with at least one tile, and CUs with a workgroup.
  auto busy = [&](const SplitPlan& p) {
    return u * std::min<long long>((long long)p.parts * p.waves, max_tiles);
  };
  auto spread = [&](const SplitPlan& p) { return std::min<long long>(u * p.parts, cus); };
  const long long b8 = busy(eight), b4 = busy(four);
  if (10 * b4 > 11 * b8) return four;
  if (eight.parts > 1 && 10 * b4 >= 9 * b8 && spread(four) > spread(eight)) return four;
  return pair_requests(s.batch, u, eight, cus);
}

// Workspace of tree_split_kernel: P.parts (acc; max, sum) slots per output row.
size_t split_workspace(const bc_shape& s, int nodes, const SplitPlan& plan, size_t* acc_bytes) {
  if (plan.parts < 2) return 0;
  const size_t slots = (size_t)s.batch * nodes * s.query_heads * plan.parts;
  *acc_bytes = (slots * s.dim * sizeof(float) + 255) & ~(size_t)255;
  return *acc_bytes + slots * 2 * sizeof(float);
}

template <int D>
void launch_split_kernel(const TreeParams& P, const SplitPlan& plan, dim3 grid,
                         hipStream_t st) {
  if (plan.waves == 4)
    tree_split_kernel<D, 4, 1><<<grid, 256, 0, st>>>(P);
  else if (plan.rq == 2)
    tree_split_kernel<D, 8, 2><<<grid, 512, 0, st>>>(P);
  else
    tree_split_kernel<D, 8, 1><<<grid, 512, 0, st>>>(P);
}

hipError_t launch_split(TreeParams& P, int dim, const SplitPlan& plan, void* workspace,
                        size_t acc_bytes, hipStream_t st) {
  P.parts = plan.parts;
  P.tiles_per_part = plan.tiles;
  if (plan.parts > 1) {
    P.part_acc = static_cast<float*>(workspace);
    P.part_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + acc_bytes);
  }
  const size_t groups = ((size_t)P.batch + plan.rq - 1) / plan.rq;
  P.grid3d = groups <= 65535;
  const dim3 grid = P.grid3d
      ? dim3((unsigned)(P.hkv * P.row_tiles), (unsigned)groups, (unsigned)plan.parts)
      : dim3((unsigned)((size_t)plan.parts * groups * P.hkv * P.row_tiles));
  if (dim == 64) launch_split_kernel<64>(P, plan, grid, st);
  else launch_split_kernel<128>(P, plan, grid, st);
  hipError_t err = hipGetLastError();
  if (err != hipSuccess || plan.parts < 2) return err;
  const size_t rows = (size_t)P.batch * P.nodes * P.hq;
  const dim3 mgrid((unsigned)((rows + 3) / 4));
  if (dim == 64) launch_merge_split<64>(P, mgrid, st);
  else launch_merge_split<128>(P, mgrid, st);
  return hipGetLastError();
}

}  // namespace

extern "C" int bc_tree_verify(bc_shape s, bc_tree_inputs in, int nodes,
                              bc_stream_t stream) {
  if (!tree_args_ok(s, in, nodes)) return BC_ERROR_INVALID_VALUE;
  TreeParams P = make_params(s, in, nodes);
  const hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const bool vec = tree_ptrs_aligned(in);
  const int cus = bch::device_cus();
  const bool known = pool_known(s);
  if (vec && known && !rows_kernel_for(P.batch, P.hkv, P.row_tiles, cus)) {
    // The reference's signature has no workspace: a plan that splits the
    // prefix borrows a slot of the library's scratch pool for the call
    // (none under graph capture or when the slot is too small: the single
    // pass below then runs).
    const SplitPlan plan = split_plan(s, nodes, cus);
    size_t acc = 0;
    const size_t need = split_workspace(s, nodes, plan, &acc);
    if (need > 0) {
      const bch::ScratchLease lease(st, need);
      if (lease.get()) return launch_split(P, s.dim, plan, lease.get(), acc, st);
    }
    const int max_tiles =
        (s.max_pages * BC_PAGE_SIZE + kTile - 1) / kTile + (nodes + kTile - 1) / kTile;
    const long long units = (long long)P.batch * P.hkv * P.row_tiles;
    return launch_split(P, s.dim, pair_requests(P.batch, units, SplitPlan{1, max_tiles, 8}, cus),
                        nullptr, 0, st);
  }
  return launch_tree(P, s.dim, vec, known, st);
}

namespace {

bool tree_shape_ok(const bc_shape& s, int nodes) {
  return s.batch >= 1 && s.query_heads >= 1 && s.kv_heads >= 1 &&
         s.query_heads % s.kv_heads == 0 && (s.dim == 64 || s.dim == 128) &&
         s.max_pages >= 1 && nodes >= 1 && nodes <= BC_MAX_TREE_NODES;
}

bool split_for(const bc_shape& s, int nodes) {
  const int row_tiles = (nodes * (s.query_heads / s.kv_heads) + 31) / 32;
  return !rows_kernel_for(s.batch, s.kv_heads, row_tiles, bch::device_cus());
}

// tree_rows_kernel, split plans of one part and calls without the pool size
// need no workspace.
size_t ws_size(const bc_shape& s, int nodes) {
  if (!pool_known(s) || !split_for(s, nodes)) return 0;
  size_t a = 0;
  return split_workspace(s, nodes, split_plan(s, nodes, bch::device_cus()), &a);
}

int tree_ws_call(bc_shape s, bc_tree_inputs in, int nodes, void* workspace,
                 size_t workspace_bytes, bc_stream_t stream) {
  if (!tree_args_ok(s, in, nodes)) return BC_ERROR_INVALID_VALUE;
  const bool vec = tree_ptrs_aligned(in);
  // Tensors that are not 16-byte aligned, and calls without the pool size,
  // take the single pass.
  if (!vec || !pool_known(s)) return bc_tree_verify(s, in, nodes, stream);
  if (!split_for(s, nodes)) return bc_tree_verify(s, in, nodes, stream);
  const SplitPlan plan = split_plan(s, nodes, bch::device_cus());
  size_t acc = 0;
  const size_t need = split_workspace(s, nodes, plan, &acc);
  if (!workspace || need == 0 || workspace_bytes < need || !aligned16(workspace))
    return bc_tree_verify(s, in, nodes, stream);
  TreeParams P = make_params(s, in, nodes);
  return launch_split(P, s.dim, plan, workspace, acc, reinterpret_cast<hipStream_t>(stream));
}

}  // namespace

extern "C" size_t bc_tree_verify_workspace_size(bc_shape s, int nodes) {
  if (!tree_shape_ok(s, nodes)) return 0;
  return ws_size(s, nodes);
}

extern "C" int bc_tree_verify_ws(bc_shape s, bc_tree_inputs in, int nodes,
                                 void* workspace, size_t workspace_bytes,
                                 bc_stream_t stream) {
  return tree_ws_call(s, in, nodes, workspace, workspace_bytes, stream);
}
