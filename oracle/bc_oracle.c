/*
 * CPU oracle for the Branchcraft paged-attention hot path.
 * TEST INFRASTRUCTURE ONLY: see bc_oracle.h.  Nothing in the product links
 * or calls this file; tests, smoke() and bench.py's cpu_baseline leg use it
 * as the checker.
 *
 * Pinned by tests/test_oracle.py against: numpy's binary16 conversion (f16
 * helpers), a float64 closed-form softmax(q.K^T*scale).V written
 * independently in numpy (decode, packed, tree), brute-force ancestor sets,
 * the reference's known-answer commit test (tests/test_torch_ops.py:99-114)
 * and the reference driver's commit case (src/main.cu:264-313).
 */
#include "bc_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

float oracle_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  uint32_t x;
  if (e == 0) {
    const float f = ldexpf((float)m, -24);
    return sign ? -f : f;
  }
  if (e == 31)
    x = sign | 0x7f800000u | (m << 13);
  else
    x = sign | ((e + 112u) << 23) | (m << 13);
  float f;
  memcpy(&f, &x, sizeof f);
  return f;
}

uint16_t oracle_f2h(float f) {
  uint32_t x;
  memcpy(&x, &f, sizeof x);
  const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
  const uint32_t ax = x & 0x7fffffffu;
  if (ax >= 0x7f800000u) /* inf / nan (quiet) */
    return sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u);
  if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
    return sign | 0x7c00u;
  if (ax < 0x38800000u) { /* below 2^-14: half subnormal or zero */
    const int e = (int)(ax >> 23);
    const int shift = 126 - e; /* value = sig * 2^-24 / 2^shift */
    if (e == 0 || shift > 24) return sign;
    const uint32_t sig = (ax & 0x7fffffu) | 0x800000u;
    uint32_t n = sig >> shift;
    const uint32_t rem = sig & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (n & 1u))) ++n;
    return sign | (uint16_t)n;
  }
  uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7fffffu) >> 13);
  const uint32_t rem = ax & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return sign | (uint16_t)h;
}

void oracle_f2h_array(const float* in, uint16_t* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_f2h(in[i]);
}

void oracle_h2f_array(const uint16_t* in, float* out, size_t n) {
  for (size_t i = 0; i < n; ++i) out[i] = oracle_h2f(in[i]);
}

static int clamp_len(int len, int max_pages) {
  if (len < 0) return 0;
  return len > max_pages * ORACLE_PAGE ? max_pages * ORACLE_PAGE : len;
}

/* ---- row-parallel driver -------------------------------------------- */

typedef void (*row_fn)(const void* ctx, int row, void* scratch);

typedef struct {
  row_fn fn;
  const void* ctx;
  int rows, threads, id;
  size_t scratch_bytes;
} row_job;

static void* row_worker(void* arg) {
  const row_job* job = (const row_job*)arg;
  void* scratch = job->scratch_bytes ? malloc(job->scratch_bytes) : NULL;
  for (int r = job->id; r < job->rows; r += job->threads) job->fn(job->ctx, r, scratch);
  free(scratch);
  return NULL;
}

static void run_rows(row_fn fn, const void* ctx, int rows, int threads,
                     size_t scratch_bytes) {
  if (threads < 1) threads = 1;
  if (threads > rows) threads = rows > 0 ? rows : 1;
  row_job* jobs = (row_job*)calloc((size_t)threads, sizeof(row_job));
  pthread_t* tids = (pthread_t*)calloc((size_t)threads, sizeof(pthread_t));
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn;
    jobs[t].ctx = ctx;
    jobs[t].rows = rows;
    jobs[t].threads = threads;
    jobs[t].id = t;
    jobs[t].scratch_bytes = scratch_bytes;
  }
  if (threads == 1) {
    row_worker(&jobs[0]);
  } else {
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, row_worker, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
  }
  free(jobs);
  free(tids);
}

/* ---- paged and packed decode ---------------------------------------- */

typedef struct {
  int batch, hq, hkv, dim, max_pages;
  const uint16_t *q, *kbase, *vbase;
  const int32_t *pages, *lengths;
  long long bs, hs, ss;
  double scale;
  int scale_is_div; /* 1: score = dot / sqrt(dim) as src/main.cu:97 */
  float* out;
  uint16_t* out_f16;
} decode_ctx;

static void decode_row(const void* vctx, int row, void* scratch) {
  const decode_ctx* c = (const decode_ctx*)vctx;
  const int b = row / c->hq, h = row % c->hq;
  const int kvh = h / (c->hq / c->hkv);
  const int D = c->dim;
  const uint16_t* q = c->q + (size_t)row * D;
  float* out = c->out + (size_t)row * D;
  const int len = clamp_len(c->lengths[b], c->max_pages);
  float* scores = (float*)scratch;
  double qd[128];
  for (int d = 0; d < D; ++d) {
    qd[d] = (double)oracle_h2f(q[d]);
    out[d] = 0.f;
  }
  float max_score = -INFINITY;
  for (int t = 0; t < len; ++t) {
    const long long phys = c->pages[(size_t)b * c->max_pages + t / ORACLE_PAGE];
    const uint16_t* k = c->kbase + phys * c->bs + kvh * c->hs + (t % ORACLE_PAGE) * c->ss;
    double dot = 0;
    for (int d = 0; d < D; ++d) dot += qd[d] * oracle_h2f(k[d]);
    scores[t] = c->scale_is_div ? (float)(dot / sqrt((double)D)) : (float)(dot * c->scale);
    if (scores[t] > max_score) max_score = scores[t];
  }
  double denom = 0;
  for (int t = 0; t < len; ++t) {
    const double p = exp((double)(scores[t] - max_score));
    denom += p;
    const long long phys = c->pages[(size_t)b * c->max_pages + t / ORACLE_PAGE];
    const uint16_t* v = c->vbase + phys * c->bs + kvh * c->hs + (t % ORACLE_PAGE) * c->ss;
    for (int d = 0; d < D; ++d) out[d] += (float)(p * oracle_h2f(v[d]));
  }
  if (denom != 0)
    for (int d = 0; d < D; ++d) out[d] /= (float)denom;
  if (c->out_f16)
    for (int d = 0; d < D; ++d) c->out_f16[(size_t)row * D + d] = oracle_f2h(out[d]);
}

void oracle_decode(int batch, int hq, int hkv, int dim, int max_pages,
                   const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   const int32_t* pages, const int32_t* lengths, float* out,
                   int threads) {
  decode_ctx c;
  memset(&c, 0, sizeof c);
  c.batch = batch;
  c.hq = hq;
  c.hkv = hkv;
  c.dim = dim;
  c.max_pages = max_pages;
  c.q = q;
  c.kbase = k;
  c.vbase = v;
  c.pages = pages;
  c.lengths = lengths;
  c.bs = (long long)ORACLE_PAGE * hkv * dim;
  c.hs = dim;
  c.ss = (long long)hkv * dim;
  c.scale_is_div = 1;
  c.out = out;
  run_rows(decode_row, &c, batch * hq, threads,
           sizeof(float) * (size_t)max_pages * ORACLE_PAGE + 16);
}

void oracle_packed_decode(int batch, int hq, int hkv, int dim, int max_pages,
                          const uint16_t* q, const uint16_t* cache,
                          const int32_t* pages, const int32_t* lengths,
                          long long bs, long long hs, long long ss,
                          long long kvs, double scale, float* out_f32,
                          uint16_t* out_f16, int threads) {
  decode_ctx c;
  memset(&c, 0, sizeof c);
  c.batch = batch;
  c.hq = hq;
  c.hkv = hkv;
  c.dim = dim;
  c.max_pages = max_pages;
  c.q = q;
  c.kbase = cache;
  c.vbase = cache + kvs;
  c.pages = pages;
  c.lengths = lengths;
  c.bs = bs;
  c.hs = hs;
  c.ss = ss;
  c.scale = scale;
  c.scale_is_div = 0;
  c.out = out_f32;
  c.out_f16 = out_f16;
  run_rows(decode_row, &c, batch * hq, threads,
           sizeof(float) * (size_t)max_pages * ORACLE_PAGE + 16);
}

/* ---- tree verification ---------------------------------------------- */

typedef struct {
  int batch, nodes, hq, hkv, dim, max_pages;
  const uint16_t *k, *v, *dq, *dk, *dv;
  const int32_t *pages, *lengths, *parent;
  float* out;
} tree_ctx;

static void tree_row(const void* vctx, int row, void* scratch) {
  const tree_ctx* c = (const tree_ctx*)vctx;
  const int D = c->dim, N = c->nodes;
  const int h = row % c->hq;
  const int node = (row / c->hq) % N;
  const int b = row / (c->hq * N);
  const int kvh = h / (c->hq / c->hkv);
  const uint16_t* q = c->dq + (size_t)row * D;
  float* out = c->out + (size_t)row * D;
  const int len = clamp_len(c->lengths[b], c->max_pages);
  /* token list: prefix tokens, then the ancestor chain leaf -> root */
  const uint16_t** kp = (const uint16_t**)scratch;
  const uint16_t** vp = kp + len + N;
  double* scores = (double*)(vp + len + N);
  int count = 0;
  for (int t = 0; t < len; ++t) {
    const size_t phys = (size_t)c->pages[(size_t)b * c->max_pages + t / ORACLE_PAGE];
    const size_t off = ((phys * ORACLE_PAGE + t % ORACLE_PAGE) * c->hkv + kvh) * D;
    kp[count] = c->k + off;
    vp[count] = c->v + off;
    ++count;
  }
  /* ancestor chain; a node is visited once (a cyclic parent array ends at
     the first repeat) */
  int cur = node;
  unsigned char* seen = (unsigned char*)(scores + len + N);
  memset(seen, 0, (size_t)N);
  while (cur >= 0 && cur < N && !seen[cur]) {
    seen[cur] = 1;
    const size_t off = (((size_t)b * N + cur) * c->hkv + kvh) * D;
    kp[count] = c->dk + off;
    vp[count] = c->dv + off;
    ++count;
    cur = c->parent[(size_t)b * N + cur];
  }
  double qd[128];
  for (int d = 0; d < D; ++d) {
    qd[d] = (double)oracle_h2f(q[d]);
    out[d] = 0.f;
  }
  double maximum = -INFINITY;
  for (int t = 0; t < count; ++t) {
    double dot = 0;
    for (int d = 0; d < D; ++d) dot += qd[d] * oracle_h2f(kp[t][d]);
    scores[t] = dot / sqrt((double)D);
    if (scores[t] > maximum) maximum = scores[t];
  }
  double denom = 0;
  for (int t = 0; t < count; ++t) {
    const double p = exp(scores[t] - maximum);
    denom += p;
    for (int d = 0; d < D; ++d) out[d] += (float)(p * oracle_h2f(vp[t][d]));
  }
  for (int d = 0; d < D; ++d) out[d] /= (float)denom;
}

void oracle_tree(int batch, int nodes, int hq, int hkv, int dim, int max_pages,
                 const uint16_t* k, const uint16_t* v, const int32_t* pages,
                 const int32_t* lengths, const uint16_t* draft_q,
                 const uint16_t* draft_k, const uint16_t* draft_v,
                 const int32_t* parent, float* out, int threads) {
  tree_ctx c;
  c.batch = batch;
  c.nodes = nodes;
  c.hq = hq;
  c.hkv = hkv;
  c.dim = dim;
  c.max_pages = max_pages;
  c.k = k;
  c.v = v;
  c.dq = draft_q;
  c.dk = draft_k;
  c.dv = draft_v;
  c.pages = pages;
  c.lengths = lengths;
  c.parent = parent;
  c.out = out;
  const size_t tokens = (size_t)max_pages * ORACLE_PAGE + nodes;
  run_rows(tree_row, &c, batch * nodes * hq, threads,
           tokens * (2 * sizeof(void*) + sizeof(double)) + (size_t)nodes + 64);
}

/* ---- bit copies ------------------------------------------------------- */

void oracle_commit(int batch, int nodes, int hkv, int dim, int phys_pages,
                   const uint16_t* draft_k, const uint16_t* draft_v,
                   uint16_t* cache_k, uint16_t* cache_v,
                   const int32_t* path_nodes, const int32_t* dest_pages,
                   const int32_t* dest_slots, int request, int accepted) {
  const size_t elems = (size_t)hkv * dim;
  if (request < 0 || request >= batch) return;
  for (int i = 0; i < accepted; ++i) {
    const int node = path_nodes[i], page = dest_pages[i], slot = dest_slots[i];
    if (node < 0 || node >= nodes || page < 0 || page >= phys_pages || slot < 0 ||
        slot >= ORACLE_PAGE)
      continue;
    const size_t src = ((size_t)request * nodes + node) * elems;
    const size_t dst = ((size_t)page * ORACLE_PAGE + slot) * elems;
    memcpy(cache_k + dst, draft_k + src, elems * sizeof(uint16_t));
    memcpy(cache_v + dst, draft_v + src, elems * sizeof(uint16_t));
  }
}

void oracle_copy_pages(int hkv, int dim, int phys_pages, uint16_t* cache_k,
                       uint16_t* cache_v, const int32_t* src_pages,
                       const int32_t* dst_pages, int count) {
  const size_t page = (size_t)ORACLE_PAGE * hkv * dim;
  for (int i = 0; i < count; ++i) {
    const int s = src_pages[i], d = dst_pages[i];
    if (s < 0 || s >= phys_pages || d < 0 || d >= phys_pages) continue;
    memmove(cache_k + (size_t)d * page, cache_k + (size_t)s * page, page * sizeof(uint16_t));
    memmove(cache_v + (size_t)d * page, cache_v + (size_t)s * page, page * sizeof(uint16_t));
  }
}

/* ---- expanded-prefix baseline ----------------------------------------- */

static int chain(const int32_t* parent_row, int nodes, int node, int* path) {
  int n = 0, cur = node;
  while (cur >= 0 && cur < nodes) {
    int repeat = 0;
    for (int i = 0; i < n; ++i) repeat |= path[i] == cur;
    if (repeat) break;
    path[n++] = cur;
    cur = parent_row[cur];
  }
  /* reverse: root first */
  for (int i = 0; i < n / 2; ++i) {
    const int t = path[i];
    path[i] = path[n - 1 - i];
    path[n - 1 - i] = t;
  }
  return n;
}

void oracle_expand_tree(int batch, int nodes, int hkv, int dim, int max_pages,
                        const uint16_t* k, const uint16_t* v,
                        const int32_t* pages, const int32_t* lengths,
                        const uint16_t* draft_k, const uint16_t* draft_v,
                        const int32_t* parent, int* seq_max_pages,
                        int* total_pages, int32_t* out_lengths,
                        int32_t* out_pages, uint16_t* out_k, uint16_t* out_v) {
  const int seqs = batch * nodes;
  int* path = (int*)malloc(sizeof(int) * (size_t)(nodes > 0 ? nodes : 1));
  int max_len = 0, total = 0;
  for (int s = 0; s < seqs; ++s) {
    const int b = s / nodes, node = s % nodes;
    const int len = clamp_len(lengths[b], max_pages) +
                    chain(parent + (size_t)b * nodes, nodes, node, path);
    if (len > max_len) max_len = len;
    total += (len + ORACLE_PAGE - 1) / ORACLE_PAGE;
  }
  const int smax = (max_len + ORACLE_PAGE - 1) / ORACLE_PAGE;
  if (seq_max_pages) *seq_max_pages = smax;
  if (total_pages) *total_pages = total;
  if (!out_lengths || !out_pages || !out_k || !out_v) {
    free(path);
    return;
  }
  const size_t tok = (size_t)hkv * dim;
  memset(out_k, 0, sizeof(uint16_t) * (size_t)(total + 7) * ORACLE_PAGE * tok);
  memset(out_v, 0, sizeof(uint16_t) * (size_t)(total + 7) * ORACLE_PAGE * tok);
  for (size_t i = 0; i < (size_t)seqs * smax; ++i) out_pages[i] = -1;
  int next_page = 0;
  for (int s = 0; s < seqs; ++s) {
    const int b = s / nodes, node = s % nodes;
    const int plen = clamp_len(lengths[b], max_pages);
    const int depth = chain(parent + (size_t)b * nodes, nodes, node, path);
    const int len = plen + depth;
    out_lengths[s] = len;
    for (int p = 0; p < (len + ORACLE_PAGE - 1) / ORACLE_PAGE; ++p)
      out_pages[(size_t)s * smax + p] = next_page++;
    for (int t = 0; t < len; ++t) {
      const size_t dp = (size_t)out_pages[(size_t)s * smax + t / ORACLE_PAGE];
      const size_t dst = (dp * ORACLE_PAGE + t % ORACLE_PAGE) * tok;
      const uint16_t *ks, *vs;
      if (t < plen) {
        const size_t sp = (size_t)pages[(size_t)b * max_pages + t / ORACLE_PAGE];
        const size_t src = (sp * ORACLE_PAGE + t % ORACLE_PAGE) * tok;
        ks = k + src;
        vs = v + src;
      } else {
        const size_t src = ((size_t)b * nodes + path[t - plen]) * tok;
        ks = draft_k + src;
        vs = draft_v + src;
      }
      memcpy(out_k + dst, ks, tok * sizeof(uint16_t));
      memcpy(out_v + dst, vs, tok * sizeof(uint16_t));
    }
  }
  free(path);
}

float oracle_max_abs_error(const float* a, const float* b, size_t n) {
  float worst = 0.f;
  for (size_t i = 0; i < n; ++i) {
    if (!isfinite(a[i]) || !isfinite(b[i])) return INFINITY;
    const float e = fabsf(a[i] - b[i]);
    if (e > worst) worst = e;
  }
  return worst;
}
