/*
 * CPU oracle for the Branchcraft paged-attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This code is the checker the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg compare against;
 * the product library never calls, links or falls back to it.
 *
 * It restates the reference's CPU oracle (src/main.cu of
 * Haaziq386/branchcraft-cuda) in plain C with the same accumulation order
 * and precision: double dot products, double softmax weights, per-element
 * float accumulation of the weighted values and a final float divide.
 * FP16 values are IEEE binary16 bit patterns (uint16_t).
 */
#ifndef BC_ORACLE_H_
#define BC_ORACLE_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_PAGE 16

/* binary16 <-> binary32, round to nearest even (as __float2half). */
float oracle_h2f(uint16_t h);
uint16_t oracle_f2h(float f);
void oracle_f2h_array(const float* in, uint16_t* out, size_t n);
void oracle_h2f_array(const uint16_t* in, float* out, size_t n);

/* Paged GQA decode, follows src/main.cu:81-113 (cpu_reference).
 * q [B,Hq,D]; k, v [P,16,Hkv,D]; pages [B,max_pages]; lengths [B];
 * out [B,Hq,D] f32 (zeros for empty rows).  Work is split over (b, h) rows
 * on `threads` POSIX threads (1 = the reference's single thread). */
void oracle_decode(int batch, int hq, int hkv, int dim, int max_pages,
                   const uint16_t* q, const uint16_t* k, const uint16_t* v,
                   const int32_t* pages, const int32_t* lengths, float* out,
                   int threads);

/* Packed-cache decode in the same arithmetic.  Token t of row b is at
 * pages[b,t/16]*bs + kvh*hs + (t%16)*ss (K) and + kvs (V); `scale` is the
 * softmax scale.  The reference's packed kernel (src/packed_decode.cu:15-60)
 * has no CPU oracle; its torch test (tests/test_torch_ops.py:77-88) is the
 * same closed form.  out_f32 receives the FP32 result before rounding,
 * out_f16 (may be null) the result rounded to FP16. */
void oracle_packed_decode(int batch, int hq, int hkv, int dim, int max_pages,
                          const uint16_t* q, const uint16_t* cache,
                          const int32_t* pages, const int32_t* lengths,
                          long long bs, long long hs, long long ss,
                          long long kvs, double scale, float* out_f32,
                          uint16_t* out_f16, int threads);

/* Tree verification, follows src/main.cu:204-240 (cpu_tree_reference):
 * every node attends to its request's prefix plus its ancestor chain
 * (itself included), all in double.  draft_q [B,N,Hq,D]; draft_k/v
 * [B,N,Hkv,D]; parent [B,N]; out [B,N,Hq,D] f32.  The parent walk stops at
 * a parent outside [0, N) or at a node it already visited. */
void oracle_tree(int batch, int nodes, int hq, int hkv, int dim, int max_pages,
                 const uint16_t* k, const uint16_t* v, const int32_t* pages,
                 const int32_t* lengths, const uint16_t* draft_q,
                 const uint16_t* draft_k, const uint16_t* draft_v,
                 const int32_t* parent, float* out, int threads);

/* Accepted-path copy, restating src/tree_attention.cu:73-89 with the
 * range checks of the build (out-of-range entries are skipped). */
void oracle_commit(int batch, int nodes, int hkv, int dim, int phys_pages,
                   const uint16_t* draft_k, const uint16_t* draft_v,
                   uint16_t* cache_k, uint16_t* cache_v,
                   const int32_t* path_nodes, const int32_t* dest_pages,
                   const int32_t* dest_slots, int request, int accepted);

/* Whole-page copy (copy-on-write clone), src/main.cu:276-281. */
void oracle_copy_pages(int hkv, int dim, int phys_pages, uint16_t* cache_k,
                       uint16_t* cache_v, const int32_t* src_pages,
                       const int32_t* dst_pages, int count);

/* Expanded-prefix baseline, follows src/main.cu:375-423
 * (make_expanded_fixture): each (request, node) becomes its own paged
 * sequence holding the prefix then the root-to-node path.  Call once with
 * null outputs to get the sizes (*seq_max_pages, *total_pages), then with
 * buffers: lengths [B*N], pages [B*N, seq_max_pages] (-1 padded),
 * k, v [total_pages+7, 16, Hkv, D] (zero-filled spare pages). */
void oracle_expand_tree(int batch, int nodes, int hkv, int dim, int max_pages,
                        const uint16_t* k, const uint16_t* v,
                        const int32_t* pages, const int32_t* lengths,
                        const uint16_t* draft_k, const uint16_t* draft_v,
                        const int32_t* parent, int* seq_max_pages,
                        int* total_pages, int32_t* out_lengths,
                        int32_t* out_pages, uint16_t* out_k, uint16_t* out_v);

/* max |a-b| over n floats; +inf if either side holds a non-finite value
 * (src/main.cu:242-250). */
float oracle_max_abs_error(const float* a, const float* b, size_t n);

#ifdef __cplusplus
}
#endif

#endif /* BC_ORACLE_H_ */
