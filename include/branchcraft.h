/*
 * Branchcraft paged-attention hot path for MI355X (gfx950): the C ABI.
 *
 * Every entry point takes plain device pointers, POD structs and a HIP
 * stream, launches asynchronously on that stream and never synchronises or
 * allocates.  Return values are HIP error codes: BC_SUCCESS (hipSuccess) or
 * BC_ERROR_INVALID_VALUE (hipErrorInvalidValue) when an argument check
 * fails, otherwise the launch error reported by the HIP runtime.
 *
 * FP16 tensors are passed as `const bc_half*` (IEEE binary16 bit patterns).
 *
 * State, per device: a cache of the CU count, and the split-scratch pool
 * that the entry points without a workspace argument (bc_packed_decode,
 * bc_tree_verify) borrow from -- BC_SCRATCH_SLOTS slots of
 * BC_SCRATCH_SLOT_BYTES in a static device array (72 MiB per GPU the
 * library runs on, held until the process ends; a slot holds the split
 * workspace of every packed decode shape up to D = 128 on 256 CUs).  A call on a stream takes
 * the slot that stream used last (reused in stream order), else a free
 * slot, else the least recently used slot whose last use was recorded in
 * the slot's event, which the stream then waits for on the device
 * (hipStreamWaitEvent).  Events are recorded only after some call has found
 * every slot owned by other streams; from then on after every use.  Calls
 * on any streams and host threads may therefore overlap, and up to
 * BC_SCRATCH_SLOTS streams run at no extra GPU cost.  Under graph capture,
 * for shapes whose split scratch exceeds a slot, when every slot is owned
 * by another stream with no recorded use, or when a HIP call of the pool
 * fails, these calls run their single-pass kernels instead (same results up
 * to floating-point reassociation).  Each slot's event is created once;
 * nothing is allocated per call.  A stream must not be destroyed while one
 * of its calls is still running (its handle may be reused).
 * bc_packed_decode_noalloc uses a separate static array
 * (BC_STATIC_SCRATCH_BYTES).
 *
 * Reference interface replaced: include/branchcraft.hpp:8-74 of
 * Haaziq386/branchcraft-cuda (namespace branchcraft, cudaError_t returns).
 */
#ifndef BRANCHCRAFT_H_
#define BRANCHCRAFT_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bc_half;
/* Same type as hipStream_t; a null stream is the default stream. */
typedef struct ihipStream_t* bc_stream_t;

enum {
  BC_SUCCESS = 0,             /* hipSuccess */
  BC_ERROR_INVALID_VALUE = 1, /* hipErrorInvalidValue */
  BC_ERROR_OUT_OF_MEMORY = 2, /* hipErrorOutOfMemory: a fixed scratch is too small */
};

/* The split-scratch pool of bc_packed_decode and bc_tree_verify: slots per
 * GPU and bytes per slot. */
#define BC_SCRATCH_SLOTS 4
#define BC_SCRATCH_SLOT_BYTES (18u << 20)

/* Tokens per KV page (reference: kPageSize, include/branchcraft.hpp:8). */
#define BC_PAGE_SIZE 16
/* Largest split count bc_decode accepts (the reference caps at 16,
 * src/paged_gqa.cu:126; the cap is raised here, scratch stays caller-sized). */
#define BC_MAX_SPLITS 256
/* Largest draft tree (reference: src/tree_attention.cu:96). */
#define BC_MAX_TREE_NODES 256

/* Reference: struct Shape, include/branchcraft.hpp:11-18 (same field order). */
typedef struct bc_shape {
  int batch;
  int query_heads;
  int kv_heads;
  int dim;            /* 64 or 128 */
  int max_pages;      /* page-table row length */
  int physical_pages; /* pool size P */
} bc_shape;

/* Reference: struct Inputs, include/branchcraft.hpp:20-30.
 * q [B,Hq,D] f16; k, v [P,16,Hkv,D] f16; pages [B,max_pages] i32;
 * lengths [B] i32; output [B,Hq,D] f32.  Empty sequences produce zeros. */
typedef struct bc_inputs {
  const bc_half* q;
  const bc_half* k;
  const bc_half* v;
  const int32_t* pages;
  const int32_t* lengths;
  float* output;
} bc_inputs;

/* Reference: struct Scratch, include/branchcraft.hpp:32-37.
 * For splits > 1 the caller provides partial_a = splits*B*Hq*D floats and
 * partial_ml = splits*B*Hq*2 floats; both may be null for splits == 1. */
typedef struct bc_scratch {
  float* partial_a;
  float* partial_ml;
} bc_scratch;

/* Reference: struct TreeInputs, include/branchcraft.hpp:43-53.
 * draft_q [B,N,Hq,D]; draft_k/draft_v [B,N,Hkv,D]; parent [B,N] with
 * parent < node or -1; output f32 [B,N,Hq,D].  prefix.q and prefix.output
 * are unused and may be null. */
typedef struct bc_tree_inputs {
  bc_inputs prefix;
  const bc_half* draft_q;
  const bc_half* draft_k;
  const bc_half* draft_v;
  const int32_t* parent;
  float* output;
} bc_tree_inputs;

/* Paged GQA decode.  splits == 1 runs one workgroup per (sequence, head
 * block), its waves splitting the pages and merging in LDS, with no scratch.
 * splits > 1 spreads the batch's pages over equal ranges of the concatenated
 * sequences, at most (splits - 1) * B + 1 of them and at most one wave of
 * workgroups (R = 4 * CUs / head blocks ranges, twice that at dim 64, and
 * at most half the table's pages), and merges the FP32
 * partial softmax states of the sequences a range boundary cuts; the
 * partials fit the reference's scratch sizes for `splits`.  FP16 tensors
 * that are not 16-byte aligned are read with 2-byte loads.
 * Replaces branchcraft::decode, include/branchcraft.hpp:39-40
 * (src/paged_gqa.cu:122-132).  Rejects: batch/Hq/Hkv < 1, Hq % Hkv != 0,
 * dim not 64/128, max_pages or physical_pages < 1, splits outside
 * [1, BC_MAX_SPLITS], a null input, null scratch with splits > 1. */
int bc_decode(bc_shape shape, bc_inputs in, bc_scratch scratch, int splits,
              bc_stream_t stream);

/* Split-count heuristic for bc_decode on a device with `cu_count` compute
 * units; returns a value in [1, BC_MAX_SPLITS]: 1 with one or two head
 * blocks once batch * head blocks >= cu_count; else 2 for batches of at
 * least one wave of flat ranges (4 * cu_count / head blocks, twice that at
 * dim 64: 128 sequences at 8 KV heads of 4 query heads and dim 128 on 256
 * CUs) at any length; else 1 for
 * max_length < 512.
 * Replaces branchcraft::auto_splits, include/branchcraft.hpp:41
 * (src/paged_gqa.cu:134-142), retuned for 256-CU MI355X workgroups: unlike
 * the reference (at most 16) it may return more than 16 (33 for 4
 * sequences of 32K tokens, 128 for one), so the caller sizes bc_decode's
 * scratch for the value it passes (splits*B*Hq*D and splits*B*Hq*2 floats).
 * The C++ branchcraft::auto_splits caps the result at 16 by default. */
int bc_auto_splits(bc_shape shape, int max_length, int cu_count);

/* Ancestor-only tree verification over a paged prefix.
 * Replaces branchcraft::tree_verify, include/branchcraft.hpp:55-56
 * (src/tree_attention.cu:93-105).  Shapes whose prefix splits (as
 * bc_tree_verify_ws would split it) run the split kernels with a slot of the
 * library's scratch pool (see the state note at the top), giving
 * bc_tree_verify_ws's results bit for bit; otherwise one workgroup per
 * (request, KV head, row tile) streams the whole prefix.  Tensors that are
 * not 16-byte aligned take an element-wise single pass.
 * Rejects, as the reference: batch/Hq/Hkv < 1, Hq % Hkv != 0, dim not
 * 64/128, max_pages < 1, nodes outside [1, BC_MAX_TREE_NODES], a null K/V,
 * page table, lengths, draft tensor, parent array or output.
 * physical_pages >= 1 gives the pool size: page ids inside a length that
 * fall outside [0, physical_pages) are skipped.  physical_pages < 1 (an
 * empty pool, as the torch op passes for a 0-page prefix_k) means the size
 * is not given: ids inside a length are trusted as in the reference (only
 * negative ones are skipped), nothing outside the lengths is read, and the
 * call runs the single-pass kernel with every request's rows attending to
 * the prefix tokens inside its length plus its ancestors. */
int bc_tree_verify(bc_shape shape, bc_tree_inputs in, int nodes,
                   bc_stream_t stream);

/* Bytes of workspace bc_tree_verify_ws needs for this shape (0 when the
 * shape does not benefit from splitting the prefix, and when
 * physical_pages < 1). */
size_t bc_tree_verify_workspace_size(bc_shape shape, int nodes);

/* bc_tree_verify with each request's tiles split over several workgroups
 * and an FP32 merge; `workspace` holds at least
 * bc_tree_verify_workspace_size bytes.  A null workspace, one smaller than
 * required or one not aligned to 16 bytes is ignored and the call is
 * bc_tree_verify's.  Results match bc_tree_verify within floating-point
 * reassociation (bit for bit when that call splits too). */
int bc_tree_verify_ws(bc_shape shape, bc_tree_inputs in, int nodes,
                      void* workspace, size_t workspace_bytes,
                      bc_stream_t stream);

/* Copy accepted draft K/V rows into physical cache slots:
 * cache[dest_pages[i], dest_slots[i]] <- draft[request, path_nodes[i]] for
 * i < accepted, K and V, bit-exact.  Entries whose node, page or slot is out
 * of range are skipped.  shape.kv_heads, shape.dim, shape.batch and
 * shape.physical_pages describe the tensors; physical_pages < 1 means the
 * pool size is not given (page ids are then only checked for >= 0), and
 * kv_heads < 1 copies nothing.  Any 2-byte aligned pointers work (16-byte
 * copies when all four are 16-byte aligned).
 * Replaces branchcraft::commit_path, include/branchcraft.hpp:61-65
 * (src/tree_attention.cu:107-122), with its rejections: a null pointer,
 * request outside [0, batch), nodes < 1, accepted outside [1, nodes], dim
 * not 64/128. */
int bc_commit_path(bc_shape shape, const bc_half* draft_k,
                   const bc_half* draft_v, bc_half* cache_k, bc_half* cache_v,
                   const int32_t* path_nodes, const int32_t* dest_pages,
                   const int32_t* dest_slots, int request, int nodes,
                   int accepted, bc_stream_t stream);

/* Accepted-path commits of several requests in one launch: entry i copies
 * the K and V rows (all heads) of draft[requests[i], path_nodes[i]] into
 * cache[dest_pages[i], dest_slots[i]], for i < count.  Drafts are
 * [shape.batch, nodes, Hkv, D]; entries with a request, node, page or slot
 * out of range are skipped (pages as for bc_commit_path; kv_heads < 1 copies
 * nothing).  No reference counterpart: it batches the
 * per-request commit_path calls of a transaction (src/tree_attention.cu:
 * 107-122; python/branchcraft_torch/transaction.py:144-148) into one launch.
 * Entries must not write the same (page, slot) twice. */
int bc_commit_paths(bc_shape shape, const bc_half* draft_k,
                    const bc_half* draft_v, bc_half* cache_k, bc_half* cache_v,
                    const int32_t* requests, const int32_t* path_nodes,
                    const int32_t* dest_pages, const int32_t* dest_slots,
                    int nodes, int count, bc_stream_t stream);

/* Copy whole pages (all 16 slots, K and V) cache[dst_pages[i]] <-
 * cache[src_pages[i]] for i < count: the copy-on-write clone of a shared
 * partial page.  Out-of-range page ids (negative, or not below
 * physical_pages when that is >= 1) and src == dst are skipped; kv_heads < 1
 * copies nothing.  All
 * pairs copy concurrently, so the destinations must be distinct and no
 * destination may also be a source; otherwise the result is unspecified.
 * Any 2-byte aligned pointers work.  No reference C++
 * counterpart: it replaces the D2D copies at src/main.cu:276-281 and the
 * torch copy_ at python/branchcraft_torch/transaction.py:133-134. */
int bc_copy_pages(bc_shape shape, bc_half* cache_k, bc_half* cache_v,
                  const int32_t* src_pages, const int32_t* dst_pages,
                  int count, bc_stream_t stream);

/* vLLM-style packed-cache decode with FP16 output.  Token t of sequence b
 * lives at element offset
 *   pages[b, t/16]*block_stride + kvh*head_stride + (t%16)*slot_stride
 * with K at that offset and V at offset + kv_stride; the head dimension is
 * contiguous.  kv_stride == dim gives the reference's logical
 * [P,Hkv,16,2D] layout; [P,2,16,Hkv,D] uses kv_stride = 16*Hkv*D.
 * Replaces branchcraft::packed_decode, include/branchcraft.hpp:70-74
 * (src/packed_decode.cu:64-82), adding kv_stride.  Rejects the bc_decode
 * shape rules plus any stride < 1 and scale <= 0 (or NaN).  Shapes that
 * split (bc_packed_decode_workspace_size > 0) run the split kernels with a
 * slot of the library's scratch pool (see the state note at the top), giving
 * bc_packed_decode_ws's results bit for bit; the others run unsplit. */
int bc_packed_decode(bc_shape shape, const bc_half* q, const bc_half* packed_kv,
                     const int32_t* pages, const int32_t* lengths,
                     bc_half* output, long long block_stride,
                     long long head_stride, long long slot_stride,
                     long long kv_stride, float scale, bc_stream_t stream);

/* Bytes of workspace bc_packed_decode_ws needs for this shape: FP32
 * partials of S slots of Hq * (D + 2) floats and one int per range, S = 2R
 * above 64 sequences where R < 4B, else R + B (at most 2R either way),
 * R = 4 * CUs / head blocks flat ranges (twice that at dim 64, at
 * most half of batch * max_pages).  0 when bc_auto_splits, given the table's
 * capacity (max_pages * 16 tokens), keeps the shape unsplit: one or two
 * head blocks whose (sequence, head block) workgroups fill the CUs; a batch
 * below R with a table under 512 tokens, one of at most 768 tokens whose
 * workgroups fit the CUs, or one of at most 1024 tokens whose workgroups
 * fill half the CUs or more.  Such calls run
 * unsplit, with no merge, whatever workspace is passed. */
size_t bc_packed_decode_workspace_size(bc_shape shape);

/* bc_packed_decode with the batch's pages spread over equal ranges of the
 * concatenated sequences, one wave of workgroups (four waves per CU, eight
 * at dim 64), and an FP32 merge of the sequences a range boundary cuts.
 * The workgroup count and the workspace size depend on the shape and the
 * device's CU count only; the kernels find the ranges from the lengths on
 * the device, so no lengths are read on the host.  A null workspace, one
 * smaller than required or not aligned to 16 bytes is ignored and the call
 * is bc_packed_decode's; a shape whose workspace size is 0 runs unsplit. */
int bc_packed_decode_ws(bc_shape shape, const bc_half* q,
                        const bc_half* packed_kv, const int32_t* pages,
                        const int32_t* lengths, bc_half* output,
                        long long block_stride, long long head_stride,
                        long long slot_stride, long long kv_stride,
                        float scale, void* workspace, size_t workspace_bytes,
                        bc_stream_t stream);

/* Bytes of the static device scratch of bc_packed_decode_noalloc (per GPU). */
#define BC_STATIC_SCRATCH_BYTES (16u << 20)

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): bc_packed_decode_ws with its split workspace taken from
 * a static device array of BC_STATIC_SCRATCH_BYTES (16 MiB) that each GPU
 * holds until the process ends, so the call allocates nothing.  Shapes whose
 * workspace (bc_packed_decode_workspace_size) exceeds that size return
 * BC_ERROR_OUT_OF_MEMORY without launching; shapes that need none run
 * unsplit.  Every call on one GPU shares that GPU's array: calls that overlap
 * on one GPU (other streams, other host threads) race and must not be
 * issued.  Otherwise the same arguments, rules and results as
 * bc_packed_decode_ws. */
int bc_packed_decode_noalloc(bc_shape shape, const bc_half* q, const bc_half* packed_kv,
                             const int32_t* pages, const int32_t* lengths,
                             bc_half* output, long long block_stride,
                             long long head_stride, long long slot_stride,
                             long long kv_stride, float scale, bc_stream_t stream);

/* Library version string, for logs. */
const char* bc_version(void);

#ifdef __cplusplus
}
#endif

#endif /* BRANCHCRAFT_H_ */
