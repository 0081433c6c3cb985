/*
 * pagedkv.h -- C ABI of the MI355X paged-KV engine (libpagedkv.so).
 *
 * This is the drop-in boundary under the candle provider's `engine = "paged"`
 * path of einyx/ai-engine.  Every entry point is plain C: opaque handles,
 * raw pointers, sizes and an int status.  No torch, HIP or Rust types cross
 * it; HIP streams are passed as `void*` (a hipStream_t, NULL = default stream).
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *   KvPool::new            crates/ai-engine-candle/src/paged/attention.rs:39-55
 *   KvPool::write          crates/ai-engine-candle/src/paged/attention.rs:57-83
 *   KvPool::gather_seq     crates/ai-engine-candle/src/paged/attention.rs:85-97
 *   build_mask + sdpa      crates/ai-engine-candle/src/paged/attention.rs:11-28,100-136
 *   decode attention slice crates/ai-engine-candle/src/paged/transformer.rs:271-292
 *   prefill attention      crates/ai-engine-candle/src/paged/transformer.rs:139-196
 *   BlockAllocator/Table   crates/ai-engine-candle/src/paged/block_table.rs:5-58
 *
 * Conventions shared by every call:
 *  - Status: 0 = PKV_OK, negative = error.  The message of the last error of a
 *    pool is returned by pkv_last_error(pool); errors of calls that have no pool
 *    (create, allocator) by pkv_last_error(NULL) on the calling thread.
 *    No call unwinds, aborts or panics across the boundary.
 *  - Threading: a pool handle is externally synchronised (one caller thread at a
 *    time, like the reference's single engine thread, engine.rs:49).  Device
 *    work is enqueued on the caller's stream and is stream-ordered; the library
 *    starts no threads.
 *  - Pool layout (per layer, K and V separately), identical to the reference's
 *    KvPool tensors: [num_blocks][block_size][n_kv_head][head_dim], row-major,
 *    element type `dtype`.  Slot s = block_id * block_size + pos % block_size
 *    addresses the row [s][n_kv_head][head_dim] (attention.rs:88-91).
 *  - Device arrays (q, k, v, out, slot mappings, block tables, lengths) are
 *    device pointers unless the parameter name ends in `_host`.
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------ */
#define PKV_OK 0
#define PKV_ERR_INVALID (-1)     /* invalid argument or shape               */
#define PKV_ERR_OOM (-2)         /* device or host allocation failed        */
#define PKV_ERR_HIP (-3)         /* HIP runtime error                       */
#define PKV_ERR_UNSUPPORTED (-4) /* shape/dtype combination not provided    */
#define PKV_ERR_CAPACITY (-5)    /* allocator: free list too short          */
#define PKV_ERR_DEVICE_DATA (-6) /* kernel saw an out-of-range id/length    */

/* ---- element types ----------------------------------------------------- */
#define PKV_F32 0
#define PKV_F16 1
#define PKV_BF16 2

/* ---- pool selectors ---------------------------------------------------- */
#define PKV_K 0
#define PKV_V 1

typedef struct pkv_pool pkv_pool;

/* Library version string, e.g. "pagedkv 0.1 gfx950". */
const char* pkv_version(void);

/* Message of the last failed call on `pool` (or of the calling thread when
 * pool is NULL).  Never NULL; "" when there was no error. */
const char* pkv_last_error(const pkv_pool* pool);

/* Allocate K and V pools for `n_layers` layers on HIP device `device`, zero
 * filled like Tensor::zeros in KvPool::new (attention.rs:39-55).  One handle
 * stands for the reference's Vec<KvPool> (engine.rs:70-72): layer l of the
 * handle is the reference's kv[l].  Block ids are shared by all layers.
 * dtype: PKV_F32 (the reference's own dtype), PKV_F16 or PKV_BF16.
 * Shape limits (PKV_ERR_UNSUPPORTED otherwise), narrower than the
 * reference's KvPool::new, which takes any sizes:
 *  - head_dim 64, 128 or 256.  The reference reads it from GGUF
 *    (`attention.key_length`, else embedding_length / head_count,
 *    arch.rs:77-83); every llama / qwen2 / qwen3 model of the supported
 *    architectures (arch.rs:27-36) has 64 or 128.
 *  - block_size a power of two in [1, 256].  The reference takes any
 *    usize (block_table.rs:17-30); its engine default and the block size of
 *    its tests is 16 (app.rs:701, tests/paged_parity.rs:33).  Sizes below
 *    16 run kernels that read a block id per lane (a 16-token attention
 *    tile then spans several blocks); other sizes (24, 48, ...) are
 *    refused: every kernel addresses a token's slot with shifts and masks.
 * n_kv_head is any count in 1 .. 1024, and the slab (2 * n_layers *
 * num_blocks * block_size * n_kv_head * head_dim elements) below 2^63
 * bytes (else PKV_ERR_UNSUPPORTED); the GQA ratio n_head / n_kv_head of the
 * attention calls is any positive integer (repeat_kv, attention.rs:113,
 * 128-136).  The pool is plain device memory from hipMalloc, allocated by
 * the library itself.  No kernel loads pool bytes that the same launch
 * stored (the fused appends hand the new rows to the attention through
 * LDS; a launch's copies and moves read each block before any write to it,
 * in the same thread), so results do not depend on the pool's caching
 * or coherence attributes. */
int pkv_pool_create(pkv_pool** out, int n_layers, int num_blocks,
                    int block_size, int n_kv_head, int head_dim, int dtype,
                    int device);
int pkv_pool_destroy(pkv_pool* pool);

/* Shape and placement queries. */
int pkv_pool_shape(const pkv_pool* pool, int* n_layers, int* num_blocks,
                   int* block_size, int* n_kv_head, int* head_dim, int* dtype);
size_t pkv_pool_layer_bytes(const pkv_pool* pool); /* bytes of one K (or V) */
int pkv_pool_layer_ptrs(const pkv_pool* pool, int layer, void** k, void** v);

/* Synchronous host<->pool byte copies (tests, debugging, checkpoints). */
int pkv_pool_read(pkv_pool* pool, int layer, int which, size_t byte_offset,
                  size_t nbytes, void* host_dst);
int pkv_pool_write(pkv_pool* pool, int layer, int which, size_t byte_offset,
                   const void* host_src, size_t nbytes);

/* Fill every layer's K and V with N(0,1) samples rounded to the pool dtype,
 * from a counter-based hash of (seed, layer, which, element index).
 * A workload generator for benchmarks; no reference counterpart. */
int pkv_pool_fill_normal(pkv_pool* pool, uint64_t seed, void* stream);

/* The check of pkv_pool_fill_normal after blocks have moved (copy-on-write,
 * compaction; no reference counterpart): counts, into *mismatches, the
 * 16-byte chunks of block blocks[i], over every layer's K and V, that differ
 * from what pkv_pool_fill_normal(seed) wrote into block origin[i].
 * blocks, origin: device int32 [n]; an id out of range counts the item as
 * mismatching and is reported by pkv_pool_check().  Synchronous. */
int pkv_pool_verify_normal(pkv_pool* pool, uint64_t seed, const int32_t* blocks,
                           const int32_t* origin, int n, uint64_t* mismatches,
                           void* stream);

/* Read every byte of blocks[i] in every layer's K and V and add their
 * 32-bit words (mod 2^64) into *sum, a device uint64 the caller zeroes;
 * asynchronous on `stream`.  No reference counterpart: the read rate of a
 * random block set (the decode roofline's read ceiling, bytes read / time)
 * and a checksum of the blocks.  blocks: device int32 [n]; an id out of
 * range is skipped and reported by pkv_pool_check(). */
int pkv_pool_read_blocks(pkv_pool* pool, const int32_t* blocks, int n, uint64_t* sum,
                         void* stream);

/* ---- KV append / scatter (KvPool::write, attention.rs:57-83) -----------
 * k, v: [n_tokens][n_kv_head][head_dim] in the pool dtype.
 * slot_mapping: [n_tokens] int32, slot = block * block_size + offset
 * (the host computes it with BlockAllocator::locate, block_table.rs:55-58).
 * Token i is copied bit-exactly to row slot_mapping[i] of layer `layer`'s K
 * and V pools; no other byte changes.  A negative slot skips the token
 * (padding); a slot >= num_blocks*block_size is not written and makes the
 * next pkv_pool_check() report PKV_ERR_DEVICE_DATA. */
int pkv_append(pkv_pool* pool, int layer, const void* k, const void* v,
               const int32_t* slot_mapping, int n_tokens, void* stream);

/* ---- gather (KvPool::gather_seq, attention.rs:85-97) -------------------
 * out_k, out_v: [len][n_kv_head][head_dim] pool dtype, bit-exact copies of
 * the rows at slot blocks[p / bs] * bs + p % bs, p = 0..len-1.
 * block_table: device int32 [ceil(len / block_size)]. */
int pkv_gather_seq(pkv_pool* pool, int layer, const int32_t* block_table,
                   int len, void* out_k, void* out_v, void* stream);

/* ---- gather of several sequences in one launch (no reference counterpart:
 * the batched form of gather_seq for callers that want the K/V of many
 * sequences contiguous, e.g. a varlen attention kernel) ------------------
 * Sequence b's positions 0 .. cu_lens[b+1]-cu_lens[b]-1 are copied, bit for
 * bit as by pkv_gather_seq with block_tables[b], to rows cu_lens[b] ..
 * cu_lens[b+1]-1 of out_k / out_v ([total_rows][n_kv_head][head_dim]).
 * cu_lens: device int32 [batch+1], cu_lens[0] = 0, nondecreasing;
 * total_rows = cu_lens[batch] (host value).  block_tables: device int32
 * [batch][max_blocks_per_seq].  batch <= 4096.  A block id out of range, or
 * a length beyond the table, zeroes those rows and is reported by
 * pkv_pool_check(). */
int pkv_gather_varlen(pkv_pool* pool, int layer, const int32_t* block_tables,
                      int max_blocks_per_seq, const int32_t* cu_lens, int batch,
                      int total_rows, void* out_k, void* out_v, void* stream);

/* ---- block copy (copy-on-write after fork; no reference counterpart) ----
 * For every layer and both K and V: block dst[i] <- block src[i], i < n.
 * src, dst: device int32 [n].  dst ids must be distinct and no dst may be a
 * src of the same call (the CoW contract: dst blocks are fresh); otherwise
 * the copies race.  An id out of range is skipped and reported by
 * pkv_pool_check().  With PKV_DEBUG set in the environment (to anything but
 * "0") the call first checks the contract on host copies of src and dst
 * (synchronising the stream) and returns PKV_ERR_INVALID, copying nothing,
 * if it is broken. */
int pkv_copy_blocks(pkv_pool* pool, const int32_t* src, const int32_t* dst,
                    int n, void* stream);

/* ---- compaction (no reference counterpart) ------------------------------
 * Moves block src_host[i] to dst_host[i] for every layer and K/V, in place:
 * the dst set may overlap the src set (e.g. survivors gathered into a
 * contiguous prefix).  src ids distinct, dst ids distinct.  The plan (chains
 * and cycles of the move graph) is built on the host, so ids are host arrays;
 * it is uploaded to a device buffer the pool allocates once, at creation,
 * for the largest plan.  Stream-ordered: the call returns once the moves are
 * enqueued (it waits only, if at all, for the previous call's plan upload
 * before reusing the pinned staging copy).  Each byte is read once and
 * written once; no scratch pool is allocated. */
int pkv_compact(pkv_pool* pool, const int32_t* src_host,
                const int32_t* dst_host, int n, void* stream);

/* ---- paged decode attention (sdpa + build_mask + the decode-step
 * attention slice, attention.rs:100-136, transformer.rs:271-292) ----------
 * One query token per sequence.
 *  q:            [batch][n_head][head_dim], pool dtype (post-RoPE).
 *  out:          [batch][n_head * head_dim], out_dtype (PKV_F32 or the pool
 *                dtype); element [b][h*head_dim + d] as in attention.rs:124-125.
 *  block_tables: [batch][max_blocks_per_seq] int32.
 *  context_lens: [batch] int32 = number of keys attended = seq_lens[b] + 1
 *                (the reference's valid_lens, transformer.rs:289).
 *  max_context_len: host int >= every context_lens[b] (the reference's
 *                kv_len, transformer.rs:241); sizes the partition grid.
 *                1 .. 2^30, and batch * n_kv_head * max(16, ceil(
 *                max_context_len / 1024)) below 2^26 (one 64-lane wave
 *                each; else PKV_ERR_INVALID / _UNSUPPORTED).
 *  scale:        multiplies q.k (the reference uses 1/sqrt(head_dim),
 *                attention.rs:118-120).
 *  k_new, v_new: NULL, or [batch][n_kv_head][head_dim]: then the call first
 *                stores them at token position context_lens[b]-1 of sequence
 *                b (KvPool::write at seq_lens[b], transformer.rs:276) and the
 *                attention sees them -- append and attention in one launch.
 * GQA: query head h reads kv head h / (n_head / n_kv_head) (attention.rs:128-136),
 * for any integer ratio; ratios above 16 run as one launch (and merge) per
 * slice of 16 query heads, each reading the group's K/V.
 * fp32 accumulation; softmax in fp32 with an exp2 formulation.
 * context_lens[b] == 0 yields a zero output row.
 * Mask: key k of row b is attended iff k < context_lens[b] -- the
 * reference's build_mask(seq_lens + 1, positions, kv_len) as the decode step
 * calls it, where positions == seq_lens (transformer.rs:289-290,
 * engine.rs:130-133), so its second bound k <= positions[b]
 * (attention.rs:22) coincides with the first.  Callers whose positions
 * differ from seq_lens use pkv_decode_attention_positions. */
int pkv_decode_attention(pkv_pool* pool, int layer, const void* q, void* out,
                         int out_dtype, const int32_t* block_tables,
                         int max_blocks_per_seq, const int32_t* context_lens,
                         int max_context_len, int batch, int n_head,
                         float scale, const void* k_new, const void* v_new,
                         void* stream);

/* pkv_decode_attention with build_mask's second bound (attention.rs:11-28):
 * key k of row b is attended iff k < context_lens[b] and k <= positions[b],
 * positions being the rows' query positions (the reference's q_positions,
 * transformer.rs:290).  positions: device int32 [batch], non-NULL.  k_new /
 * v_new are still stored at context_lens[b] - 1 (KvPool::write at seq_lens,
 * transformer.rs:276) and attended only when positions[b] >=
 * context_lens[b] - 1.  A negative position attends no key: the row is
 * zero, nothing is stored for it, and pkv_pool_check() reports
 * PKV_ERR_DEVICE_DATA.  Other arguments and limits as pkv_decode_attention;
 * the split-context merge uses the same bounded lengths. */
int pkv_decode_attention_positions(pkv_pool* pool, int layer, const void* q, void* out,
                                   int out_dtype, const int32_t* block_tables,
                                   int max_blocks_per_seq, const int32_t* context_lens,
                                   const int32_t* positions, int max_context_len, int batch,
                                   int n_head, float scale, const void* k_new, const void* v_new,
                                   void* stream);

/* Workspace that pkv_decode_attention needs for a given batch/length; the
 * pool grows its internal workspace on demand with a hipMalloc.  The buffer
 * it replaces stays allocated, since queued work may still read it, until
 * the next reserve call, pkv_pool_destroy, or a later growth that would
 * otherwise keep more retired bytes than the new workspace holds (that
 * growth synchronises the device and frees them).  Callers that must not
 * allocate or synchronise later (stream capture, serving loops) reserve the
 * largest shape they will use up front; the reserve calls synchronise the
 * device when they free replaced buffers. */
size_t pkv_decode_workspace_bytes(const pkv_pool* pool, int batch, int n_head,
                                  int max_context_len);
int pkv_pool_reserve_decode(pkv_pool* pool, int batch, int n_head,
                            int max_context_len);

/* pkv_decode_attention without any allocation.  No counterpart in the
 * reference: for callers that cannot allocate device memory during a call
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as pkv_decode_attention
 * (bit for bit), but the split-context partials go to a static device array
 * of PKV_NOALLOC_SCRATCH_BYTES that every GPU the library runs on holds for
 * the life of the process, not to the pool's workspace; the call makes no
 * hipMalloc, hipFree or other allocating call and records no profile
 * events.  A launch whose partials need more than the array
 * (pkv_decode_workspace_bytes > PKV_NOALLOC_SCRATCH_BYTES, e.g. batch 256
 * with contexts up to 32k on 8 kv heads of 128) returns PKV_ERR_UNSUPPORTED
 * before anything is enqueued.  All calls on one GPU share its array, so
 * calls that overlap on one GPU (different streams, threads or pools)
 * race: the caller orders them, e.g. on one stream. */
#define PKV_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int pkv_decode_attention_noalloc(pkv_pool* pool, int layer, const void* q, void* out,
                                 int out_dtype, const int32_t* block_tables,
                                 int max_blocks_per_seq, const int32_t* context_lens,
                                 int max_context_len, int batch, int n_head,
                                 float scale, const void* k_new, const void* v_new,
                                 void* stream);

/* ---- chunked prefill attention (prefill_seq attention,
 * transformer.rs:139-196, generalised to a prior context) -----------------
 * Sequence s has q_len_s = cu_q_lens[s+1]-cu_q_lens[s] query tokens whose K/V
 * are already in the pool (pkv_append); its context has context_lens[s] keys
 * in total, so query i sits at position context_lens[s]-q_len_s+i and
 * attends keys 0..that position (causal; the reference's mask j > i -> -inf
 * when the prior context is empty).
 *  q:   [total_q][n_head][head_dim] pool dtype;  out: [total_q][n_head*head_dim].
 *  cu_q_lens: [n_seqs+1] int32; context_lens: [n_seqs] int32;
 *  block_tables: [n_seqs][max_blocks_per_seq] int32.
 *  max_q_len, max_context_len: host upper bounds, at most 2^30.  scale > 0 and finite
 *  (the reference's 1/sqrt(head_dim)); otherwise PKV_ERR_INVALID.
 *  Any GQA ratio n_head / n_kv_head; every pool dtype and head_dim. */
int pkv_prefill_attention(pkv_pool* pool, int layer, const void* q, void* out,
                          int out_dtype, const int32_t* cu_q_lens,
                          const int32_t* context_lens,
                          const int32_t* block_tables, int max_blocks_per_seq,
                          int n_seqs, int max_q_len, int max_context_len,
                          int n_head, float scale, void* stream);

/* pkv_prefill_attention with the chunk's K/V stored in the same launch (the
 * reference stores every prompt token with KvPool::write before attending,
 * transformer.rs:173-177; pkv_append + pkv_prefill_attention in one call).
 * k_new, v_new: [total_q][n_kv_head][head_dim] in the pool dtype, 16-byte
 * aligned; token i of sequence s is stored at its position
 * context_lens[s] - q_len_s + i (slot from block_tables) and attended from
 * these rows, so the result and the pool afterwards equal pkv_append
 * followed by pkv_prefill_attention.  A block id out of range is reported by
 * pkv_pool_check(). */
int pkv_prefill_attention_append(pkv_pool* pool, int layer, const void* q,
                                 void* out, int out_dtype,
                                 const int32_t* cu_q_lens,
                                 const int32_t* context_lens,
                                 const int32_t* block_tables,
                                 int max_blocks_per_seq, int n_seqs,
                                 int max_q_len, int max_context_len,
                                 int n_head, float scale, const void* k_new,
                                 const void* v_new, void* stream);

/* Workspace of pkv_prefill_attention for the given launch shape: launches
 * with few row blocks (fewer than can fill the GPU) split long key ranges
 * into parts that are merged afterwards, with partial results in the pool's
 * workspace (0: no split).  The pool grows the workspace on demand;
 * callers that must not allocate later reserve it up front. */
size_t pkv_prefill_workspace_bytes(const pkv_pool* pool, int n_seqs, int n_head,
                                   int max_q_len, int max_context_len);
int pkv_pool_reserve_prefill(pkv_pool* pool, int n_seqs, int n_head,
                             int max_q_len, int max_context_len);

/* ---- a layer's mixed batch in one call (engine step of run_loop,
 * engine.rs:62-237: some sequences prefill a prompt chunk, the others decode
 * one token; the reference attends them one sequence at a time,
 * transformer.rs:139-196 and 271-292) -------------------------------------
 * The arguments of pkv_prefill_attention(_append) and of
 * pkv_decode_attention, as two structs; n_head and scale are shared.  The
 * result (every output row, every stored K/V row, pkv_pool_check's error
 * bits) is identical, bit for bit, to pkv_prefill_attention(_append)
 * followed by pkv_decode_attention on the same stream: for 16-bit pools with
 * head_dim 64 or 128 and n_head / n_kv_head of 4 or 8 (f16 at head_dim 128:
 * 8 only) both run in one kernel launch, their workgroups sharing the CUs
 * (the prefill is bound by MFMA and instruction issue, the decode by HBM);
 * other shapes run the two calls in sequence.  A NULL batch, or one with
 * n_seqs / batch == 0, leaves just the other call.  The two batches must
 * not share the blocks their new rows are stored in (under copy-on-write a
 * sequence appends only to blocks it alone holds).  Workspace: the decode
 * partials and the prefill split partials side by side
 * (pkv_mixed_workspace_bytes). */
typedef struct pkv_prefill_batch {
  const void* q;               /* [total_q][n_head][head_dim], pool dtype */
  void* out;                   /* [total_q][n_head * head_dim], out_dtype */
  int out_dtype;
  const int32_t* cu_q_lens;    /* [n_seqs + 1] */
  const int32_t* context_lens; /* [n_seqs] */
  const int32_t* block_tables; /* [n_seqs][max_blocks_per_seq] */
  int max_blocks_per_seq;
  int n_seqs;
  int max_q_len;
  int max_context_len;
  const void* k_new;           /* chunk K/V stored by the call, or both NULL */
  const void* v_new;
} pkv_prefill_batch;

typedef struct pkv_decode_batch {
  const void* q;               /* [batch][n_head][head_dim], pool dtype */
  void* out;                   /* [batch][n_head * head_dim], out_dtype */
  int out_dtype;
  const int32_t* block_tables; /* [batch][max_blocks_per_seq] */
  int max_blocks_per_seq;
  const int32_t* context_lens; /* [batch], new token included */
  int max_context_len;
  int batch;
  const void* k_new;           /* new token's K/V stored by the call, or both NULL */
  const void* v_new;
} pkv_decode_batch;

int pkv_mixed_attention(pkv_pool* pool, int layer, const pkv_prefill_batch* prefill,
                        const pkv_decode_batch* decode, int n_head, float scale,
                        void* stream);
size_t pkv_mixed_workspace_bytes(const pkv_pool* pool, int n_head,
                                 const pkv_prefill_batch* prefill,
                                 const pkv_decode_batch* decode);

/* ---- rotary position embedding (crates/ai-engine-candle/src/paged/rope.rs,
 * applied per row in the decode step, transformer.rs:252-269) ---------------
 * Tables as Rope::new (rope.rs:14-23): theta_i = 1 / freq_base^(2 i / rope_dim)
 * in f32, angle[p][i] = (float)p * theta_i, cos/sin in f32, shape
 * [max_seq][rope_dim / 2].  The rotation is candle's rotate-half rope that
 * apply_rope uses (rope.rs:38-42): for the halves x1 = x[i], x2 = x[i + d/2]
 * of a head row, out[i] = x1 cos - x2 sin, out[i + d/2] = x1 sin + x2 cos,
 * in f32 with every product rounded (no fused multiply-add), then rounded to
 * the output dtype.  rope_dim is the head_dim of the rows it rotates. */
typedef struct pkv_rope pkv_rope;

/* Fills host arrays cos_host, sin_host [max_seq][rope_dim / 2] (host only). */
int pkv_rope_tables_host(int rope_dim, float freq_base, int max_seq,
                         float* cos_host, float* sin_host);
/* Tables computed on the host (as above) and kept in device memory. */
int pkv_rope_create(pkv_rope** out, int rope_dim, float freq_base, int max_seq,
                    int device);
int pkv_rope_destroy(pkv_rope* rope);
/* Device pointers of the tables (e.g. to share them with other kernels). */
int pkv_rope_tables(const pkv_rope* rope, const float** cos_dev,
                    const float** sin_dev);
/* x: [n_tokens][n_head][rope_dim] in in_dtype; out: same shape in out_dtype
 * (each PKV_F32, PKV_F16 or PKV_BF16; out may alias x when the dtypes
 * match).  positions: device int32 [n_tokens], token t rotated by row
 * positions[t] (Rope::gather, rope.rs:28-32).  A position outside
 * [0, max_seq) leaves that token's rows unwritten and makes the next
 * pkv_rope_check() report PKV_ERR_DEVICE_DATA. */
int pkv_rope_apply(pkv_rope* rope, const void* x, int in_dtype, void* out,
                   int out_dtype, const int32_t* positions, int n_tokens,
                   int n_head, void* stream);
int pkv_rope_check(pkv_rope* rope);

/* Decode attention with the rotary embedding applied inside the kernel: the
 * decode step's per-row RoPE of q and of the new k (transformer.rs:252-269)
 * followed by pkv_decode_attention (same arguments and results).  q and
 * k_new are the projections before rotation and v_new the new values, all
 * in in_dtype (PKV_F32 -- the reference's activations -- or the pool dtype);
 * the rotated q and k are rounded to the pool dtype, as stored k rows are.
 * positions: device int32 [batch] or NULL; NULL uses context_lens[b] - 1,
 * the reference's decode position (positions == seq_lens, engine.rs:130-133).
 * Given, they also bound the keys attended as in
 * pkv_decode_attention_positions (the reference's decode step passes the
 * same positions to the rotation and to build_mask, transformer.rs:237,290).
 * rope->rope_dim must equal the pool's head_dim.  A position outside
 * [0, max_seq) is reported by pkv_pool_check() and rotates by position 0. */
int pkv_decode_attention_rope(pkv_pool* pool, int layer, const pkv_rope* rope,
                              const int32_t* positions, int in_dtype,
                              const void* q, void* out, int out_dtype,
                              const int32_t* block_tables,
                              int max_blocks_per_seq,
                              const int32_t* context_lens, int max_context_len,
                              int batch, int n_head, float scale,
                              const void* k_new, const void* v_new,
                              void* stream);

/* The prefill step's glue in one launch (prefill_seq, transformer.rs:
 * 160-174: apply_rope to q and k, then KvPool::write of every token's k and
 * v, attention.rs:57-83): k rows rotated by positions[t] and v rows stored
 * at slot_mapping[t], as pkv_append; with q (not NULL), its rows rotated
 * into q_out for pkv_prefill_attention.
 *  k, v: [n_tokens][n_kv_head][head_dim], q: [n_tokens][n_head][head_dim],
 *  all in in_dtype (PKV_F32, PKV_F16 or PKV_BF16), 16-byte aligned; the
 *  stored rows and q_out are in the pool dtype (q_out may alias q when
 *  in_dtype is the pool dtype).  positions, slot_mapping: device int32
 *  [n_tokens]; slot < 0 skips that token's k/v (its q is still rotated).
 *  Rotation and rounding as pkv_rope_apply.  A position outside
 *  [0, max_seq) leaves that token's rotated rows unwritten and a slot
 *  beyond the pool its k/v; pkv_pool_check() reports either. */
int pkv_append_rope(pkv_pool* pool, int layer, const pkv_rope* rope,
                    const int32_t* positions, int in_dtype, const void* k,
                    const void* v, const int32_t* slot_mapping, int n_tokens,
                    const void* q, void* q_out, int n_head, void* stream);

/* ---- token selection (crates/ai-engine-runtime/src/sample.rs:12-55) --------
 * The engine copies each logits row to the host and samples it with
 * SamplingConfig {temperature of the request, top_p: None, top_k: None,
 * seed: 42} (crates/ai-engine-candle/src/paged/engine.rs:58-60,145-162,226);
 * this selects on the device and leaves one int32 per row.
 *  logits: device, row b at logits + b * row_stride elements, `vocab` values
 *  each, dtype PKV_F32 / PKV_F16 / PKV_BF16.  temperatures: device f32
 *  [batch], or NULL (every row greedy).  tokens: device int32 [batch].
 * Row b is argmax (first maximum; NaN never chosen; 0 when no value exceeds
 * -inf) when temperatures[b] == 0 or vocab <= 1.  Otherwise sample(): y =
 * logit / temperature sorted descending (ties in index order), the first
 * top_k kept (top_k == 0: None), p = softmax over them, the shortest prefix
 * whose cumulative p reaches top_p kept and renormalised (top_p >= 1 or NaN:
 * None), and the first token at which the cumulative p reaches r =
 * StdRng::seed_from_u64(seed).gen::<f32>() -- the same r on every call, as
 * in the reference.  The token equals the reference's except where its f32
 * running sums fall within their rounding of r or top_p.  Temperatures must
 * be finite and logits of sampled rows free of NaN (the reference's sort is
 * unspecified there).  vocab < 2^24 (probability masses are 2^-40 fixed
 * point summed in 64 bits).  Runs on the calling thread's current device.
 * Batches of at most 128 rows with temperatures and no top_k / top_p split
 * each row over G = min(32, 256 / batch, ceil(vocab / 4096)) workgroups,
 * with 57,624 + 4,096 G bytes per row of partial histograms (at most 184 KiB
 * per row; 1.5 MB for 8 rows, 8.4 MB for 128) in a stream-ordered allocation
 * on `stream` (hipMallocAsync / hipFreeAsync, capturable in a HIP graph); if
 * that allocation fails, one workgroup per row.  Both give the same tokens. */
int pkv_sample(const void* logits, int dtype, long long row_stride, int batch,
               int vocab, const float* temperatures, int top_k, float top_p,
               uint64_t seed, int32_t* tokens, void* stream);
/* sample() of crates/ai-engine-runtime/src/sample.rs:12-48 with the
 * reference's own f32 arithmetic, bit for bit: the token equals the
 * reference's on every row, including rows where its f32 rounding alone
 * moves the pick (pkv_sample matches those only to within that rounding).
 * Same arguments as pkv_sample except top_p: NaN is None and any other value
 * is Some(top_p), as in the reference, where Some(1.0) still truncates once
 * the f32 running sum reaches 1.  Exponentials are glibc's expf (what
 * f32::exp calls on x86-64 Linux), restated on the device and equal to the
 * host libm on every argument the path uses (<= 0); the order is, for f32
 * logits, buckets of y sorted only where a running sum needs the order
 * (rows that need more: a stable radix sort of every key), and for 16-bit
 * logits runs of equal values from a histogram of their 65,536 possible
 * keys; every f32 running sum (the softmax denominator, top_p's cumulative
 * sum, the r threshold) takes exactly the reference's rounding steps.
 * Scratch: 1 MB per row for f16/bf16 logits, 8 bytes per logit per row for
 * f32, at most 512 MB per launch (larger batches run in several launches),
 * in a stream-ordered allocation on `stream`.  One 1024-thread workgroup per
 * row. */
int pkv_sample_exact(const void* logits, int dtype, long long row_stride, int batch,
                     int vocab, const float* temperatures, int top_k, float top_p,
                     uint64_t seed, int32_t* tokens, void* stream);
/* pkv_sample_exact that also reports, for verification (no reference
 * counterpart), which kernel selected each row: routes (device int32
 * [batch]) gets 0 (argmax: temperature 0 or vocab <= 1), 1 (f32 logits:
 * buckets of y, sorted only where a running sum needs the order), 2 (runs
 * of equal 16-bit values; f32 rows whose logits are all bf16 values when
 * the buckets left them) or 3 (the radix sort of every logit).  Tokens are
 * those of pkv_sample_exact. */
int pkv_sample_exact_routes(const void* logits, int dtype, long long row_stride, int batch,
                            int vocab, const float* temperatures, int top_k, float top_p,
                            uint64_t seed, int32_t* tokens, int32_t* routes, void* stream);
/* The exp pkv_sample_exact uses, exposed for verification (no reference
 * counterpart): out[i] = expf(in[i]) as glibc computes it; device arrays of
 * n floats, on `stream`. */
int pkv_sample_expf(const float* in, float* out, long long n, void* stream);
/* StdRng::seed_from_u64(seed).gen::<f32>() (sample.rs:41-42; host only). */
float pkv_sample_draw(uint64_t seed);

/* Kernel timing (instrumentation; no reference counterpart).  While enabled,
 * every pkv_decode_attention, pkv_prefill_attention, pkv_copy_blocks and
 * pkv_compact call records HIP events, owned by the pool, on its stream right
 * before and right after its main kernel -- the partition kernel of decode,
 * not its split-context merge; the one kernel of the others (for compaction,
 * after the plan upload).  pkv_pool_profile_read synchronises,
 * returns the summed main-kernel time in ms and the number of timed
 * launches since the last read, and clears the record. */
int pkv_pool_profile(pkv_pool* pool, int enable);
int pkv_pool_profile_read(pkv_pool* pool, double* total_ms, int* launches);

/* Synchronise the pool's device and report (then clear) any out-of-range
 * slot/block id or length a kernel met since the last check:
 * PKV_OK or PKV_ERR_DEVICE_DATA. */
int pkv_pool_check(pkv_pool* pool);

/* ---- host block bookkeeping (BlockAllocator / BlockTable,
 * block_table.rs:5-58).  Pure host code, usable without a GPU. ------------ */
typedef struct pkv_allocator pkv_allocator;
typedef struct pkv_table pkv_table;

/* BlockAllocator::new: free list [num_blocks-1, ..., 1, 0], pops from the end
 * so the first blocks handed out are 0, 1, 2, ... (block_table.rs:17-21). */
pkv_allocator* pkv_allocator_new(size_t num_blocks, size_t block_size);
void pkv_allocator_free(pkv_allocator* a);
size_t pkv_allocator_free_count(const pkv_allocator* a);       /* :23-25 */
size_t pkv_allocator_blocks_for(const pkv_allocator* a, size_t n_tokens); /* :27-30 */
/* :32-47  PKV_OK, or PKV_ERR_CAPACITY with nothing allocated. */
int pkv_allocator_ensure_capacity(pkv_allocator* a, pkv_table* t,
                                  size_t n_tokens);
/* :49-52  appends the table's blocks to the free list in table order. */
void pkv_allocator_release(pkv_allocator* a, pkv_table* t);
/* :54-58  PKV_ERR_INVALID when pos is beyond the table (the reference panics). */
int pkv_allocator_locate(const pkv_allocator* a, const pkv_table* t,
                         size_t pos, uint32_t* block_id, size_t* slot);

pkv_table* pkv_table_new(void);
void pkv_table_free(pkv_table* t);
size_t pkv_table_len(const pkv_table* t);
const uint32_t* pkv_table_blocks(const pkv_table* t);

/* ---- continuous-batching scheduler (run_loop / prefill block bookkeeping,
 * crates/ai-engine-candle/src/paged/engine.rs:62-237).  Pure host code.
 *
 * The reference's engine thread interleaves scheduling with the model; here
 * the scheduling is a step machine the caller drives around its own model
 * forward:  pkv_sched_step() returns the plan of the next forward (rows, block
 * tables, context lengths, slot mappings, copy-on-write copies), the caller
 * runs the layers (pkv_copy_blocks, pkv_append / pkv_decode_attention /
 * pkv_prefill_attention), samples one token per producing row and hands them
 * to pkv_sched_complete().  What the reference sends on a request's channel
 * (Ok(token) / Err(message) / channel closed) comes back as events.
 *
 * prefill_chunk == 0 reproduces run_loop exactly: an iteration first admits
 * requests (engine.rs:77-100) and prefills each whole prompt (a plan of
 * prefill rows), then runs the capacity/eviction pass and one decode step for
 * every running sequence (engine.rs:102-178, a plan of decode rows).
 * prefill_chunk > 0 is chunked prefill: each step carries the next chunk of
 * every prompt in flight (at most step_token_budget prompt tokens) together
 * with the decode rows.  Extensions with no reference counterpart: fork
 * (shared blocks under reference counts; the first write to a shared block
 * copies it, reported in the plan) and compaction (live blocks renumbered to
 * [0, live) with the fewest moves, returned for pkv_compact). */
typedef struct pkv_sched pkv_sched;

typedef struct {
  int max_num_seqs;      /* EngineConfig (engine.rs:30-36) */
  int block_size;
  int kv_cache_blocks;
  int max_seq;
  int32_t eos_token_id;
  int prefill_chunk;     /* 0: whole prompts (the reference) */
  int step_token_budget; /* chunked mode: prompt tokens per step (0: none) */
} pkv_sched_config;

#define PKV_EV_TOKEN 0    /* Ok(token) */
#define PKV_EV_FINISHED 1 /* the sequence ended; its blocks are released */
#define PKV_EV_ERROR 2    /* Err(message); the sequence ended */

typedef struct {
  int64_t seq;
  int kind;
  int32_t token;
  char message[120];
} pkv_sched_event;

/* One forward's plan; the arrays stay valid until the next step, complete,
 * fork or compact call.  Rows are the prefill rows, then the decode rows. */
typedef struct {
  int n_prefill, n_decode, n_rows, max_blocks, n_tokens, n_copies;
  const int64_t* row_seq;       /* [n_rows] */
  const int32_t* block_tables;  /* [n_rows][max_blocks], 0-padded */
  const int32_t* context_lens;  /* [n_rows] keys attended after the writes */
  const int32_t* cu_q_lens;     /* [n_prefill + 1] offsets of prompt tokens */
  const int32_t* q_start;       /* [n_prefill] position of each chunk's first token */
  const int32_t* slot_mapping;  /* [n_tokens] chunk tokens, then one per decode row */
  const int32_t* positions;     /* [n_tokens] position of each new token */
  const int8_t* produces;       /* [n_rows] 1 if the row yields a token */
  const int32_t* copy_src;      /* [n_copies] copy before the writes */
  const int32_t* copy_dst;
} pkv_sched_plan;

/* Message of the calling thread's last failed pkv_sched_* call. */
const char* pkv_sched_last_error(void);
int pkv_sched_create(pkv_sched** out, const pkv_sched_config* cfg);
void pkv_sched_destroy(pkv_sched* s);
/* GenRequest (engine.rs:13-18) without the channel; *id names its events. */
int pkv_sched_submit(pkv_sched* s, int prompt_len, int max_tokens, int64_t* id);
/* Plans the next forward; n_rows == 0 means nothing is runnable. */
int pkv_sched_step(pkv_sched* s, pkv_sched_plan* plan);
/* tokens: one per producing row, in row order (n = their count).  error !=
 * NULL reports a failed forward: every row's sequence ends with Err (the
 * reference's "prefill: ..." / "forward: ..." paths). */
int pkv_sched_complete(pkv_sched* s, const int32_t* tokens, int n,
                       const char* error);
/* Next event; returns 1 and fills *ev, or 0 when there is none. */
int pkv_sched_poll(pkv_sched* s, pkv_sched_event* ev);
/* Fork a decoding sequence: the child shares its blocks (copy-on-write) and
 * continues from the same position and pending token. */
int pkv_sched_fork(pkv_sched* s, int64_t parent, int max_tokens, int64_t* child);
/* Renumber live blocks to [0, live); src/dst (capacity cap) receive the moves
 * for pkv_compact, *n their count. */
int pkv_sched_compact(pkv_sched* s, int32_t* src, int32_t* dst, int cap, int* n);
/* Introspection: counts, a sequence's table (NULL if it is not live). */
int pkv_sched_counts(const pkv_sched* s, int* running, int* waiting,
                     int* free_blocks);
int pkv_sched_table(const pkv_sched* s, int64_t seq, const uint32_t** blocks,
                    int* n_blocks, int* pos);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
