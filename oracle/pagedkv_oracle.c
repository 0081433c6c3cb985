/*
 * pagedkv_oracle.c -- CPU oracle for the paged-KV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file restates, in plain C, what the
 * reference's candle `engine = "paged"` path computes, so that the HIP
 * kernels of libpagedkv can be checked against it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it, and only
 * as the checker or as the timed CPU baseline -- never as a product path.
 *
 * Reference files restated (paths relative to the reference repository):
 *   crates/ai-engine-candle/src/paged/attention.rs   (KvPool, build_mask, sdpa)
 *   crates/ai-engine-candle/src/paged/transformer.rs (decode/prefill slices)
 * The reference's arithmetic runs inside candle-core/candle-nn 0.10.2 and
 * gemm 0.19.0 (Cargo.lock:1220-1223,1276-1279,3037-3040), which are not in
 * the reference tree; their published semantics are restated (row-major
 * matmul in f32, softmax_last_dim = exp(x - max) / sum, affine scale).
 * Summation order inside gemm is not reproducible here, so the f32
 * restatements agree with the reference to rounding, and attention parity
 * is a tolerance check (bit-exact only for the byte-moving functions).
 *
 * How each function is pinned (tests/test_oracle.py):
 *   orc_build_mask        - the reference's own KAT (attention.rs:142-156).
 *   orc_kv_write/gather   - closed form (slot = blocks[p/bs]*bs + p%bs) and
 *                           the "no other byte changes" invariant.
 *   orc_sdpa_f32          - torch.nn.functional.scaled_dot_product_attention
 *                           in float64 (independent library routine), special
 *                           cases (one key -> that V row; equal keys -> mean V;
 *                           dominant key -> its V row), mutation checks.
 *   orc_decode_step_f32   - equals orc_paged_attention_f64 on ragged inputs
 *                           (padding invariance) and orc_sdpa_f32 on the
 *                           gathered inputs; orc_decode_step_faithful_f32
 *                           gives the same bits (it only adds the copies).
 *   orc_prefill_*         - reduces to the reference prefill mask (P = 0), to
 *                           decode (one query), chunk-split invariance, and
 *                           brute-force torch float64 on tiny inputs.
 *   orc_copy/compact      - closed-form out-of-place memcpy.
 *   orc_rope_table        - the reference's KAT (rope.rs:49-63: gathered rows
 *                           equal table rows), float64 restatement of
 *                           p * base^(-2i/d) within 1 ulp, cos^2 + sin^2 = 1,
 *                           position 0 = (1, 0).
 *   orc_rope_apply        - identity at position 0, pairwise norm
 *                           preservation, rotation composition, relative-
 *                           position invariance of q.k, float64 rotation.
 *   orc_sample/argmax     - the reference's four KATs (ai-engine-runtime
 *                           tests/sample.rs), closed forms (uniform logits
 *                           pick floor(r * V), two-token logistic, top-k and
 *                           top-p renormalisation), first-maximum and NaN
 *                           rules of argmax.
 *   orc_expf_glibc        - the device restatement of glibc's expf (what the
 *                           exact sampler uses), checked here against the
 *                           host libm's expf on every float <= 0
 *                           (orc_expf_mismatches).
 *   orc_chacha_block      - the public ChaCha20 and ChaCha12 all-zero key
 *                           test vectors; orc_pcg32_output - the pcg32
 *                           reference demo sequence (initstate 42, initseq
 *                           54).  orc_seed_from_u64's wiring (increment,
 *                           advance before output) and the f32 conversion
 *                           follow the crates' published source and are
 *                           otherwise unpinned.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_F32 0
#define ORC_F16 1
#define ORC_BF16 2

/* ------------------------------------------------------------------------ */
/* dtype helpers: exact widening of f16/bf16 to f32                          */
/* ------------------------------------------------------------------------ */
static inline float orc_bf16_to_f32(uint16_t h) {
    uint32_t u = ((uint32_t)h) << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    uint32_t u;
    if (exp == 0) {
        if (man == 0) {
            u = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while ((man & 0x400) == 0);
            man &= 0x3ff;
            u = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1f) {
        u = sign | 0x7f800000u | (man << 13);
    } else {
        u = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static inline float orc_load(const void* base, int dtype, size_t i) {
    if (dtype == ORC_F32) return ((const float*)base)[i];
    uint16_t h = ((const uint16_t*)base)[i];
    return dtype == ORC_BF16 ? orc_bf16_to_f32(h) : orc_f16_to_f32(h);
}

static inline size_t orc_esize(int dtype) { return dtype == ORC_F32 ? 4 : 2; }

/* Widen n elements of `dtype` to f32 (exact). */
void orc_widen(const void* src, int dtype, size_t n, float* dst) {
    for (size_t i = 0; i < n; i++) dst[i] = orc_load(src, dtype, i);
}

/* ------------------------------------------------------------------------ */
/* KvPool::write (attention.rs:57-83): per new token i, locate(start_pos+i)  */
/* -> (blocks[pos/bs], pos%bs) (block_table.rs:55-58), then the row          */
/* [block, slot, :, :] of K and V is replaced by k[i], v[i].  The reference  */
/* does it with a functional slice_assign; the stored values are the same.   */
/* Returns -1 if a position is beyond the table (the reference panics).      */
/* ------------------------------------------------------------------------ */
int orc_kv_write(void* k_pool, void* v_pool, size_t elem_bytes, size_t bs,
                 size_t n_kv, size_t hd, const uint32_t* blocks,
                 size_t n_table_blocks, size_t start_pos, const void* k,
                 const void* v, size_t n_new) {
    const size_t row = n_kv * hd * elem_bytes;
    for (size_t i = 0; i < n_new; i++) {
        size_t pos = start_pos + i;
        size_t bi = pos / bs;
        if (bi >= n_table_blocks) return -1;
        size_t slot = (size_t)blocks[bi] * bs + pos % bs;
        memcpy((char*)k_pool + slot * row, (const char*)k + i * row, row);
        memcpy((char*)v_pool + slot * row, (const char*)v + i * row, row);
    }
    return 0;
}

/* KvPool::gather_seq (attention.rs:85-97): idx[p] = blocks[p/bs]*bs + p%bs,
 * index_select on the pool flattened to (N*bs, n_kv, hd). */
int orc_gather_seq(const void* k_pool, const void* v_pool, size_t elem_bytes,
                   size_t bs, size_t n_kv, size_t hd, const uint32_t* blocks,
                   size_t n_table_blocks, size_t len, void* out_k,
                   void* out_v) {
    const size_t row = n_kv * hd * elem_bytes;
    for (size_t p = 0; p < len; p++) {
        size_t bi = p / bs;
        if (bi >= n_table_blocks) return -1;
        size_t idx = (size_t)blocks[bi] * bs + p % bs;
        memcpy((char*)out_k + p * row, (const char*)k_pool + idx * row, row);
        memcpy((char*)out_v + p * row, (const char*)v_pool + idx * row, row);
    }
    return 0;
}

/* build_mask (attention.rs:11-28): (batch, 1, 1, kv_len) additive mask,
 * -inf where k >= seq_lens[b] or k > q_positions[b], else 0. */
void orc_build_mask(const int64_t* seq_lens, const int64_t* q_positions,
                    size_t batch, size_t kv_len, float* out) {
    for (size_t b = 0; b < batch; b++)
        for (size_t k = 0; k < kv_len; k++)
            out[b * kv_len + k] =
                ((int64_t)k >= seq_lens[b] || (int64_t)k > q_positions[b])
                    ? -INFINITY
                    : 0.0f;
}

/* candle_nn::ops::softmax_last_dim on one row: max, exp(x - max), sum,
 * divide (published candle-nn 0.10.2 CPU semantics). */
static void orc_softmax_row_f32(float* x, size_t n) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; i++) mx = x[i] > mx ? x[i] : mx;
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - mx);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

/* sdpa (attention.rs:100-126) with repeat_kv (:128-136), all in f32:
 *   q: (B, H, Lq, hd); k, v: (B, KVH, kv, hd); mask: (B, 1, Lq, kv)
 *   query head h reads kv head h / (H / KVH) (consecutive repeat);
 *   att = (q @ k^T) * scale; att += mask; softmax over kv; out = att @ v;
 *   result (B, Lq, H*hd), element [b, i, h*hd + d] (:124-125). */
void orc_sdpa_f32(const float* q, const float* k, const float* v,
                  const float* mask, size_t B, size_t H, size_t KVH,
                  size_t Lq, size_t kv, size_t hd, float scale, float* out) {
    size_t rep = H / KVH;
    float* att = (float*)malloc(sizeof(float) * (kv ? kv : 1));
    for (size_t b = 0; b < B; b++)
        for (size_t h = 0; h < H; h++) {
            size_t g = h / rep;
            const float* kb = k + (b * KVH + g) * kv * hd;
            const float* vb = v + (b * KVH + g) * kv * hd;
            for (size_t i = 0; i < Lq; i++) {
                const float* qi = q + ((b * H + h) * Lq + i) * hd;
                const float* mi = mask + (b * Lq + i) * kv;
                for (size_t j = 0; j < kv; j++) {
                    float s = 0.0f;
                    for (size_t d = 0; d < hd; d++) s += qi[d] * kb[j * hd + d];
                    att[j] = s * scale + mi[j];
                }
                orc_softmax_row_f32(att, kv);
                float* o = out + (b * Lq + i) * H * hd + h * hd;
                for (size_t d = 0; d < hd; d++) {
                    float acc = 0.0f;
                    for (size_t j = 0; j < kv; j++) acc += att[j] * vb[j * hd + d];
                    o[d] = acc;
                }
            }
        }
    free(att);
}

/* Transformer::decode_step, attention slice (transformer.rs:271-292), in f32
 * on f32 pools (the reference's KvPool dtype):
 *   for each row b: write k_new[b], v_new[b] at pos seq_lens[b] (:276), then
 *   gather seq_lens[b]+1 rows (:277), zero-pad to kv_len = max(seq_lens)+1
 *   (:241,:278-281); stack to (B, KVH, kv_len, hd) (:285-286); mask with
 *   valid_lens = seq_lens+1 and positions (:289-290); sdpa (:292).
 * k_pool/v_pool are modified (the append).  tables: [B][max_nb] uint32.
 * Returns -1 on a position beyond a table. */
int orc_decode_step_f32(float* k_pool, float* v_pool, size_t bs, size_t KVH,
                        size_t hd, const uint32_t* tables, size_t max_nb,
                        const int64_t* seq_lens, const int64_t* positions,
                        const float* q, const float* k_new,
                        const float* v_new, size_t B, size_t H, float scale,
                        float* out) {
    size_t kv_len = 0;
    for (size_t b = 0; b < B; b++)
        if ((size_t)seq_lens[b] + 1 > kv_len) kv_len = (size_t)seq_lens[b] + 1;
    const size_t row = KVH * hd;
    float* k_all = (float*)calloc(B * KVH * kv_len * hd, sizeof(float));
    float* v_all = (float*)calloc(B * KVH * kv_len * hd, sizeof(float));
    float* gk = (float*)malloc(sizeof(float) * kv_len * row);
    float* gv = (float*)malloc(sizeof(float) * kv_len * row);
    int rc = 0;
    for (size_t b = 0; b < B && rc == 0; b++) {
        const uint32_t* tb = tables + b * max_nb;
        rc = orc_kv_write(k_pool, v_pool, 4, bs, KVH, hd, tb, max_nb,
                          (size_t)seq_lens[b], k_new + b * row,
                          v_new + b * row, 1);
        if (rc) break;
        size_t len = (size_t)seq_lens[b] + 1;
        rc = orc_gather_seq(k_pool, v_pool, 4, bs, KVH, hd, tb, max_nb, len,
                            gk, gv);
        /* pad_with_zeros + cat + transpose(1,2): (len, KVH, hd) -> (KVH, kv_len, hd) */
        for (size_t p = 0; p < len; p++)
            for (size_t g = 0; g < KVH; g++)
                for (size_t d = 0; d < hd; d++) {
                    size_t dst = ((b * KVH + g) * kv_len + p) * hd + d;
                    k_all[dst] = gk[(p * KVH + g) * hd + d];
                    v_all[dst] = gv[(p * KVH + g) * hd + d];
                }
    }
    if (rc == 0) {
        int64_t* valid = (int64_t*)malloc(sizeof(int64_t) * B);
        for (size_t b = 0; b < B; b++) valid[b] = seq_lens[b] + 1;
        float* mask = (float*)malloc(sizeof(float) * B * kv_len);
        orc_build_mask(valid, positions, B, kv_len, mask);
        orc_sdpa_f32(q, k_all, v_all, mask, B, H, KVH, 1, kv_len, hd, scale,
                     out);
        free(mask);
        free(valid);
    }
    free(k_all);
    free(v_all);
    free(gk);
    free(gv);
    return rc;
}

/* The reference's cost model (CPU baseline variant "reference-faithful"):
 * KvPool::write assigns each row with candle's slice_assign, which builds a
 * new full pool tensor (attention.rs:73-80), so every appended row first
 * copies the whole K pool and the whole V pool.  The copies go to a second
 * buffer that then becomes the pool; the attention is orc_decode_step_f32's
 * (write -> gather -> pad -> mask -> sdpa).  The pools hold the result. */
int orc_decode_step_faithful_f32(float* k_pool, float* v_pool, size_t num_blocks,
                                 size_t bs, size_t KVH, size_t hd,
                                 const uint32_t* tables, size_t max_nb,
                                 const int64_t* seq_lens, const int64_t* positions,
                                 const float* q, const float* k_new,
                                 const float* v_new, size_t B, size_t H,
                                 float scale, float* out) {
    const size_t bytes = num_blocks * bs * KVH * hd * sizeof(float);
    float* kbuf = (float*)malloc(bytes);
    float* vbuf = (float*)malloc(bytes);
    if (!kbuf || !vbuf) {
        free(kbuf);
        free(vbuf);
        return -2;
    }
    float *kc = k_pool, *vc = v_pool, *ko = kbuf, *vo = vbuf;
    const size_t row = KVH * hd;
    int rc = 0;
    for (size_t b = 0; b < B && rc == 0; b++) {
        float* t;
        memcpy(ko, kc, bytes);
        t = kc; kc = ko; ko = t;
        memcpy(vo, vc, bytes);
        t = vc; vc = vo; vo = t;
        rc = orc_kv_write(kc, vc, 4, bs, KVH, hd, tables + b * max_nb, max_nb,
                          (size_t)seq_lens[b], k_new + b * row, v_new + b * row, 1);
    }
    if (rc == 0)
        rc = orc_decode_step_f32(kc, vc, bs, KVH, hd, tables, max_nb, seq_lens, positions,
                                 q, k_new, v_new, B, H, scale, out);
    if (kc != k_pool) memcpy(k_pool, kc, bytes);
    if (vc != v_pool) memcpy(v_pool, vc, bytes);
    free(kbuf);
    free(vbuf);
    return rc;
}

/* The reference's cost model for a prompt chunk (CPU baseline variant
 * "reference-faithful"): C tokens at positions prior .. prior + C - 1 of one
 * sequence.  prefill_seq stores every token with KvPool::write
 * (transformer.rs:173-177), whose slice_assign builds a new full pool per
 * token (attention.rs:73-80): the first n_copies tokens copy the whole K and
 * V pool before their row is written (the rest are written in place, so a
 * bounded sample can time the copies apart from the attention).  The
 * attention is dense as in prefill_seq (transformer.rs:139-148,180-196):
 * the sequence's prior + C rows gathered from the pool (gather_seq,
 * attention.rs:85-97), a (C, prior + C) additive mask with -inf at key
 * j > prior + i, and sdpa over every key of every query row.
 *   q: (C, H, hd); k_new, v_new: (C, KVH, hd); out: (C, H * hd).
 * Returns -1 on a position beyond the table, -2 on allocation failure. */
int orc_prefill_chunk_faithful_f32(float* k_pool, float* v_pool, size_t num_blocks,
                                   size_t bs, size_t KVH, size_t hd, const uint32_t* table,
                                   size_t n_table_blocks, size_t prior, size_t C,
                                   size_t n_copies, const float* q, const float* k_new,
                                   const float* v_new, size_t H, float scale, float* out) {
    const size_t bytes = num_blocks * bs * KVH * hd * sizeof(float);
    const size_t row = KVH * hd, n = prior + C;
    float* kbuf = n_copies ? (float*)malloc(bytes) : NULL;
    float* vbuf = n_copies ? (float*)malloc(bytes) : NULL;
    float* gk = (float*)malloc(sizeof(float) * (n ? n : 1) * row);
    float* gv = (float*)malloc(sizeof(float) * (n ? n : 1) * row);
    float* kt = (float*)malloc(sizeof(float) * (n ? n : 1) * row);
    float* vt = (float*)malloc(sizeof(float) * (n ? n : 1) * row);
    float* qt = (float*)malloc(sizeof(float) * (C ? C : 1) * H * hd);
    float* mask = (float*)malloc(sizeof(float) * (C ? C : 1) * (n ? n : 1));
    int rc = 0;
    if ((n_copies && (!kbuf || !vbuf)) || !gk || !gv || !kt || !vt || !qt || !mask) rc = -2;
    float *kc = k_pool, *vc = v_pool, *ko = kbuf, *vo = vbuf;
    for (size_t i = 0; i < C && rc == 0; i++) {
        if (i < n_copies) {
            float* t;
            memcpy(ko, kc, bytes);
            t = kc; kc = ko; ko = t;
            memcpy(vo, vc, bytes);
            t = vc; vc = vo; vo = t;
        }
        rc = orc_kv_write(kc, vc, 4, bs, KVH, hd, table, n_table_blocks, prior + i,
                          k_new + i * row, v_new + i * row, 1);
    }
    if (rc == 0) rc = orc_gather_seq(kc, vc, 4, bs, KVH, hd, table, n_table_blocks, n, gk, gv);
    if (rc == 0) {
        /* (n, KVH, hd) -> (KVH, n, hd); q (C, H, hd) -> (H, C, hd) */
        for (size_t p = 0; p < n; p++)
            for (size_t g = 0; g < KVH; g++)
                for (size_t d = 0; d < hd; d++) {
                    kt[(g * n + p) * hd + d] = gk[(p * KVH + g) * hd + d];
                    vt[(g * n + p) * hd + d] = gv[(p * KVH + g) * hd + d];
                }
        for (size_t i = 0; i < C; i++)
            for (size_t h = 0; h < H; h++)
                memcpy(qt + (h * C + i) * hd, q + (i * H + h) * hd, sizeof(float) * hd);
        for (size_t i = 0; i < C; i++)
            for (size_t j = 0; j < n; j++) mask[i * n + j] = j > prior + i ? -INFINITY : 0.0f;
        orc_sdpa_f32(qt, kt, vt, mask, 1, H, KVH, C, n, hd, scale, out);
    }
    if (kc != k_pool) memcpy(k_pool, kc, bytes);
    if (vc != v_pool) memcpy(v_pool, vc, bytes);
    free(kbuf);
    free(vbuf);
    free(gk);
    free(gv);
    free(kt);
    free(vt);
    free(qt);
    free(mask);
    return rc;
}

/* Closed form in fp64: paged decode attention straight off the block tables,
 * ragged (no padding).  For every (b, h): keys p = 0..ctx_lens[b]-1 at slot
 * tables[b][p/bs]*bs + p%bs, kv head h / (H/KVH), s_p = scale * q.k_p,
 * out = sum_p softmax(s)_p v_p.  Pools are element type `dtype` (widened
 * exactly).  ctx_lens[b] == 0 gives a zero row. */
void orc_paged_attention_f64(const void* k_pool, const void* v_pool,
                             int dtype, size_t bs, size_t KVH, size_t hd,
                             const uint32_t* tables, size_t max_nb,
                             const int64_t* ctx_lens, const float* q,
                             size_t B, size_t H, double scale, double* out) {
    size_t rep = H / KVH;
    for (size_t b = 0; b < B; b++) {
        size_t n = (size_t)ctx_lens[b];
        double* s = (double*)malloc(sizeof(double) * (n ? n : 1));
        for (size_t h = 0; h < H; h++) {
            size_t g = h / rep;
            const float* qh = q + (b * H + h) * hd;
            double* o = out + (b * H + h) * hd;
            for (size_t d = 0; d < hd; d++) o[d] = 0.0;
            if (n == 0) continue;
            double mx = -INFINITY;
            for (size_t p = 0; p < n; p++) {
                size_t slot = (size_t)tables[b * max_nb + p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                double acc = 0.0;
                for (size_t d = 0; d < hd; d++)
                    acc += (double)qh[d] * (double)orc_load(k_pool, dtype, base + d);
                s[p] = acc * scale;
                if (s[p] > mx) mx = s[p];
            }
            double sum = 0.0;
            for (size_t p = 0; p < n; p++) {
                s[p] = exp(s[p] - mx);
                sum += s[p];
            }
            for (size_t p = 0; p < n; p++) {
                size_t slot = (size_t)tables[b * max_nb + p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                double w = s[p] / sum;
                for (size_t d = 0; d < hd; d++)
                    o[d] += w * (double)orc_load(v_pool, dtype, base + d);
            }
        }
        free(s);
    }
}

/* Closed form in fp64 for chunked prefill with a prior context: sequence s
 * has ql = cu_q[s+1]-cu_q[s] queries whose K/V are already stored; query i
 * is at position ctx_lens[s]-ql+i and attends keys 0..that position.  With
 * an empty prior context this is prefill_seq's causal attention
 * (transformer.rs:139-148,191-196: mask j > i -> -inf). */
void orc_prefill_attention_f64(const void* k_pool, const void* v_pool,
                               int dtype, size_t bs, size_t KVH, size_t hd,
                               const uint32_t* tables, size_t max_nb,
                               const int64_t* cu_q, const int64_t* ctx_lens,
                               size_t n_seqs, const float* q, size_t H,
                               double scale, double* out) {
    size_t rep = H / KVH;
    for (size_t sq = 0; sq < n_seqs; sq++) {
        size_t q0 = (size_t)cu_q[sq], ql = (size_t)(cu_q[sq + 1] - cu_q[sq]);
        size_t n = (size_t)ctx_lens[sq];
        const uint32_t* tb = tables + sq * max_nb;
        double* s = (double*)malloc(sizeof(double) * (n ? n : 1));
        for (size_t i = 0; i < ql; i++) {
            long long posi = (long long)n - (long long)ql + (long long)i;
            for (size_t h = 0; h < H; h++) {
                size_t g = h / rep;
                const float* qh = q + ((q0 + i) * H + h) * hd;
                double* o = out + ((q0 + i) * H + h) * hd;
                for (size_t d = 0; d < hd; d++) o[d] = 0.0;
                if (posi < 0) continue;
                size_t nk = (size_t)posi + 1;
                double mx = -INFINITY;
                for (size_t p = 0; p < nk; p++) {
                    size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                    size_t base = (slot * KVH + g) * hd;
                    double acc = 0.0;
                    for (size_t d = 0; d < hd; d++)
                        acc += (double)qh[d] * (double)orc_load(k_pool, dtype, base + d);
                    s[p] = acc * scale;
                    if (s[p] > mx) mx = s[p];
                }
                double sum = 0.0;
                for (size_t p = 0; p < nk; p++) {
                    s[p] = exp(s[p] - mx);
                    sum += s[p];
                }
                for (size_t p = 0; p < nk; p++) {
                    size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                    size_t base = (slot * KVH + g) * hd;
                    double w = s[p] / sum;
                    for (size_t d = 0; d < hd; d++)
                        o[d] += w * (double)orc_load(v_pool, dtype, base + d);
                }
            }
        }
        free(s);
    }
}

/* prefill_seq attention slice (transformer.rs:139-148,179-196) in f32 for
 * one sequence of N tokens with in-register K/V:
 *   q: (H, N, hd); k, v: (KVH, N, hd); causal mask j > i -> -inf;
 *   GQA expand; att = (q @ k^T) * scale + mask; softmax; att @ v;
 *   out (N, H*hd) (:196). */
void orc_prefill_seq_f32(const float* q, const float* k, const float* v,
                         size_t H, size_t KVH, size_t N, size_t hd,
                         float scale, float* out) {
    float* mask = (float*)malloc(sizeof(float) * N * N);
    for (size_t i = 0; i < N; i++)
        for (size_t j = 0; j < N; j++) mask[i * N + j] = j > i ? -INFINITY : 0.0f;
    orc_sdpa_f32(q, k, v, mask, 1, H, KVH, N, N, hd, scale, out);
    free(mask);
}

/* Block copy over every layer and K/V: block dst[i] <- block src[i].
 * layer_bytes = one layer's K (or V) pool size; block_bytes = one block.
 * The pool buffer holds [n_layers][2][num_blocks * block_bytes]. */
void orc_copy_blocks(void* pool, size_t n_layers, size_t layer_bytes,
                     size_t block_bytes, const int32_t* src,
                     const int32_t* dst, size_t n) {
    for (size_t l = 0; l < n_layers * 2; l++) {
        char* base = (char*)pool + l * layer_bytes;
        for (size_t i = 0; i < n; i++)
            memmove(base + (size_t)dst[i] * block_bytes,
                    base + (size_t)src[i] * block_bytes, block_bytes);
    }
}

/* Compaction closed form: new[dst[i]] = old[src[i]] for all i, computed out
 * of place (a full copy of the old pool), every other block unchanged. */
int orc_compact(void* pool, size_t n_layers, size_t layer_bytes,
                size_t block_bytes, const int32_t* src, const int32_t* dst,
                size_t n) {
    char* old = (char*)malloc(layer_bytes);
    if (!old) return -1;
    for (size_t l = 0; l < n_layers * 2; l++) {
        char* base = (char*)pool + l * layer_bytes;
        memcpy(old, base, layer_bytes);
        for (size_t i = 0; i < n; i++)
            memcpy(base + (size_t)dst[i] * block_bytes,
                   old + (size_t)src[i] * block_bytes, block_bytes);
    }
    free(old);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* CPU baseline: the reference's decode attention math (write at seq_lens,   */
/* attend seq_lens+1 keys, scale after the dot product, max/exp/sum/divide   */
/* softmax, P.V) done in place on the pool in its storage dtype, ragged      */
/* lengths, OpenMP over (sequence, kv head).  This is the reference-math     */
/* in-place variant timed by bench.py; it is not the faithful per-append     */
/* full-pool copy of slice_assign (attention.rs:73-80), which is infeasible  */
/* at the benchmark sizes.                                                   */
/* ------------------------------------------------------------------------ */
void orc_decode_inplace(void* k_pool, void* v_pool, int dtype, size_t bs,
                        size_t KVH, size_t hd, const int32_t* tables,
                        size_t max_nb, const int32_t* ctx_lens,
                        const void* q, const void* k_new, const void* v_new,
                        size_t B, size_t H, float scale, float* out,
                        int n_threads) {
    const size_t es = orc_esize(dtype);
    const size_t rep = H / KVH;
    /* append first (transformer.rs:276), bit-exact row copy */
    for (size_t b = 0; b < B; b++) {
        if (ctx_lens[b] <= 0 || !k_new) continue;
        size_t pos = (size_t)ctx_lens[b] - 1;
        size_t slot = (size_t)tables[b * max_nb + pos / bs] * bs + pos % bs;
        memcpy((char*)k_pool + slot * KVH * hd * es,
               (const char*)k_new + b * KVH * hd * es, KVH * hd * es);
        memcpy((char*)v_pool + slot * KVH * hd * es,
               (const char*)v_new + b * KVH * hd * es, KVH * hd * es);
    }
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel
#endif
    {
        size_t maxn = 0;
        for (size_t b = 0; b < B; b++)
            if ((size_t)ctx_lens[b] > maxn) maxn = (size_t)ctx_lens[b];
        float* s = (float*)malloc(sizeof(float) * rep * (maxn ? maxn : 1));
        float* qf = (float*)malloc(sizeof(float) * rep * hd);
        float* kf = (float*)malloc(sizeof(float) * hd);
        float* acc = (float*)malloc(sizeof(float) * rep * hd);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (long long w = 0; w < (long long)(B * KVH); w++) {
            size_t b = (size_t)w / KVH, g = (size_t)w % KVH;
            size_t n = (size_t)ctx_lens[b];
            const int32_t* tb = tables + b * max_nb;
            for (size_t r = 0; r < rep; r++)
                for (size_t d = 0; d < hd; d++)
                    qf[r * hd + d] = orc_load(q, dtype, (b * H + g * rep + r) * hd + d);
            for (size_t p = 0; p < n; p++) {
                size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                for (size_t d = 0; d < hd; d++) kf[d] = orc_load(k_pool, dtype, base + d);
                for (size_t r = 0; r < rep; r++) {
                    float dot = 0.0f;
                    for (size_t d = 0; d < hd; d++) dot += qf[r * hd + d] * kf[d];
                    s[r * n + p] = dot * scale;
                }
            }
            for (size_t r = 0; r < rep; r++) {
                float mx = -INFINITY, sum = 0.0f;
                for (size_t p = 0; p < n; p++) mx = s[r * n + p] > mx ? s[r * n + p] : mx;
                for (size_t p = 0; p < n; p++) {
                    s[r * n + p] = expf(s[r * n + p] - mx);
                    sum += s[r * n + p];
                }
                for (size_t p = 0; p < n; p++) s[r * n + p] /= sum;
            }
            for (size_t i = 0; i < rep * hd; i++) acc[i] = 0.0f;
            for (size_t p = 0; p < n; p++) {
                size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                for (size_t d = 0; d < hd; d++) kf[d] = orc_load(v_pool, dtype, base + d);
                for (size_t r = 0; r < rep; r++) {
                    float w = s[r * n + p];
                    for (size_t d = 0; d < hd; d++) acc[r * hd + d] += w * kf[d];
                }
            }
            for (size_t r = 0; r < rep; r++)
                memcpy(out + (b * H + g * rep + r) * hd, acc + r * hd, sizeof(float) * hd);
        }
        free(s);
        free(qf);
        free(kf);
        free(acc);
    }
}

/* CPU baseline for chunked prefill: the reference's prefill_seq attention
 * math (transformer.rs:139-148,179-196: per-token K/V store, then
 * S = q.k^T * scale with the causal mask, max/exp/sum/divide softmax, P.V,
 * all f32) in place on the pool, extended to a prior context: sequence s's
 * chunk of ql = cu_q[s+1]-cu_q[s] tokens sits at positions
 * ctx_lens[s]-ql .. ctx_lens[s]-1.  k_new/v_new (T, KVH, hd) are stored first
 * when non-NULL.  OpenMP over (sequence, query head, 16-query row block). */
void orc_prefill_inplace(void* k_pool, void* v_pool, int dtype, size_t bs,
                         size_t KVH, size_t hd, const int32_t* tables,
                         size_t max_nb, const int32_t* cu_q,
                         const int32_t* ctx_lens, size_t n_seqs, const void* q,
                         const void* k_new, const void* v_new, size_t H,
                         float scale, float* out, int n_threads) {
    const size_t es = orc_esize(dtype);
    const size_t rep = H / KVH;
    const size_t RB = 16;
    if (k_new) {
        for (size_t sq = 0; sq < n_seqs; sq++) {
            size_t q0 = (size_t)cu_q[sq], ql = (size_t)(cu_q[sq + 1] - cu_q[sq]);
            size_t p0 = (size_t)ctx_lens[sq] - ql;
            for (size_t i = 0; i < ql; i++) {
                size_t pos = p0 + i;
                size_t slot = (size_t)tables[sq * max_nb + pos / bs] * bs + pos % bs;
                memcpy((char*)k_pool + slot * KVH * hd * es,
                       (const char*)k_new + (q0 + i) * KVH * hd * es, KVH * hd * es);
                memcpy((char*)v_pool + slot * KVH * hd * es,
                       (const char*)v_new + (q0 + i) * KVH * hd * es, KVH * hd * es);
            }
        }
    }
    size_t n_work = 0, maxn = 1;
    for (size_t sq = 0; sq < n_seqs; sq++) {
        size_t ql = (size_t)(cu_q[sq + 1] - cu_q[sq]);
        n_work += H * ((ql + RB - 1) / RB);
        if ((size_t)ctx_lens[sq] > maxn) maxn = (size_t)ctx_lens[sq];
    }
#ifdef _OPENMP
    if (n_threads > 0) omp_set_num_threads(n_threads);
#pragma omp parallel
#endif
    {
        float* s = (float*)malloc(sizeof(float) * RB * maxn);
        float* qf = (float*)malloc(sizeof(float) * RB * hd);
        float* kf = (float*)malloc(sizeof(float) * hd);
        float* acc = (float*)malloc(sizeof(float) * RB * hd);
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (long long w = 0; w < (long long)n_work; w++) {
            /* locate (sequence, head, row block) of work item w */
            size_t rem = (size_t)w, sq = 0, nrb = 0;
            for (; sq < n_seqs; sq++) {
                size_t ql = (size_t)(cu_q[sq + 1] - cu_q[sq]);
                nrb = (ql + RB - 1) / RB;
                if (rem < H * nrb) break;
                rem -= H * nrb;
            }
            size_t h = rem / nrb, rb = rem % nrb, g = h / rep;
            size_t q0 = (size_t)cu_q[sq], ql = (size_t)(cu_q[sq + 1] - cu_q[sq]);
            size_t n = (size_t)ctx_lens[sq], p0 = n - ql;
            size_t i0 = rb * RB, ni = ql - i0 < RB ? ql - i0 : RB;
            size_t nk = p0 + i0 + ni; /* keys the block's last row attends */
            const int32_t* tb = tables + sq * max_nb;
            for (size_t r = 0; r < ni; r++)
                for (size_t d = 0; d < hd; d++)
                    qf[r * hd + d] = orc_load(q, dtype, ((q0 + i0 + r) * H + h) * hd + d);
            for (size_t p = 0; p < nk; p++) {
                size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                for (size_t d = 0; d < hd; d++) kf[d] = orc_load(k_pool, dtype, base + d);
                for (size_t r = 0; r < ni; r++) {
                    float dot = 0.0f;
                    for (size_t d = 0; d < hd; d++) dot += qf[r * hd + d] * kf[d];
                    /* causal mask (transformer.rs:139-148): key p > query position -> -inf */
                    s[r * maxn + p] = p > p0 + i0 + r ? -INFINITY : dot * scale;
                }
            }
            for (size_t r = 0; r < ni; r++) {
                float mx = -INFINITY, sum = 0.0f;
                float* sr = s + r * maxn;
                for (size_t p = 0; p < nk; p++) mx = sr[p] > mx ? sr[p] : mx;
                for (size_t p = 0; p < nk; p++) {
                    sr[p] = expf(sr[p] - mx);
                    sum += sr[p];
                }
                for (size_t p = 0; p < nk; p++) sr[p] /= sum;
            }
            for (size_t i = 0; i < ni * hd; i++) acc[i] = 0.0f;
            for (size_t p = 0; p < nk; p++) {
                size_t slot = (size_t)tb[p / bs] * bs + p % bs;
                size_t base = (slot * KVH + g) * hd;
                for (size_t d = 0; d < hd; d++) kf[d] = orc_load(v_pool, dtype, base + d);
                for (size_t r = 0; r < ni; r++) {
                    float wt = s[r * maxn + p];
                    for (size_t d = 0; d < hd; d++) acc[r * hd + d] += wt * kf[d];
                }
            }
            for (size_t r = 0; r < ni; r++)
                memcpy(out + ((q0 + i0 + r) * H + h) * hd, acc + r * hd, sizeof(float) * hd);
        }
        free(s);
        free(qf);
        free(kf);
        free(acc);
    }
}

/* Number of OpenMP threads the baseline uses for a requested count. */
/* ------------------------------------------------------------------------ */
/* rotary position embedding (crates/ai-engine-candle/src/paged/rope.rs)      */
/* ------------------------------------------------------------------------ */
/* Rope::new (rope.rs:14-23): theta_i = 1 / base^(2 i / dim) in f32 (powf),
 * freqs[p][i] = (float)p * theta_i (the matmul of a (max_seq, 1) column by a
 * (1, dim/2) row: one product per element), cos/sin in f32 (libm). */
void orc_rope_table(size_t rope_dim, float base, size_t max_seq, float* cos_t,
                    float* sin_t) {
    size_t half = rope_dim / 2;
    for (size_t i = 0; i < half; i++) {
        float theta = 1.0f / powf(base, 2.0f * (float)i / (float)rope_dim);
        for (size_t p = 0; p < max_seq; p++) {
            float f = (float)p * theta;
            cos_t[p * half + i] = cosf(f);
            sin_t[p * half + i] = sinf(f);
        }
    }
}

/* apply_rope (rope.rs:38-42) = candle_nn::rotary_emb::rope, rotate-half:
 * for the halves x1 = x[i], x2 = x[i + d/2] of every (token, head) row,
 * out[i] = x1 cos - x2 sin, out[i + d/2] = x1 sin + x2 cos, in f32 with each
 * product rounded (no fused multiply-add; the Makefile turns contraction
 * off).  Row t uses its own position pos[t] (transformer.rs:252-269). */
void orc_rope_apply(const float* x, float* out, size_t n_tokens, size_t n_head,
                    size_t d, const float* cos_t, const float* sin_t,
                    const int32_t* pos) {
    size_t half = d / 2;
    for (size_t t = 0; t < n_tokens; t++) {
        const float* c = cos_t + (size_t)pos[t] * half;
        const float* s = sin_t + (size_t)pos[t] * half;
        for (size_t h = 0; h < n_head; h++) {
            const float* xr = x + (t * n_head + h) * d;
            float* o = out + (t * n_head + h) * d;
            for (size_t i = 0; i < half; i++) {
                float x1 = xr[i], x2 = xr[i + half];
                float a = x1 * c[i], b = x2 * s[i];
                float e = x1 * s[i], f = x2 * c[i];
                o[i] = a - b;
                o[i + half] = e + f;
            }
        }
    }
}

int orc_threads(int requested) {
#ifdef _OPENMP
    if (requested > 0) return requested;
    return omp_get_max_threads();
#else
    (void)requested;
    return 1;
#endif
}

/* ------------------------------------------------------------------------ */
/* token selection: sample() and argmax() of                                */
/* crates/ai-engine-runtime/src/sample.rs:12-55, which the paged engine      */
/* calls per row with SamplingConfig {temperature, top_p: None, top_k: None, */
/* seed: 42} (crates/ai-engine-candle/src/paged/engine.rs:58-60,162,226).    */
/*                                                                           */
/* The draw r comes from rand 0.8.6 (Cargo.lock:5080-5083):                  */
/* StdRng::seed_from_u64(seed).gen::<f32>().  StdRng is ChaCha12 (rand_chacha */
/* 0.3.1); seed_from_u64 is rand_core 0.6.4's default: a PCG32 stream        */
/* (multiplier 6364136223846793005, increment 11634580027462260723, state    */
/* advanced before each output, XSH-RR output) fills the 32-byte key, eight  */
/* little-endian words; the block counter and stream start at 0; gen::<f32>  */
/* takes the first output word w and returns (w >> 8) * 2^-24.  None of      */
/* these crates is in the reference tree; their published algorithms are    */
/* restated here.                                                            */
/* ------------------------------------------------------------------------ */
static inline uint32_t orc_rotl32(uint32_t x, int n) { return (x << n) | (x >> (32 - n)); }

/* PCG32 XSH-RR output of a 64-bit state. */
uint32_t orc_pcg32_output(uint64_t state) {
    uint32_t xs = (uint32_t)(((state >> 18) ^ state) >> 27);
    uint32_t rot = (uint32_t)(state >> 59);
    return (xs >> rot) | (xs << ((32u - rot) & 31u));
}

/* One ChaCha block: constants, 8 key words, 64-bit counter, 64-bit stream. */
void orc_chacha_block(const uint32_t* key, uint64_t counter, uint64_t stream, int rounds,
                      uint32_t* out) {
    uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
    for (int i = 0; i < 8; ++i) s[4 + i] = key[i];
    s[12] = (uint32_t)counter;
    s[13] = (uint32_t)(counter >> 32);
    s[14] = (uint32_t)stream;
    s[15] = (uint32_t)(stream >> 32);
    uint32_t x[16];
    memcpy(x, s, sizeof x);
#define ORC_QR(a, b, c, d)                                   \
    x[a] += x[b]; x[d] = orc_rotl32(x[d] ^ x[a], 16);         \
    x[c] += x[d]; x[b] = orc_rotl32(x[b] ^ x[c], 12);         \
    x[a] += x[b]; x[d] = orc_rotl32(x[d] ^ x[a], 8);          \
    x[c] += x[d]; x[b] = orc_rotl32(x[b] ^ x[c], 7);
    for (int r = 0; r < rounds; r += 2) {
        ORC_QR(0, 4, 8, 12) ORC_QR(1, 5, 9, 13) ORC_QR(2, 6, 10, 14) ORC_QR(3, 7, 11, 15)
        ORC_QR(0, 5, 10, 15) ORC_QR(1, 6, 11, 12) ORC_QR(2, 7, 8, 13) ORC_QR(3, 4, 9, 14)
    }
#undef ORC_QR
    for (int i = 0; i < 16; ++i) out[i] = x[i] + s[i];
}

/* rand_core 0.6.4 SeedableRng::seed_from_u64 for a 32-byte seed. */
void orc_seed_from_u64(uint64_t state, uint32_t* key) {
    for (int i = 0; i < 8; ++i) {
        state = state * 6364136223846793005ull + 11634580027462260723ull;
        key[i] = orc_pcg32_output(state);
    }
}

/* StdRng::seed_from_u64(seed).gen::<f32>() (sample.rs:41-42). */
float orc_sample_draw(uint64_t seed) {
    uint32_t key[8], blk[16];
    orc_seed_from_u64(seed, key);
    orc_chacha_block(key, 0, 0, 12, blk);
    return (float)(blk[0] >> 8) * (1.0f / 16777216.0f);
}

/* argmax (sample.rs:50-55): fold from (0, -inf) keeping strictly greater
 * values, so the first maximum wins and NaN never does. */
int64_t orc_argmax(const float* x, size_t n) {
    size_t bi = 0;
    float bv = -INFINITY;
    for (size_t i = 0; i < n; ++i)
        if (x[i] > bv) { bi = i; bv = x[i]; }
    return (int64_t)bi;
}

static const float* orc_sort_keys;
/* sort_by(b.partial_cmp(a)) is a stable descending sort: equal values keep
 * index order, and -0.0 equals +0.0 (NaN inputs are not supported). */
static int orc_desc_cmp(const void* a, const void* b) {
    size_t i = *(const size_t*)a, j = *(const size_t*)b;
    float x = orc_sort_keys[i], y = orc_sort_keys[j];
    if (x > y) return -1;
    if (x < y) return 1;
    return i < j ? -1 : (i > j ? 1 : 0);
}

/* sample (sample.rs:12-48).  precise = 0: the reference's arithmetic, f32
 * throughout with libm expf and running sums in the sorted order.
 * precise = 1: the same steps on the same f32 values y and y - max, with
 * exp, the normalisation and the running sums in double -- the value the
 * f32 version approximates, used to separate the reference's rounding from
 * a wrong selection.  top_k <= 0 is None; has_top_p = 0 is None.  *margin
 * gets the distance of the decisive running sums from their thresholds (r,
 * and top_p when it cuts), in the mode's own arithmetic (0 when the
 * fallback to the last token is taken). */
int64_t orc_sample(const float* logits, size_t n, float temperature, int top_k, int has_top_p,
                   float top_p, uint64_t seed, int precise, double* margin) {
    if (margin) *margin = INFINITY;
    if (temperature == 0.0f || n <= 1) return orc_argmax(logits, n);
    float* y = malloc(n * sizeof(float));
    size_t* idx = malloc(n * sizeof(size_t));
    double* p = malloc(n * sizeof(double));
    for (size_t i = 0; i < n; ++i) { y[i] = logits[i] / temperature; idx[i] = i; }
    orc_sort_keys = y;
    qsort(idx, n, sizeof(size_t), orc_desc_cmp);
    size_t len = n;
    if (top_k > 0 && (size_t)top_k < len) len = (size_t)top_k;
    float max_x = y[idx[0]];
    /* f32 mode keeps every intermediate in float (each value rounded to
     * float on assignment); precise mode keeps doubles */
    double sum = 0.0;
    float sum32 = 0.0f;
    for (size_t i = 0; i < len; ++i) {
        float d = y[idx[i]] - max_x;
        if (precise) { p[i] = exp((double)d); sum += p[i]; }
        else { float e = expf(d); p[i] = e; sum32 += e; }
    }
    for (size_t i = 0; i < len; ++i) {
        if (precise) p[i] /= sum;
        else p[i] = (float)((float)p[i] / sum32);
    }
    double m = INFINITY;
    if (has_top_p) {
        double cum = 0.0;
        float cum32 = 0.0f;
        size_t cutoff = len;
        for (size_t i = 0; i < len; ++i) {
            double prev, now;
            if (precise) { prev = cum; cum += p[i]; now = cum; }
            else { prev = cum32; cum32 += (float)p[i]; now = cum32; }
            if (precise ? now >= (double)top_p : cum32 >= top_p) {
                cutoff = i + 1;
                double d1 = (double)top_p - prev, d2 = now - top_p;
                m = d1 < d2 ? d1 : d2;
                break;
            }
        }
        len = cutoff;
        double s = 0.0;
        float s32 = 0.0f;
        for (size_t i = 0; i < len; ++i) { s += p[i]; s32 += (float)p[i]; }
        for (size_t i = 0; i < len; ++i) {
            if (precise) p[i] /= s;
            else p[i] = (float)((float)p[i] / s32);
        }
    }
    float r = orc_sample_draw(seed);
    double acc = 0.0;
    float acc32 = 0.0f;
    int64_t tok = (int64_t)idx[len - 1];
    double mr = 0.0;
    for (size_t i = 0; i < len; ++i) {
        double prev, now;
        if (precise) { prev = acc; acc += p[i]; now = acc; }
        else { prev = acc32; acc32 += (float)p[i]; now = acc32; }
        if (precise ? (double)r <= now : r <= acc32) {
            tok = (int64_t)idx[i];
            double d1 = (double)r - prev, d2 = now - r;
            mr = d1 < d2 ? d1 : d2;
            break;
        }
    }
    if (margin) *margin = m < mr ? m : mr;
    free(y);
    free(idx);
    free(p);
    return tok;
}

/* ------------------------------------------------------------------------ */
/* expf.  The reference's f32::exp is the C library's expf on its host; on   */
/* x86-64 Linux that is glibc's (the algorithm of Arm's Optimized Routines,  */
/* glibc >= 2.28, built for FMA hardware).  orc_expf_host evaluates the      */
/* host libm itself.  orc_expf_glibc restates the algorithm as the GPU's     */
/* exact sampler computes it (pkv_sample.hip, expf_glibc): x N / ln2 = k + r */
/* (N = 32, k by the 1.5 * 2^52 shift), r by one fused multiply-add,          */
/* exp(x) = 2^(k/N) (table of 2^(i/32) rounded to double) times a cubic in r */
/* with the published minimax coefficients, in double, rounded once.         */
/* Algorithm, table values and coefficients: Arm Optimized Routines          */
/* (math/expf.c, exp2f_data.c; Copyright (c) Arm Limited, MIT OR Apache-2.0  */
/* WITH LLVM-exception), the expf glibc has used since 2.28.                 */
/* orc_expf_mismatches counts the inputs where the two disagree, so a test  */
/* can pin the restatement to the host libm on every float <= 0.             */
/* ------------------------------------------------------------------------ */
void orc_expf_host(const float* x, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = expf(x[i]);
}

static const uint64_t orc_exp2_tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

uint64_t orc_exp2_tab_entry(int i) { return orc_exp2_tab[i & 31]; }

float orc_expf_glibc(float x) {
    const double N = 32.0;
    const double inv_ln2_n = 0x1.71547652b82fep0 * N, shift = 0x1.8p52;
    const double c0 = 0x1.c6af84b912394p-5 / N / N / N, c1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double c2 = 0x1.62e42ff0c52d6p-1 / N;
    if (x != x) return x + x;
    if (x == -INFINITY) return 0.0f;
    if (x > 0x1.62e42ep6f) return INFINITY;
    if (x < -0x1.9fe368p6f) return 0.0f;
    double xd = (double)x, z = inv_ln2_n * xd, kd = z + shift;
    uint64_t ki, t;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    double r = fma(inv_ln2_n, xd, -kd);
    t = orc_exp2_tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    double zz = fma(c0, r, c1), r2 = r * r, y = fma(c2, r, 1.0);
    y = fma(zz, r2, y);
    return (float)(y * s);
}

/* Inputs with bit patterns lo, lo + step, ... <= hi where orc_expf_glibc
 * and the host expf differ; *first gets the first one (0: none). */
int64_t orc_expf_mismatches(uint32_t lo, uint32_t hi, uint32_t step, uint32_t* first) {
    int64_t bad = 0;
    uint32_t f = 0;
    const int64_t n = ((int64_t)hi - (int64_t)lo) / (int64_t)step + 1;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (int64_t j = 0; j < n; ++j) {
        uint32_t b = lo + (uint32_t)(j * (int64_t)step);
        float x, a, m;
        memcpy(&x, &b, 4);
        a = expf(x);
        m = orc_expf_glibc(x);
        if (memcmp(&a, &m, 4) != 0) {
            ++bad;
#pragma omp critical
            if (!f || b < f) f = b;
        }
    }
    if (first) *first = f;
    return bad;
}
