// pkv_decode_dev.h -- the paged decode-attention kernel body (gfx950),
// shared by the decode launch (pkv_decode.hip) and the mixed prefill +
// decode launch (pkv_mixed.hip).  Design notes: pkv_decode.hip.
#pragma once

#include <type_traits>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {


constexpr int kWavesPerBlock = 4;

// Largest decode tile in tokens of the RoPE kernels with fewer than eight
// query heads per wave (K and V of one tile are held in registers while the
// tile is processed); 64 or 32.
#ifndef PKV_DECODE_TILE
#define PKV_DECODE_TILE 64
#endif

// Partition planning: the longest context partition in tokens, and the
// number of (sequence, kv head, partition) waves below which partitions
// are halved (down to 64 tokens) to spread a small batch over the CUs.
#ifndef PKV_DECODE_PART_MAX
#define PKV_DECODE_PART_MAX 1024
#endif
#ifndef PKV_DECODE_MIN_ITEMS
#define PKV_DECODE_MIN_ITEMS 2048
#endif
// Work-list launches of up to PKV_DECODE_SUB_SPLIT_MAX_ITEMS full-length
// items cut each context's last PART_MAX tokens into this many parts.
#ifndef PKV_DECODE_SUB_SPLIT
#define PKV_DECODE_SUB_SPLIT 2
#endif
#ifndef PKV_DECODE_SUB_SPLIT_MAX_ITEMS
#define PKV_DECODE_SUB_SPLIT_MAX_ITEMS 8192
#endif

// R is the number of query heads a wave carries (1, 2, 4, 8 or 16): the
// GQA ratio itself, or the next of these widths above it, the extra heads
// being zero rows of the MFMA A operand whose results are never stored.
template <int DT, int HD, int R, bool ROPE = false>
struct DCfg {
  static constexpr int E = DT == PKV_F32 ? 4 : 2;  // element bytes
  static constexpr int RB = HD * E;                // row bytes
  static constexpr int NF = RB / 64;               // QK fragments per lane per row
  static constexpr int NST0 = 16 / NF;
  // Tile (tokens in flight per wave): 32, 16 for sixteen heads (four times
  // the GQA-4 accumulators).  A K fragment load reads 64 bytes of each of 16
  // rows (the MFMA operand layout); streams of such loads lose bandwidth as
  // more of them are in flight per CU: 32-token tiles at two waves per SIMD
  // (128 KiB per CU) read 6.9 TB/s in a probe of this access pattern, 64-token
  // ones (256 KiB) 6.2 TB/s, and the decode follows (Llama-3-8B shape 394
  // against 406-411 us, Llama-3-70B 449 against 460 us, Llama-3.2-1B 8.5
  // against 8.7-8.8 us).  The RoPE kernels (more registers live around the
  // loop) measured the other way (410 against 400 us) and keep 64 tokens
  // below GQA 8, and 48 for bf16 rows of 128 at GQA 8.
  static constexpr int NSTMAX =
      (R >= 16  ? 16
       : !ROPE  ? 32
       : R >= 8 ? (DT == PKV_BF16 && HD == 128 ? 48 : 32)
                : PKV_DECODE_TILE) /
      16;
  static constexpr int NST = NST0 < 1 ? 1 : (NST0 > NSTMAX ? NSTMAX : NST0);  // sub-tiles
  static constexpr int TILE = 16 * NST;            // tokens per tile
  static constexpr int CH = RB / 16;               // 16-byte chunks per row
  static constexpr int TPL = 64 / CH;              // tokens per V load
  static constexpr int NV = TILE / TPL;            // V loads per tile
  static constexpr int EPL = 16 / E;               // elements per chunk
  static constexpr int PP = R <= 4 ? 4 : R;        // LDS pitch of a P row
  static constexpr int RG = (R + 3) / 4;           // MFMA row groups with heads
  static_assert(R == 1 || R == 2 || R == 4 || R == 8 || R == 16, "group width");
  static_assert(CH <= 64, "row wider than a wave of 16-byte chunks");
  static_assert(TILE % TPL == 0, "tile/V-load mismatch");
};

struct DecodeKArgs {
  char* k_pool;
  char* v_pool;
  const char* q;
  void* out;
  int out_f32;
  const int32_t* block_tables;
  int mbps;
  const int32_t* context_lens;
  int max_context_len;
  int batch;
  int kvh;
  int num_blocks;
  int bs_log2;
  int part_tokens;
  int sub_tokens;  // the last PT tokens of a context split into parts of this many
  int pt_log2;     // log2 of part_tokens and sub_tokens (both powers of two)
  int sub_log2;
  int max_parts;
  float scale_log2;
  const char* k_new;
  const char* v_new;
  float* part_ml;
  float* part_o;
  uint32_t* err;
  const float* rope_cos;  // RoPE tables [rope_max][HD / 2], or null
  const float* rope_sin;
  int rope_max;
  const int32_t* positions;  // null: position = context_len - 1
  int in_f32;                // q / k_new / v_new are f32 (else the pool dtype)
  // GQA: kv head g serves query heads g * rtot .. g * rtot + rtot - 1; this
  // launch computes heads h0 .. h0 + rq - 1 of every group (rq <= the
  // kernel's width R; rtot > 16 takes several launches).
  int rq;
  int rtot;
  int h0;
  int store_new;  // 1: the launch stores k_new / v_new into the pool
  // 1: wave item -> (sequence, partition) by arithmetic, every sequence
  // given max_parts slots (small launches); 0: the longest-first work list.
  int direct;
};

// Partitions of a context of ctx tokens: nf = (ctx - 1) / PT full
// partitions of PT tokens, then the remaining ctx - nf PT tokens (1 .. PT)
// in parts of SUB tokens, the last one shorter (SUB == PT: ceil(ctx / PT)
// partitions of PT).  ctx <= 0: none.  Cutting the last PT tokens finer
// puts short items at the end of the longest-first work list, so the
// launch's final round of waves is short (the main kernel and the merge use
// the same layout).  PT = 2^ptl and SUB = 2^subl.
__device__ __forceinline__ int part_count(int ctx, int ptl, int subl, int* nf_out = nullptr) {
  const int nf = ctx > 0 ? (ctx - 1) >> ptl : 0;
  if (nf_out) *nf_out = nf;
  return ctx > 0 ? nf + ((ctx - (nf << ptl) + (1 << subl) - 1) >> subl) : 0;
}
__device__ __forceinline__ int part_begin(int p, int nf, int ptl, int subl) {
  return p < nf ? p << ptl : (nf << ptl) + ((p - nf) << subl);
}

// Floats per (sequence, kv head, partition) item in the (m, l) region of
// the split-context partials: one 128-byte line, (m, l) of up to 16 heads.
constexpr int kMlFloats = 32;

// Context lengths of up to kCtxCache sequences are staged in LDS once per
// workgroup; the work-list search and every item's length read them there.
constexpr int kCtxCache = 2048;

// LDS of one decode workgroup: each wave's P slice, the staged context
// lengths, and each wave's copy of the new token's K and V rows as stored
// (fused append).
template <int DT, int HD, int R, bool ROPE = false>
struct DecodeSmem {
  using C = DCfg<DT, HD, R, ROPE>;
  float p[kWavesPerBlock][C::TILE * C::PP];
  int ctx[kCtxCache];
  alignas(16) char nl[kWavesPerBlock][2 * C::RB];
};

// Host side (pkv_decode.hip).  Group width of the kernel instantiated for a
// GQA ratio: the ratio itself or the next of 1, 2, 4, 8, 16.
int group_width(int r);
// Kernel arguments of slice h0 (query heads h0 .. h0 + 15 of every group)
// of a decode launch whose partials go to `partials`; items = waves.
DecodeKArgs decode_kargs(const pkv_pool* p, int layer, const DecodeArgs& a, char* partials,
                         int h0, long long* items);
// The split-context merge after the main kernel (nothing with one partition).
hipError_t launch_decode_merge(const pkv_pool* p, const DecodeKArgs& k, hipStream_t stream);

namespace {


// N elements of a row, from f32 or 16-bit storage, as floats.
template <int DT, int N>
__device__ __forceinline__ void load_elems(const char* row, int elem, bool f32,
                                           float (&x)[N]) {
  auto from_f32 = [&]() {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(row + (size_t)(elem + i) * 4);
      x[i] = v[0];
      x[i + 1] = v[1];
      x[i + 2] = v[2];
      x[i + 3] = v[3];
    }
  };
  if constexpr (DT == PKV_F32) {
    from_f32();
  } else {
    static_assert(N == 8, "16-bit rows are read 8 elements (16 bytes) at a time");
    if (f32)
      from_f32();
    else
      widen16<DT, 8>(ld16(row + (size_t)elem * 2), x);
  }
}

// 16 bytes of pool-dtype storage from EPL floats (round to nearest even).
template <int DT, int EPL>
__device__ __forceinline__ u32x4 pack16(const float (&x)[EPL]) {
  if constexpr (DT == PKV_F32) {
    return u32x4{__float_as_uint(x[0]), __float_as_uint(x[1]), __float_as_uint(x[2]),
                 __float_as_uint(x[3])};
  } else {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t lo = DT == PKV_BF16 ? f32_to_bf16_bits(x[2 * i]) : f32_to_f16_bits(x[2 * i]);
      const uint32_t hi =
          DT == PKV_BF16 ? f32_to_bf16_bits(x[2 * i + 1]) : f32_to_f16_bits(x[2 * i + 1]);
      w[i] = lo | (hi << 16);
    }
    return w;
  }
}

// Rotate-half RoPE of N element pairs (x1 = first half, x2 = second half):
// o1 = x1 cos - x2 sin, o2 = x1 sin + x2 cos, each product rounded in f32.
template <int N>
__device__ __forceinline__ void rope_rotate(float (&x1)[N], float (&x2)[N], const float* c,
                                            const float* s) {
#pragma clang fp contract(off)
#pragma unroll
  for (int i = 0; i < N; ++i) {
    const float a = x1[i], b = x2[i];
    x1[i] = a * c[i] - b * s[i];
    x2[i] = a * s[i] + b * c[i];
  }
}

template <int EPL>
__device__ __forceinline__ void store_out(void* out, size_t elem_off, int out_f32,
                                          int dt, const float (&x)[EPL]) {
  if (out_f32) {
    float* o = reinterpret_cast<float*>(out) + elem_off;
#pragma unroll
    for (int i = 0; i < EPL; i += 4)
      *reinterpret_cast<f32x4*>(o + i) = f32x4{x[i], x[i + 1], x[i + 2], x[i + 3]};
  } else if (EPL == 8) {
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t lo = dt == PKV_BF16 ? f32_to_bf16_bits(x[2 * i]) : f32_to_f16_bits(x[2 * i]);
      uint32_t hi = dt == PKV_BF16 ? f32_to_bf16_bits(x[2 * i + 1]) : f32_to_f16_bits(x[2 * i + 1]);
      w[i] = lo | (hi << 16);
    }
    *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(out) + elem_off) = w;
  } else {
    // f32 pool with f32 output is the only EPL == 4 case (handled above);
    // 16-bit outputs of an f32 pool are rejected on the host.
  }
}

__device__ __forceinline__ int clamp_ctx(const DecodeKArgs& a, int ctx, int BS) {
  return ctx < 0 ? 0 : min(ctx, min(a.max_context_len, a.mbps * BS));
}

// Inclusive prefix sum across the 64 lanes of a wave in lane order, on DPP:
// shifts by 1, 2, 4 and 8 lanes within each 16-lane row (lanes shifted in
// from outside the row add 0), then lane 15's sum broadcast into rows 1 and
// 3 and lane 31's into rows 2 and 3 (no LDS round trips).
__device__ __forceinline__ int wave_incl_scan(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}


// Keys row b attends: context_lens[b] (ctx_raw), bounded by positions[b] + 1
// when positions are given -- build_mask's two bounds k < seq_lens[b] and
// k <= q_positions[b] (attention.rs:22).  A negative position attends
// nothing (reported by the kernel).  Unclamped, like ctx_raw.
__device__ __forceinline__ int attended_len(const DecodeKArgs& a, int b, int ctx_raw) {
  if (!a.positions) return ctx_raw;
  const int pos = a.positions[b];
  return pos < 0 ? 0 : (pos >= ctx_raw ? ctx_raw : pos + 1);
}

// Attended lengths (attended_len) of the batch: the first n from LDS, the
// rest from global memory.
struct CtxLens {
  const DecodeKArgs* a;
  const int* lds;    // LDS copy of the first n entries
  int n;
  __device__ __forceinline__ int operator[](int b) const {
    return b < n ? lds[b] : attended_len(*a, b, a->context_lens[b]);
  }
};

// Buckets of the last partitions' lengths, (j * SUB / NB, (j + 1) * SUB / NB].
constexpr int kLptBuckets = 16;

// The sequence of rank k (0-based) when the batch is ordered by bucket
// (bucket_of(b) in [0, kLptBuckets), highest bucket first) and by sequence
// index within a bucket: per-bucket ballot counts over the batch, then the
// rank of the wanted sequence within its bucket.  Wave-uniform.
template <typename BucketOf>
__device__ __forceinline__ bool nth_by_bucket(int batch, long long k, int lane,
                                              BucketOf bucket_of, int& b) {
  int cnt[kLptBuckets];
#pragma unroll
  for (int j = 0; j < kLptBuckets; ++j) cnt[j] = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int bk = b0 + lane < batch ? bucket_of(b0 + lane) : -1;
#pragma unroll
    for (int j = 0; j < kLptBuckets; ++j) cnt[j] += __popcll(__ballot(bk == j));
  }
  int want = -1;
#pragma unroll
  for (int j = kLptBuckets - 1; j >= 0; --j) {
    if (want < 0) {
      if (k < cnt[j]) want = j;
      else k -= cnt[j];
    }
  }
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int bk = b0 + lane < batch ? bucket_of(b0 + lane) : -1;
    const unsigned long long mask = __ballot(bk == want);
    const int c = __popcll(mask);
    if (k < c) {
      const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
      const unsigned long long hit = __ballot(bk == want && below == (int)k);
      b = b0 + __ffsll((long long)hit) - 1;
      return true;
    }
    k -= c;
  }
  return false;  // k >= batch
}

// Item k of a list made of count_of(b) consecutive items per sequence, in
// sequence order: its sequence b and index j within the sequence, via a
// wave prefix sum over 64 sequences per step.  Otherwise k is reduced by the
// list's length and false returned.  Wave-uniform.
template <typename CountOf>
__device__ __forceinline__ bool find_in_list(int batch, long long& k, int lane, CountOf count_of,
                                             int& b, int& j) {
  long long base = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int f = b0 + lane < batch ? count_of(b0 + lane) : 0;
    const int incl = wave_incl_scan(f);
    const int excl = incl - f;
    const unsigned long long hit = __ballot(k >= base + excl && k < base + incl);
    if (hit) {
      const int hl = __ffsll((long long)hit) - 1;
      b = b0 + hl;
      j = (int)(k - base - readlane_i(excl, hl));
      return true;
    }
    base += readlane_i(incl, 63);
  }
  k -= base;
  return false;
}

// Work list of one launch, in dispatch order: first every full partition
// (p < nf(b), PT tokens each) in sequence order, then every part of a
// sequence's last PT tokens but its last (SUB tokens each) in sequence
// order, then the last partition of every sequence (p = n_parts(b) - 1;
// p = 0 with an empty context) from the longest length bucket down,
// sequence order within a bucket.  Hardware dispatch in grid order then
// approximates longest-processing-time-first scheduling, and the grid's
// surplus waves (the host sizes it for the longest context) sit past the
// end of the list.  Each wave finds its (b, p) from the context lengths.
__device__ bool locate_pair(const DecodeKArgs& a, const CtxLens& cl, long long kpair, int lane,
                            int BS, int& b, int& p) {
  const int PT = a.part_tokens, SUB = a.sub_tokens, ptl = a.pt_log2, subl = a.sub_log2;
  auto layout = [&](int bb, int& nf) { return part_count(clamp_ctx(a, cl[bb], BS), ptl, subl, &nf); };
  long long k = kpair;
  int j = 0;
  if (find_in_list(a.batch, k, lane, [&](int bb) { int nf; layout(bb, nf); return nf; }, b, j)) {
    p = j;
    return true;
  }
  if (SUB < PT &&
      find_in_list(a.batch, k, lane, [&](int bb) {
        int nf;
        const int np = layout(bb, nf);
        return np > nf + 1 ? np - nf - 1 : 0;
      }, b, j)) {
    int nf;
    layout(b, nf);
    p = nf + j;
    return true;
  }
  if (k >= a.batch) return false;
  // the last partition: its length bucket over (0, SUB]
  auto last_bucket = [&](int bb) -> int {
    int nf;
    const int np = layout(bb, nf);
    const int ctx = clamp_ctx(a, cl[bb], BS);
    const int len = np > 0 ? ctx - part_begin(np - 1, nf, ptl, subl) : 0;  // 0 .. SUB
    return len <= 0 ? 0 : ((len - 1) * kLptBuckets) >> subl;
  };
  if (!nth_by_bucket(a.batch, k, lane, last_bucket, b)) return false;
  int nf;
  const int np = layout(b, nf);
  p = np > 0 ? np - 1 : 0;
  return true;
}

// One workgroup of the decode launch: block index bid, LDS in sm.
// SB (block_size below 16): the 16 tokens of a K sub-tile, and the tokens of
// a V load, span several blocks, so each lane takes its own token's block
// id from the partition's table slice (an LDS-crossbar permute) instead of
// one wave-uniform id per sub-tile.
template <int DT, int HD, int R, bool ROPE, bool SB = false>
__device__ __forceinline__ void decode_body(const DecodeKArgs& a, int bid,
                                            DecodeSmem<DT, HD, R, ROPE>& sm) {
  using C = DCfg<DT, HD, R, ROPE>;
  auto& p_lds_all = sm.p;
  auto& ctx_lds = sm.ctx;
  auto& new_lds_all = sm.nl;

  // The wave index is uniform within a wave; readfirstlane tells the
  // compiler so, which keeps every per-wave quantity in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  float* p_lds = p_lds_all[wave];

  const int H = a.kvh * a.rtot;
  const int rq = a.rq;  // query heads of this launch per group (<= R)
  const int BS = 1 << a.bs_log2;
  const int PT = a.part_tokens, SUB = a.sub_tokens, ptl = a.pt_log2, subl = a.sub_log2;
  // items (and so block ids) < 2^26: decode_validate refuses larger launches
  const unsigned item = (unsigned)bid * kWavesPerBlock + wave;
  const unsigned kvh = (unsigned)a.kvh;
  const unsigned rest = item / kvh;  // item = (b, p) * kvh + g
  const int g = (int)(item - rest * kvh);
  int b = 0, p = 0;
  CtxLens cl{&a, ctx_lds, 0};
  if (a.direct) {  // launch-uniform
    // Small launches: (b, p) straight from the item, so the wave issues its
    // context length, table slice and Q loads at once (no staging round
    // trip); slots past a sequence's partitions exit below.
    b = (int)(rest / (unsigned)a.max_parts);
    p = (int)(rest - (unsigned)b * a.max_parts);
    if (b >= a.batch) return;
  } else {
    cl.n = min(a.batch, kCtxCache);
    for (int i = threadIdx.x; i < cl.n; i += kWavesPerBlock * kWave)
      ctx_lds[i] = attended_len(a, i, a.context_lens[i]);
    __syncthreads();
    if (!locate_pair(a, cl, rest, lane, BS, b, p)) return;
  }

  const int G = lane >> 4;
  const int col = lane & 15;
  // The partition's first token and length bound: p * PT with the plain
  // layout (known before the context length, which the direct mapping has
  // not read yet), else from the layout of the staged length.
  int t_begin = p * PT, plen = PT;
  if (SUB < PT) {  // launch-uniform; work-list launches only
    int nf;
    part_count(clamp_ctx(a, cl[b], BS), ptl, subl, &nf);
    t_begin = part_begin(p, nf, ptl, subl);
    plen = p < nf ? PT : SUB;
  }
  const int blk_begin = t_begin >> a.bs_log2;
  // Loads that do not depend on the context length go out first: the block
  // ids the partition spans (partitions are block-aligned and span at most
  // 64 blocks, decode_plan; lane i holds entry blk_begin + i, ids past the
  // sequence's blocks are never used) and, without RoPE, the Q group as the
  // MFMA A operand (row = head lane % 16, k-slice lane / 16).
  const int span = plen >> a.bs_log2 > 1 ? plen >> a.bs_log2 : 1;
  int tbl = 0;
  if (lane < span && blk_begin + lane < a.mbps)
    tbl = a.block_tables[(size_t)b * a.mbps + blk_begin + lane];
  u32x4 qf[C::NF];
  if constexpr (!ROPE) {
    const char* qrow = a.q + ((size_t)b * H + g * a.rtot + a.h0 + (col < rq ? col : 0)) * C::RB;
#pragma unroll
    for (int f = 0; f < C::NF; ++f)
      qf[f] = col < rq ? ld16(qrow + 64 * f + 16 * G) : u32x4{0, 0, 0, 0};
  }

  // ctx: the keys attended (the partition layout's length); ctx_raw: the
  // context length, where the new token goes
  const int alen = cl[b];
  const int ctx_raw = a.positions ? a.context_lens[b] : alen;
  const int ctx_c = clamp_ctx(a, ctx_raw, BS);
  const bool clamped = ctx_c != ctx_raw;
  if (clamped && lane == 0 && p == 0) atomicOr(a.err, PKV_EBIT_LENGTH);
  if (a.positions && lane == 0 && p == 0 && a.positions[b] < 0) atomicOr(a.err, PKV_EBIT_POSITION);
  const int ctx = min(clamp_ctx(a, alen, BS), ctx_c);
  const int n_parts = part_count(ctx, ptl, subl);
  const int c = lane % C::CH;   // 16-byte chunk of a row (PV / output mapping)
  const int tg = lane / C::CH;  // token group of a V load

  if (ctx == 0) {
    if (p == 0 && lane < C::CH) {
      float z[C::EPL];
#pragma unroll
      for (int e = 0; e < C::EPL; ++e) z[e] = 0.0f;
#pragma unroll
      for (int h = 0; h < R; ++h)
        if (h < rq)
          store_out<C::EPL>(a.out, ((size_t)b * H + g * a.rtot + a.h0 + h) * HD + c * C::EPL,
                            a.out_f32, DT, z);
    }
    return;
  }
  if (p >= n_parts) return;

  const int t_end = min(ctx, t_begin + plen);
  const int nblk = ((t_end - 1) >> a.bs_log2) - blk_begin + 1;  // <= span
  // the new token's position (stored by the last partition's wave, also
  // when the positions bound leaves it out of the attended keys)
  const int new_pos = (a.k_new != nullptr && !clamped) ? ctx_c - 1 : -1;

  int rpos = 0;  // RoPE position of this sequence's new token
  if constexpr (ROPE) {
    // Rotate Q in the kernel (transformer.rs:252-269).  Fragment f of a lane
    // holds elements f * 64/E + G * EPL .. + EPL - 1, so the partner of each
    // element (+ HD/2) sits in fragment f + NF/2 of the same lane.
    rpos = a.positions ? a.positions[b] : ctx_raw - 1;
    if (rpos < 0 || rpos >= a.rope_max) {
      if (lane == 0) atomicOr(a.err, PKV_EBIT_POSITION);
      rpos = 0;
    }
    const size_t irb = a.in_f32 ? (size_t)HD * 4 : (size_t)C::RB;
    const char* qrow = a.q + ((size_t)b * H + g * a.rtot + a.h0 + (col < rq ? col : 0)) * irb;
    const float* cr = a.rope_cos + (size_t)rpos * (HD / 2);
    const float* sr = a.rope_sin + (size_t)rpos * (HD / 2);
#pragma unroll
    for (int f = 0; f < C::NF / 2; ++f) {
      const int e0 = f * (64 / C::E) + G * C::EPL;
      float x1[C::EPL], x2[C::EPL], cs[C::EPL], sn[C::EPL];
      load_elems<DT, C::EPL>(qrow, e0, a.in_f32, x1);
      load_elems<DT, C::EPL>(qrow, e0 + HD / 2, a.in_f32, x2);
      load_elems<PKV_F32, C::EPL>(reinterpret_cast<const char*>(cr), e0, true, cs);
      load_elems<PKV_F32, C::EPL>(reinterpret_cast<const char*>(sr), e0, true, sn);
      rope_rotate<C::EPL>(x1, x2, cs, sn);
      qf[f] = col < rq ? pack16<DT, C::EPL>(x1) : u32x4{0, 0, 0, 0};
      qf[f + C::NF / 2] = col < rq ? pack16<DT, C::EPL>(x2) : u32x4{0, 0, 0, 0};
    }
  }
  const bool tbl_bad = lane < nblk && (tbl < 0 || tbl >= a.num_blocks);
  const uint64_t bad_blocks = __ballot(tbl_bad);
  if (tbl_bad) {
    atomicOr(a.err, PKV_EBIT_BLOCK);
    tbl = 0;
  }

  const size_t head_off = (size_t)g * C::RB;
  const size_t slot_stride = (size_t)a.kvh * C::RB;

  // Fused append: the wave of the last partition stores the new token's row
  // (write before attend) and keeps the stored bytes in its LDS slice; its
  // last tile takes that token's K and V from there.  The attention thus
  // never reads back the pool bytes this launch writes, so no ordering of a
  // store before a load of the same address is assumed, on any memory type.
  char* new_lds = new_lds_all[wave];
  const bool store_here = new_pos >= 0 && p == n_parts - 1;
  const bool has_new = store_here && new_pos == ctx - 1;  // the last tile attends it
  if (store_here) {
    // its block: from the partition's table slice, or (past the attended
    // keys) read from the table and checked; a bad id stores nothing
    const int nb_idx = new_pos >> a.bs_log2;
    int blk;
    bool bad_store;
    if (nb_idx - blk_begin < nblk) {
      blk = readlane_i(tbl, nb_idx - blk_begin);
      bad_store = (bad_blocks >> (nb_idx - blk_begin)) & 1;
    } else {
      blk = a.block_tables[(size_t)b * a.mbps + nb_idx];
      bad_store = blk < 0 || blk >= a.num_blocks;
      if (bad_store && lane == 0) atomicOr(a.err, PKV_EBIT_BLOCK);
    }
    const bool do_store = a.store_new && !bad_store;
    size_t off = ((size_t)(bad_store ? 0 : blk) * BS + (new_pos & (BS - 1))) * slot_stride + head_off;
    char* kst = a.k_pool + off;
    char* vst = a.v_pool + off;
    if constexpr (ROPE) {
      // k rotated like q (same position), v converted; chunk c < CH/2 and its
      // partner c + CH/2 are rotated together by lane c.
      const size_t irb = a.in_f32 ? (size_t)HD * 4 : (size_t)C::RB;
      const char* krow = a.k_new + ((size_t)b * a.kvh + g) * irb;
      const char* vrow = a.v_new + ((size_t)b * a.kvh + g) * irb;
      if (lane < C::CH / 2) {
        const int e0 = lane * C::EPL;
        float x1[C::EPL], x2[C::EPL], cs[C::EPL], sn[C::EPL];
        load_elems<DT, C::EPL>(krow, e0, a.in_f32, x1);
        load_elems<DT, C::EPL>(krow, e0 + HD / 2, a.in_f32, x2);
        load_elems<PKV_F32, C::EPL>(
            reinterpret_cast<const char*>(a.rope_cos + (size_t)rpos * (HD / 2)), e0, true, cs);
        load_elems<PKV_F32, C::EPL>(
            reinterpret_cast<const char*>(a.rope_sin + (size_t)rpos * (HD / 2)), e0, true, sn);
        rope_rotate<C::EPL>(x1, x2, cs, sn);
        const u32x4 k1 = pack16<DT, C::EPL>(x1), k2 = pack16<DT, C::EPL>(x2);
        st16(new_lds + lane * 16, k1);
        st16(new_lds + (lane + C::CH / 2) * 16, k2);
        if (do_store) {
          st16(kst + lane * 16, k1);
          st16(kst + (lane + C::CH / 2) * 16, k2);
        }
      }
      if (lane < C::CH) {
        float x[C::EPL];
        load_elems<DT, C::EPL>(vrow, lane * C::EPL, a.in_f32, x);
        const u32x4 v1 = pack16<DT, C::EPL>(x);
        st16(new_lds + C::RB + lane * 16, v1);
        if (do_store) st16(vst + lane * 16, v1);
      }
    } else if (lane < C::CH) {
      const u32x4 k1 = ld16(a.k_new + ((size_t)b * a.kvh + g) * C::RB + lane * 16);
      const u32x4 v1 = ld16(a.v_new + ((size_t)b * a.kvh + g) * C::RB + lane * 16);
      st16(new_lds + lane * 16, k1);
      st16(new_lds + C::RB + lane * 16, v1);
      if (do_store) {
        st16(kst + lane * 16, k1);
        st16(vst + lane * 16, v1);
      }
    }
  }

  // A row is addressed as a wave-uniform base (pool + head + physical block)
  // plus a 32-bit per-lane offset (slot in block, 16-byte fragment).
  // Tokens past t_end are clamped to t_end - 1: a valid row whose score is
  // masked (K) or whose weight is exactly 0 (V).
  const char* kh = a.k_pool + head_off;
  const char* vh = a.v_pool + head_off;
  const size_t blk_stride = (size_t)BS * slot_stride;
  const int tmask = BS - 1;
  const int lg = a.bs_log2;

  // Block of a token of the partition: lane i of tbl holds the id of block
  // blk_begin + i.  A wave-uniform token's id is a readlane; with SB each
  // lane's own token's id is a permute across the lanes.
  auto lane_block = [&](int tok) {
    return __builtin_amdgcn_ds_bpermute(((tok >> lg) - blk_begin) << 2, tbl);
  };
  // K fragment f of sub-tile st: token lane % 16, k-slice lane / 16; the four
  // lanes of a token read 64 contiguous bytes.  With block_size >= 16 the 16
  // tokens of a sub-tile share one block.
  auto k_row = [&](int tile_base, int st) {
    const int t0 = min(tile_base + 16 * st, t_end - 1);
    const int tok = min(tile_base + 16 * st + col, t_end - 1);
    if constexpr (SB)
      return kh + (size_t)lane_block(tok) * blk_stride +
             ((uint32_t)((tok & tmask) * slot_stride) + 16 * G);
    const char* base = kh + (size_t)readlane_i(tbl, (t0 >> lg) - blk_begin) * blk_stride;
    return base + ((uint32_t)((tok & tmask) * slot_stride) + 16 * G);
  };
  // V load i of a tile: TPL consecutive tokens (one block when block_size
  // >= TPL), lane = (token group tg, 16-byte chunk c): consecutive lanes
  // read consecutive bytes.
  auto v_chunk = [&](int tile_base, int i) {
    const int t0 = min(tile_base + i * C::TPL, t_end - 1);
    const int tok = min(tile_base + i * C::TPL + tg, t_end - 1);
    if constexpr (SB)
      return vh + (size_t)lane_block(tok) * blk_stride +
             ((uint32_t)((tok & tmask) * slot_stride) + 16 * c);
    const char* base = vh + (size_t)readlane_i(tbl, (t0 >> lg) - blk_begin) * blk_stride;
    return base + ((uint32_t)((tok & tmask) * slot_stride) + 16 * c);
  };

  float m[4], lsum[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    m[j] = -INFINITY;
    lsum[j] = 0.0f;
  }
  float o[R][C::EPL];
#pragma unroll
  for (int h = 0; h < R; ++h)
#pragma unroll
    for (int e = 0; e < C::EPL; ++e) o[h][e] = 0.0f;

  const int ntiles = (t_end - t_begin + C::TILE - 1) / C::TILE;
  u32x4 kf[C::NST][C::NF];
  u32x4 vf[C::NV];
#pragma unroll
  for (int st = 0; st < C::NST; ++st) {
    const char* r = k_row(t_begin, st);
#pragma unroll
    for (int f = 0; f < C::NF; ++f) kf[st][f] = ld16_stream(r + 64 * f);
  }
#pragma unroll
  for (int i = 0; i < C::NV; ++i) vf[i] = ld16_stream(v_chunk(t_begin, i));

  // One tile, software-pipelined at distance one tile: every K fragment is
  // reloaded with the next tile's fragment right after its MFMA has read
  // it, and every V chunk right after its P.V, so a whole tile of loads is
  // always in flight and the registers are reused in place.  The last tile
  // is instantiated without the reloads, which keeps all load counts static
  // for the compiler's wait insertion.
  auto tile_body = [&](const int tile_base, auto prefetch) {
    constexpr bool PF = decltype(prefetch)::value;
    const int next = tile_base + C::TILE;
    if constexpr (!PF) {
      // The last tile holds the new token (position t_end - 1, where every
      // clamped lane points too): its K and V come from the LDS copy.
      if (has_new) {
#pragma unroll
        for (int st = 0; st < C::NST; ++st)
          if (tile_base + 16 * st + col >= new_pos) {
#pragma unroll
            for (int f = 0; f < C::NF; ++f) kf[st][f] = ld16(new_lds + 64 * f + 16 * G);
          }
#pragma unroll
        for (int i = 0; i < C::NV; ++i)
          if (tile_base + i * C::TPL + tg >= new_pos) vf[i] = ld16(new_lds + C::RB + 16 * c);
      }
    }
    f32x4 acc[C::NST];
#pragma unroll
    for (int st = 0; st < C::NST; ++st) {
      acc[st] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int f = 0; f < C::NF; ++f) mfma_frag<DT>(qf[f], kf[st][f], acc[st]);
      if constexpr (PF) {
        const char* r = k_row(next, st);
#pragma unroll
        for (int f = 0; f < C::NF; ++f) kf[st][f] = ld16_stream(r + 64 * f);
      }
    }

    // ---- online softmax (exp2 domain) ----
    float sc[C::NST][4];
#pragma unroll
    for (int st = 0; st < C::NST; ++st) {
      bool valid = tile_base + 16 * st + col < t_end;
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[st][j] = valid ? acc[st][j] * a.scale_log2 : -INFINITY;
    }
    float alpha[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float tmax = sc[0][j];
#pragma unroll
      for (int st = 1; st < C::NST; ++st) tmax = fmaxf(tmax, sc[st][j]);
      tmax = row_max16(tmax);
      float mnew = fmaxf(m[j], tmax);
      alpha[j] = fast_exp2(m[j] - mnew);
      m[j] = mnew;
      float ssum = 0.0f;
#pragma unroll
      for (int st = 0; st < C::NST; ++st) {
        sc[st][j] = fast_exp2(sc[st][j] - mnew);
        ssum += sc[st][j];
      }
      lsum[j] = lsum[j] * alpha[j] + ssum;
    }
    if (G < C::RG) {
#pragma unroll
      for (int st = 0; st < C::NST; ++st)
        *reinterpret_cast<f32x4*>(p_lds + (16 * st + col) * C::PP + 4 * G) =
            f32x4{sc[st][0], sc[st][1], sc[st][2], sc[st][3]};
    }
    __builtin_amdgcn_wave_barrier();

    // ---- P.V in fp32 ----
#pragma unroll
    for (int h = 0; h < R; ++h) {
      float ah = readlane_f(alpha[h & 3], 16 * (h >> 2));
#pragma unroll
      for (int e = 0; e < C::EPL; ++e) o[h][e] *= ah;
    }
#pragma unroll
    for (int i = 0; i < C::NV; ++i) {
      const float* pr = p_lds + (i * C::TPL + tg) * C::PP;
      float ph[R];
      if constexpr (R >= 4) {
#pragma unroll
        for (int h = 0; h < R; h += 4) {
          f32x4 t4 = *reinterpret_cast<const f32x4*>(pr + h);
          ph[h] = t4[0];
          ph[h + 1] = t4[1];
          ph[h + 2] = t4[2];
          ph[h + 3] = t4[3];
        }
      } else {
#pragma unroll
        for (int h = 0; h < R; ++h) ph[h] = pr[h];
      }
      float x[C::EPL];
      widen16<DT, C::EPL>(vf[i], x);
      if constexpr (PF) vf[i] = ld16_stream(v_chunk(next, i));
#pragma unroll
      for (int h = 0; h < R; ++h)
#pragma unroll
        for (int e = 0; e < C::EPL; ++e) o[h][e] = fmaf(ph[h], x[e], o[h][e]);
    }
    __builtin_amdgcn_wave_barrier();
  };
  for (int t = 0; t + 1 < ntiles; ++t)
    tile_body(t_begin + t * C::TILE, std::true_type{});
  tile_body(t_begin + (ntiles - 1) * C::TILE, std::false_type{});

  // ---- partition epilogue ----
  // P.V accumulators are summed over the token groups (lanes with equal
  // chunk c) on the VALU; every group then holds the full row and the
  // groups share the stores: group tg writes heads tg, tg + NG, ...
  constexpr int NG = 64 / C::CH;
#pragma unroll
  for (int j = 0; j < 4; ++j) lsum[j] = row_sum16(lsum[j]);
#pragma unroll
  for (int h = 0; h < R; ++h)
#pragma unroll
    for (int e = 0; e < C::EPL; ++e) o[h][e] = group_sum<C::CH>(o[h][e]);

  float mh[R], lh[R];
#pragma unroll
  for (int h = 0; h < R; ++h) {
    mh[h] = readlane_f(m[h & 3], 16 * (h >> 2));
    lh[h] = readlane_f(lsum[h & 3], 16 * (h >> 2));
  }

  if (n_parts == 1) {
#pragma unroll
    for (int h = 0; h < R; ++h) {
      if (h % NG != tg || h >= rq) continue;
      float inv = 1.0f / lh[h];
      float x[C::EPL];
#pragma unroll
      for (int e = 0; e < C::EPL; ++e) x[e] = o[h][e] * inv;
      store_out<C::EPL>(a.out, ((size_t)b * H + g * a.rtot + a.h0 + h) * HD + c * C::EPL,
                        a.out_f32, DT, x);
    }
    return;
  }

  // Partials go out with non-temporal stores: they are read once, by the
  // merge kernel, and stay out of the way of the K/V read stream (cfg4-size
  // launches: 4.5 % faster than with ordinary stores).  Every store
  // instruction writes whole, contiguous 128-byte lines: quad j of a lane's
  // EPL elements (elements c EPL + 4j ..) goes to float 4 CH j + 4c of the
  // head's partial row (the merge reads it back in that order), and the
  // (m, l) pairs fill one line per item (kMlFloats).
  const size_t pair = (size_t)b * a.kvh + g;
  float* ml = a.part_ml + (pair * a.max_parts + p) * kMlFloats;
  float* po = a.part_o + (pair * a.max_parts + p) * R * HD;
#pragma unroll
  for (int h = 0; h < R; ++h) {
    if (h % NG != tg || h >= rq) continue;
#pragma unroll
    for (int e = 0; e < C::EPL; e += 4)
      __builtin_nontemporal_store(f32x4{o[h][e], o[h][e + 1], o[h][e + 2], o[h][e + 3]},
                                  reinterpret_cast<f32x4*>(po + h * HD + C::CH * e + 4 * c));
  }
  // (m, l) of the R heads: lanes 0 .. 2R-1, padded with zeros to the line
  if (lane < kMlFloats) {
    float v = 0.0f;
#pragma unroll
    for (int h = 0; h < R; ++h)
      if ((lane >> 1) == h) v = (lane & 1) ? lh[h] : mh[h];
    __builtin_nontemporal_store(v, ml + lane);
  }
}

}  // namespace
}  // namespace pkv
