// pkv_decode.hip -- paged decode attention with fused KV append (gfx950).
//
// Replaces, for one layer of a decode step, the reference's per-row
// KvPool::write + gather_seq + pad + cat + build_mask + sdpa sequence
// (crates/ai-engine-candle/src/paged/transformer.rs:271-292,
//  crates/ai-engine-candle/src/paged/attention.rs:11-28,57-136) by one launch.
//
// Work decomposition: one wavefront per (sequence b, kv head g, context
// partition p).  The wave carries the whole GQA query group of g (R query
// heads h = g*R .. g*R+R-1, attention.rs:128-136) so every K/V byte of the
// partition is read from HBM exactly once per decode step.
//
// Per tile of TILE tokens:
//   * K: each lane loads 16-byte fragments of its token's row straight from
//     the block (block-table indirection resolved per 16-token sub-tile with
//     v_readlane from a per-partition table slice held in one VGPR) into the
//     B operand of v_mfma_f32_16x16x32_{bf16,f16} (v_mfma_f32_16x16x4f32 for
//     f32 pools); the Q group is the A operand.  S = Q K^T lands with token =
//     lane % 16 and head = 4 * (lane / 16) + register.  The four lanes of a
//     token read 64 contiguous bytes per instruction.
//   * Online softmax in the exp2 domain (scores pre-multiplied by
//     scale * log2 e), running max and partial sums per 16-lane row, row
//     max/sum by DPP row rotations.
//   * P goes through a 1-2 KB LDS slice of the wave; V is read with fully
//     coalesced 16-byte loads (consecutive lanes = consecutive 16 bytes of a
//     row) and P.V is accumulated in fp32 FMAs, so the softmax weights never
//     lose precision.
// Split-context: a sequence with n_parts > 1 partitions writes (m, l, O)
// partials; a second, small kernel merges them with log-sum-exp weights.
// (A last-arriver merge inside the main kernel needs agent-scope release/
// acquire fences per wave, i.e. an L2 writeback + invalidate on every XCD;
// measured on MI355X that cost more than half the kernel's throughput.  The
// kernel boundary provides the same visibility once per launch.)
//
// Fused append: with k_new/v_new given, the wave owning the last partition
// of (b, g) first stores the new token's K/V row at position context_len-1
// (slot = table[pos / bs] * bs + pos % bs, block_table.rs:55-58), makes it
// visible to itself with a workgroup-scope fence, and then reads it back
// like every other row -- write-then-attend exactly as transformer.rs:276-277,
// with no data-dependent loads in the main loop.
#include <mutex>
#include <type_traits>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kWavesPerBlock = 4;

// Largest decode tile in tokens (K and V of one tile are held in registers
// while the tile is processed); 64 or 32.
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

// R is the number of query heads a wave carries (1, 2, 4, 8 or 16): the
// GQA ratio itself, or the next of these widths above it, the extra heads
// being zero rows of the MFMA A operand whose results are never stored.
template <int DT, int HD, int R>
struct DCfg {
  static constexpr int E = DT == PKV_F32 ? 4 : 2;  // element bytes
  static constexpr int RB = HD * E;                // row bytes
  static constexpr int NF = RB / 64;               // QK fragments per lane per row
  static constexpr int NST0 = 16 / NF;
  // GQA 8 holds twice the P.V accumulators.  Two waves per SIMD fit a
  // 48-token tile for bf16 rows of 128 (238 registers; f16 widening needs
  // more) and a 32-token tile otherwise.  The kernel is bound by the loads
  // in flight, so the larger tile is faster where it fits (-3 % on the
  // Llama-3-70B shape); narrower rows keep 32, where the shorter partitions
  // of small batches would waste more of a 48-token tile.  Sixteen heads
  // hold four times the GQA-4 accumulators: 16-token tiles.
  static constexpr int NSTMAX =
      (R >= 16 ? 16 : R >= 8 ? (DT == PKV_BF16 && HD == 128 ? 48 : 32) : PKV_DECODE_TILE) / 16;
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

// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    int y = __builtin_amdgcn_ds_bpermute((lane - off) << 2, x);
    if (lane >= off) x += y;
  }
  return x;
}

// Context lengths of up to kCtxCache sequences are staged in LDS once per
// workgroup; the work-list search and every item's length read them there.
constexpr int kCtxCache = 2048;

struct CtxLens {
  const int32_t* g;  // global context_lens
  const int* lds;    // LDS copy of the first n entries
  int n;
  __device__ __forceinline__ int operator[](int b) const { return b < n ? lds[b] : g[b]; }
};

// Buckets of the last partitions' lengths, (j * PT / NB, (j + 1) * PT / NB].
constexpr int kLptBuckets = 16;

// Work list of one launch, in dispatch order: first every full partition
// (p < n_parts(b) - 1, PT tokens each) in sequence order, then the last,
// shorter partition of every sequence (p = n_parts(b) - 1; p = 0 with an
// empty context) from the longest length bucket down, sequence order within
// a bucket.  Hardware dispatch in grid order then approximates
// longest-processing-time-first scheduling, and the grid's surplus waves
// (the host sizes it for the longest context) sit past the end of the list.
// Each wave finds its (b, p) from the context lengths, 64 sequences per
// step: a wave prefix sum of full-partition counts, per-bucket ballot
// counts of the last partitions, and the rank of the wanted sequence within
// its bucket.
__device__ bool locate_pair(const DecodeKArgs& a, const CtxLens& cl, long long kpair, int lane,
                            int BS, int& b, int& p) {
  const int PT = a.part_tokens;
  long long base = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    const int bb = b0 + lane;
    int f = 0;
    if (bb < a.batch) {
      const int ctx = clamp_ctx(a, cl[bb], BS);
      const int np = (ctx + PT - 1) / PT;
      f = np > 1 ? np - 1 : 0;
    }
    const int incl = wave_incl_scan(f, lane);
    const int excl = incl - f;
    const unsigned long long hit = __ballot(kpair >= base + excl && kpair < base + incl);
    if (hit) {
      const int hl = __ffsll((long long)hit) - 1;
      b = b0 + hl;
      p = (int)(kpair - base - readlane_i(excl, hl));
      return true;
    }
    base += readlane_i(incl, 63);
  }
  long long k2 = kpair - base;
  if (k2 >= a.batch) return false;

  // Last partition of sequence bb: its bucket and partition index.
  auto last_of = [&](int bb, int& np) -> int {
    const int ctx = clamp_ctx(a, cl[bb], BS);
    np = (ctx + PT - 1) / PT;
    const int len = ctx - (np > 0 ? np - 1 : 0) * PT;  // 0 (empty context) .. PT
    return len <= 0 ? 0 : (len - 1) * kLptBuckets / PT;
  };
  int cnt[kLptBuckets];
#pragma unroll
  for (int j = 0; j < kLptBuckets; ++j) cnt[j] = 0;
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    int np = 0;
    const int bk = b0 + lane < a.batch ? last_of(b0 + lane, np) : -1;
#pragma unroll
    for (int j = 0; j < kLptBuckets; ++j) cnt[j] += __popcll(__ballot(bk == j));
  }
  int want = -1;
#pragma unroll
  for (int j = kLptBuckets - 1; j >= 0; --j) {
    if (want < 0) {
      if (k2 < cnt[j]) want = j;
      else k2 -= cnt[j];
    }
  }
  for (int b0 = 0; b0 < a.batch; b0 += 64) {
    int np = 0;
    const int bk = b0 + lane < a.batch ? last_of(b0 + lane, np) : -1;
    const unsigned long long mask = __ballot(bk == want);
    const int c = __popcll(mask);
    if (k2 < c) {
      const int below = __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                                  __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0));
      const unsigned long long hit = __ballot(bk == want && below == (int)k2);
      const int hl = __ffsll((long long)hit) - 1;
      b = b0 + hl;
      const int npb = readlane_i(np, hl);
      p = npb > 0 ? npb - 1 : 0;
      return true;
    }
    k2 -= c;
  }
  return false;  // not reached: the bucket counts cover every sequence
}

template <int DT, int HD, int R, bool ROPE>
__global__ void __launch_bounds__(kWavesPerBlock * kWave)
    decode_kernel(DecodeKArgs a) {
  using C = DCfg<DT, HD, R>;
  __shared__ float p_lds_all[kWavesPerBlock][C::TILE * C::PP];
  __shared__ int ctx_lds[kCtxCache];
  // The new token's K and V rows as stored (fused append), per wave.
  __shared__ __attribute__((aligned(16))) char new_lds_all[kWavesPerBlock][2 * C::RB];

  // The wave index is uniform within a wave; readfirstlane tells the
  // compiler so, which keeps every per-wave quantity in SGPRs.
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  float* p_lds = p_lds_all[wave];

  const int H = a.kvh * a.rtot;
  const int rq = a.rq;  // query heads of this launch per group (<= R)
  const int BS = 1 << a.bs_log2;
  const int PT = a.part_tokens;
  const long long item = (long long)blockIdx.x * kWavesPerBlock + wave;
  const int g = (int)(item % a.kvh);
  int b = 0, p = 0;
  CtxLens cl{a.context_lens, ctx_lds, 0};
  if (a.direct) {  // launch-uniform
    // Small launches: (b, p) straight from the item, so the wave issues its
    // context length, table slice and Q loads at once (no staging round
    // trip); slots past a sequence's partitions exit below.
    const long long rest = item / a.kvh;
    b = (int)(rest / a.max_parts);
    p = (int)(rest - (long long)b * a.max_parts);
    if (b >= a.batch) return;
  } else {
    cl.n = min(a.batch, kCtxCache);
    for (int i = threadIdx.x; i < cl.n; i += kWavesPerBlock * kWave) ctx_lds[i] = a.context_lens[i];
    __syncthreads();
    if (!locate_pair(a, cl, item / a.kvh, lane, BS, b, p)) return;
  }

  const int G = lane >> 4;
  const int col = lane & 15;
  const int t_begin = p * PT;
  const int blk_begin = t_begin >> a.bs_log2;
  // Loads that do not depend on the context length go out first: the block
  // ids a full partition spans (partitions are block-aligned and span at
  // most 64 blocks, decode_plan; lane i holds entry blk_begin + i, ids past
  // the sequence's blocks are never used) and, without RoPE, the Q group as
  // the MFMA A operand (row = head lane % 16, k-slice lane / 16).
  const int span = PT >> a.bs_log2 > 1 ? PT >> a.bs_log2 : 1;
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

  const int ctx_raw = cl[b];
  const int ctx = clamp_ctx(a, ctx_raw, BS);
  const bool clamped = ctx != ctx_raw;
  if (clamped && lane == 0 && p == 0) atomicOr(a.err, PKV_EBIT_LENGTH);
  const int n_parts = (ctx + PT - 1) / PT;
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

  const int t_end = min(ctx, t_begin + PT);
  const int nblk = ((t_end - 1) >> a.bs_log2) - blk_begin + 1;  // <= span
  const int new_pos = (a.k_new != nullptr && !clamped) ? ctx - 1 : -1;

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
  if (lane < nblk && (tbl < 0 || tbl >= a.num_blocks)) {
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
  const bool has_new = new_pos >= 0 && p == n_parts - 1;
  if (has_new) {
    int blk = readlane_i(tbl, (new_pos >> a.bs_log2) - blk_begin);
    size_t off = ((size_t)blk * BS + (new_pos & (BS - 1))) * slot_stride + head_off;
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
        if (a.store_new) {
          st16(kst + lane * 16, k1);
          st16(kst + (lane + C::CH / 2) * 16, k2);
        }
      }
      if (lane < C::CH) {
        float x[C::EPL];
        load_elems<DT, C::EPL>(vrow, lane * C::EPL, a.in_f32, x);
        const u32x4 v1 = pack16<DT, C::EPL>(x);
        st16(new_lds + C::RB + lane * 16, v1);
        if (a.store_new) st16(vst + lane * 16, v1);
      }
    } else if (lane < C::CH) {
      const u32x4 k1 = ld16(a.k_new + ((size_t)b * a.kvh + g) * C::RB + lane * 16);
      const u32x4 v1 = ld16(a.v_new + ((size_t)b * a.kvh + g) * C::RB + lane * 16);
      st16(new_lds + lane * 16, k1);
      st16(new_lds + C::RB + lane * 16, v1);
      if (a.store_new) {
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

  // K fragment f of sub-tile st: token lane % 16, k-slice lane / 16; the four
  // lanes of a token read 64 contiguous bytes.  block_size >= 16, so the 16
  // tokens of a sub-tile share one block.
  auto k_row = [&](int tile_base, int st) {
    const int t0 = min(tile_base + 16 * st, t_end - 1);
    const int tok = min(tile_base + 16 * st + col, t_end - 1);
    const char* base = kh + (size_t)readlane_i(tbl, (t0 >> lg) - blk_begin) * blk_stride;
    return base + ((uint32_t)((tok & tmask) * slot_stride) + 16 * G);
  };
  // V load i of a tile: TPL consecutive tokens (one block), lane = (token
  // group tg, 16-byte chunk c): consecutive lanes read consecutive bytes.
  auto v_chunk = [&](int tile_base, int i) {
    const int t0 = min(tile_base + i * C::TPL, t_end - 1);
    const int tok = min(tile_base + i * C::TPL + tg, t_end - 1);
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
  // launches: 4.5 % faster than with ordinary stores).
  const size_t pair = (size_t)b * a.kvh + g;
  float* ml = a.part_ml + (pair * a.max_parts + p) * R * 2;
  float* po = a.part_o + (pair * a.max_parts + p) * R * HD;
#pragma unroll
  for (int h = 0; h < R; ++h) {
    if (h % NG != tg || h >= rq) continue;
#pragma unroll
    for (int e = 0; e < C::EPL; e += 4)
      __builtin_nontemporal_store(f32x4{o[h][e], o[h][e + 1], o[h][e + 2], o[h][e + 3]},
                                  reinterpret_cast<f32x4*>(po + h * HD + c * C::EPL + e));
  }
  // (m, l) of the R heads: one store instruction from lanes 0 .. 2R-1 (a
  // contiguous 8R-byte write) rather than 2R separate 4-byte writes.
  if (lane < 2 * R) {
    float v = 0.0f;
#pragma unroll
    for (int h = 0; h < R; ++h)
      if ((lane >> 1) == h) v = (lane & 1) ? lh[h] : mh[h];
    __builtin_nontemporal_store(v, ml + lane);
  }
}

// Merge of the partitions of (b, g) for sequences with more than one
// partition: M = max_p m_p, L = sum_p l_p 2^(m_p - M),
// O = sum_p O_p 2^(m_p - M) / L (all in the exp2 domain of the main kernel).
// One wave per query head (b, g, h).  The first loads go out together,
// before the context length that says how many partitions there are has
// arrived: the (m, l) pairs of partitions 0..63 (one per lane) and the first
// PPI * MU partial rows O_p (16-byte chunks, HD / 4 lanes per row,
// 64 / (HD / 4) rows per load instruction), all within the launch's
// max_parts slots of the pair; entries of partitions the sequence does not
// have are masked out once the length is known.  Longer sequences load the
// rest in further rounds.  The row groups are summed with lane shuffles at
// the end.  Context clamping is identical to the main kernel.
// Row loads in flight per lane: 8 for rows of 64 (32 partitions per round,
// which covers the small launches of short rows), else 4 (8 or 16 rows).
template <int HD>
constexpr int merge_unroll() { return HD == 64 ? 8 : 4; }

__device__ __forceinline__ float wave_max_f(float x) {
#pragma unroll
  for (int mk = 1; mk < kWave; mk <<= 1) x = fmaxf(x, shfl_xor_f(x, mk));
  return x;
}
__device__ __forceinline__ float wave_sum_f(float x) {
#pragma unroll
  for (int mk = 1; mk < kWave; mk <<= 1) x += shfl_xor_f(x, mk);
  return x;
}

template <int HD>
__global__ void __launch_bounds__(kWavesPerBlock * kWave)
    decode_merge_kernel(DecodeKArgs a, int R, int dt) {
  // R: the main kernel's group width (partials hold R heads per partition);
  // heads h < a.rq of each group are merged.
  constexpr int LPR = HD / 4;      // lanes per partial row (16 B each)
  constexpr int PPI = kWave / LPR; // partial rows per load instruction
  constexpr int kMergeUnroll = merge_unroll<HD>();
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const long long qh = (long long)blockIdx.x * kWavesPerBlock + wave;  // (b, g, h)
  const long long pair = qh / a.rq;
  const int h = (int)(qh - pair * a.rq);
  if (pair >= (long long)a.batch * a.kvh) return;
  const int b = (int)(pair / a.kvh);
  const int g = (int)(pair % a.kvh);
  const int BS = 1 << a.bs_log2;
  const size_t pstride_ml = (size_t)R * 2;   // floats between partitions
  const size_t pstride_o = (size_t)R * HD;
  const float* mlb = a.part_ml + (size_t)pair * a.max_parts * pstride_ml + 2 * h;
  const int q = lane / LPR;  // row group
  const int c = lane % LPR;  // 16-byte chunk of the row
  const float* pob = a.part_o + ((size_t)pair * a.max_parts * R + h) * HD + 4 * c;
  const int mp = a.max_parts;

  const int ctx_raw = a.context_lens[b];
  float m0 = -INFINITY, l0 = 0.0f;  // partition `lane`
  if (lane < mp) {
    m0 = mlb[(size_t)lane * pstride_ml];
    l0 = mlb[(size_t)lane * pstride_ml + 1];
  }
  f32x4 ov0[kMergeUnroll];
  float mv0[kMergeUnroll];
#pragma unroll
  for (int u = 0; u < kMergeUnroll; ++u) {
    const int pp = u * PPI + q;
    const bool ok = pp < mp;
    ov0[u] = ok ? *reinterpret_cast<const f32x4*>(pob + (size_t)pp * pstride_o)
                : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    mv0[u] = ok ? mlb[(size_t)pp * pstride_ml] : -INFINITY;
  }
  const int ctx = clamp_ctx(a, ctx_raw, BS);
  const int n_parts = (ctx + a.part_tokens - 1) / a.part_tokens;
  if (n_parts <= 1) return;
  // entries of partitions past n_parts hold whatever the slots held: select,
  // never multiply, them away
  if (lane >= n_parts) {
    m0 = -INFINITY;
    l0 = 0.0f;
  }
#pragma unroll
  for (int u = 0; u < kMergeUnroll; ++u)
    if (u * PPI + q >= n_parts) {
      ov0[u] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      mv0[u] = -INFINITY;
    }
  float M = m0;
  for (int p0 = kWave; p0 < n_parts; p0 += kWave)
    if (p0 + lane < n_parts) M = fmaxf(M, mlb[(size_t)(p0 + lane) * pstride_ml]);
  M = wave_max_f(M);
  float L = lane < n_parts ? fast_exp2(m0 - M) * l0 : 0.0f;
  for (int p0 = kWave; p0 < n_parts; p0 += kWave) {
    const int pp = p0 + lane;
    if (pp < n_parts) {
      const float* e = mlb + (size_t)pp * pstride_ml;
      L += fast_exp2(e[0] - M) * e[1];
    }
  }
  L = wave_sum_f(L);

  f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int u = 0; u < kMergeUnroll; ++u) {
    const float w = fast_exp2(mv0[u] - M);  // 0 for absent rows
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, ov0[u][i], acc[i]);
  }
  for (int p0 = PPI * kMergeUnroll; p0 < n_parts; p0 += PPI * kMergeUnroll) {
    f32x4 ov[kMergeUnroll];
    float mv[kMergeUnroll];
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const int pp = p0 + u * PPI + q;
      const bool ok = pp < n_parts;
      ov[u] = ok ? *reinterpret_cast<const f32x4*>(pob + (size_t)pp * pstride_o)
                 : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      mv[u] = ok ? mlb[(size_t)pp * pstride_ml] : -INFINITY;
    }
#pragma unroll
    for (int u = 0; u < kMergeUnroll; ++u) {
      const float w = fast_exp2(mv[u] - M);  // 0 for absent rows
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, ov[u][i], acc[i]);
    }
  }
#pragma unroll
  for (int mk = LPR; mk < kWave; mk <<= 1)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] += shfl_xor_f(acc[i], mk);
  if (lane >= LPR) return;

  const float inv = 1.0f / L;
  const size_t eo = ((size_t)b * a.kvh * a.rtot + g * a.rtot + a.h0 + h) * HD + 4 * c;
  if (a.out_f32) {
    *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + eo) =
        f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
  } else {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = dt == PKV_BF16 ? f32_to_bf16_bits(acc[i] * inv) : f32_to_f16_bits(acc[i] * inv);
    typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
    *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(a.out) + eo) =
        u32x2{w[0] | (w[1] << 16), w[2] | (w[3] << 16)};
  }
}

template <int DT, int HD, int R>
hipError_t launch_t(const DecodeKArgs& k, long long items, hipStream_t s) {
  unsigned grid = (unsigned)((items + kWavesPerBlock - 1) / kWavesPerBlock);
  if (k.rope_cos)
    decode_kernel<DT, HD, R, true><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
  else
    decode_kernel<DT, HD, R, false><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
  return hipGetLastError();
}

// Group width of the kernel instantiated for a GQA ratio (a slice of at
// most 16 heads of it): the ratio itself or the next of 1, 2, 4, 8, 16.
int group_width(int r) {
  int w = 1;
  while (w < r && w < 16) w <<= 1;
  return w;
}

template <int DT, int HD>
hipError_t launch_r(int R, const DecodeKArgs& k, long long items, hipStream_t s) {
  switch (R) {
    case 1: return launch_t<DT, HD, 1>(k, items, s);
    case 2: return launch_t<DT, HD, 2>(k, items, s);
    case 4: return launch_t<DT, HD, 4>(k, items, s);
    case 8: return launch_t<DT, HD, 8>(k, items, s);
    case 16: return launch_t<DT, HD, 16>(k, items, s);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t launch_hd(int HD, int R, const DecodeKArgs& k, long long items, hipStream_t s) {
  switch (HD) {
    case 64: return launch_r<DT, 64>(R, k, items, s);
    case 128: return launch_r<DT, 128>(R, k, items, s);
    case 256: return launch_r<DT, 256>(R, k, items, s);
    default: return hipErrorInvalidValue;
  }
}

// Launches of at most this many (sequence, kv head, partition) slots map
// waves to items directly instead of through the longest-first work list:
// they fit on the GPU at once, so dispatch order buys nothing, and the
// direct mapping saves the context-length staging round trip.
constexpr long long kDirectMaxItems = 2048;

int ilog2i(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

}  // namespace

bool decode_supported(const pkv_pool* p, int n_head) {
  if (n_head <= 0 || n_head % p->n_kv_head != 0) return false;
  return p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256;
}

void decode_plan(const pkv_pool* p, int batch, int n_head, int max_context_len,
                 int* part_tokens, int* max_parts) {
  (void)n_head;
  long long pairs = (long long)batch * p->n_kv_head;
  int mc = max_context_len > 0 ? max_context_len : 1;
  // Partition length: 1024 tokens (512 KB of K+V per bf16 head of 128).
  // The split-context partials (m, l, O) are written in the middle of the
  // K/V read stream, and those writes cost far more than their bytes
  // (measured on the Llama-3-8B decode: 0-10 % of the kernel depending on
  // where the workspace lands in HBM with 512-token partitions, a third of
  // that with 1024); the longest-first work list keeps the longer items
  // from lengthening the tail.  Shorter partitions are used when the batch
  // is too small to give every CU several waves.
  int pt = PKV_DECODE_PART_MAX;
  while (pt > 64 && pairs * ((mc + pt - 1) / pt) < PKV_DECODE_MIN_ITEMS) pt >>= 1;
  // The per-partition table slice must fit one wave (<= 64 block ids).
  // Partitions start at multiples of pt, so with block_size <= pt they are
  // block-aligned and span pt / block_size blocks (one block otherwise).
  while (pt > 64 && (pt >> ilog2i(p->block_size)) > 64) pt >>= 1;
  *part_tokens = pt;
  *max_parts = (mc + pt - 1) / pt;
}

size_t decode_workspace_bytes(const pkv_pool* p, int batch, int n_head,
                              int max_context_len) {
  int pt = 0, mp = 0;
  decode_plan(p, batch, n_head, max_context_len, &pt, &mp);
  size_t pairs = (size_t)batch * p->n_kv_head;
  size_t R = (size_t)group_width(n_head / p->n_kv_head);  // partial heads per partition
  if (mp <= 1) return 256;
  size_t ml = ((pairs * mp * R * 2 * 4 + 255) / 256) * 256;
  size_t po = pairs * mp * R * (size_t)p->head_dim * 4;
  return ml + po;
}

hipError_t launch_decode(const pkv_pool* p, int layer, const DecodeArgs& a, char* partials,
                         hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  int pt = 0, mp = 0;
  decode_plan(p, a.batch, a.n_head, a.max_context_len, &pt, &mp);
  size_t pairs = (size_t)a.batch * p->n_kv_head;
  const int rtot = a.n_head / p->n_kv_head;
  const int R = group_width(rtot);  // kernel width; ratios above 16 run in slices of 16
  DecodeKArgs k{};
  k.k_pool = p->layer_k(layer);
  k.v_pool = p->layer_v(layer);
  k.q = reinterpret_cast<const char*>(a.q);
  k.out = a.out;
  k.out_f32 = a.out_dtype == PKV_F32;
  k.block_tables = a.block_tables;
  k.mbps = a.max_blocks_per_seq;
  k.context_lens = a.context_lens;
  k.max_context_len = a.max_context_len;
  k.batch = a.batch;
  k.kvh = p->n_kv_head;
  k.num_blocks = p->num_blocks;
  k.bs_log2 = ilog2i(p->block_size);
  k.part_tokens = pt;
  k.max_parts = mp;
  k.scale_log2 = a.scale * 1.4426950408889634f;
  k.k_new = reinterpret_cast<const char*>(a.k_new);
  k.v_new = reinterpret_cast<const char*>(a.v_new);
  k.rope_cos = a.rope_cos;
  k.rope_sin = a.rope_sin;
  k.rope_max = a.rope_max;
  k.positions = a.positions;
  k.in_f32 = a.in_f32;
  k.rtot = rtot;
  // small launches (every wave resident at once): direct wave mapping
  k.direct = (long long)pairs * mp <= kDirectMaxItems;
  size_t ml_bytes = ((pairs * mp * R * 2 * 4 + 255) / 256) * 256;
  k.part_ml = reinterpret_cast<float*>(partials);
  k.part_o = reinterpret_cast<float*>(partials + ml_bytes);
  k.err = p->err;
  long long items = (long long)pairs * mp;
  hipError_t e = hipSuccess;
  // Slices of at most 16 query heads per group, each a main launch and its
  // merge (stream-ordered, so the slices share the workspace); the first
  // slice stores the new token, every slice attends to it.
  for (int h0 = 0; h0 < rtot; h0 += 16) {
    k.h0 = h0;
    k.rq = rtot - h0 < R ? rtot - h0 : R;
    k.store_new = h0 == 0;
    const bool timed = h0 == 0;  // the profile events bracket the first slice
    if (timed && ev_begin && (e = hipEventRecord(ev_begin, stream)) != hipSuccess) return e;
    switch (p->dtype) {
      case PKV_F32: e = launch_hd<PKV_F32>(p->head_dim, R, k, items, stream); break;
      case PKV_F16: e = launch_hd<PKV_F16>(p->head_dim, R, k, items, stream); break;
      default: e = launch_hd<PKV_BF16>(p->head_dim, R, k, items, stream); break;
    }
    if (e != hipSuccess) return e;
    if (timed && ev_end && (e = hipEventRecord(ev_end, stream)) != hipSuccess) return e;
    if (mp <= 1) continue;
    unsigned grid = (unsigned)((pairs * k.rq + kWavesPerBlock - 1) / kWavesPerBlock);
    switch (p->head_dim) {
      case 64: decode_merge_kernel<64><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
      case 128: decode_merge_kernel<128><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
      default: decode_merge_kernel<256><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
    }
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  return e;
}

// ---- scratch of the allocation-free entry point -------------------------
// The split-context partials of pkv_decode_attention_noalloc live in this
// file-scope device array: every GPU the library runs on holds its own copy
// for the life of the process.  Host code never uses the array's name as an
// address (on the host it is only a stand-in for the symbol): the address of
// each device's copy comes from hipGetSymbolAddress, looked up once per
// device with that device current, and is what the kernels receive.
// Nothing in it needs clearing between calls: every partial a merge reads
// was written by the same call's main kernel.
constexpr size_t kNoallocScratch = PKV_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kNoallocScratch];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static char* g_scratch_ptr[kMaxDevices] = {};

size_t noalloc_scratch_bytes() { return kNoallocScratch; }

hipError_t noalloc_scratch(int device, char** ptr) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* addr = nullptr;
    const hipError_t e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = static_cast<char*>(addr);
  }
  *ptr = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace pkv
