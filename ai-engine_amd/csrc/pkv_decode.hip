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

#include "pkv_decode_dev.h"

namespace pkv {
namespace {

template <int DT, int HD, int R, bool ROPE, bool SB>
__global__ void __launch_bounds__(kWavesPerBlock * kWave)
    decode_kernel(DecodeKArgs a) {
  __shared__ DecodeSmem<DT, HD, R, ROPE> sm;
  decode_body<DT, HD, R, ROPE, SB>(a, blockIdx.x, sm);
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
// rest in further rounds.  The row groups are summed with permlane swaps at
// the end.  Context clamping is identical to the main kernel.
// Row loads in flight per lane: 8 for rows of 64 (32 partitions per round,
// which covers the small launches of short rows), else 4 (8 or 16 rows).
template <int HD>
constexpr int merge_unroll() { return HD == 64 ? 8 : 4; }

// Cross-lane steps without LDS round trips: DPP rotations within each
// 16-lane row, and the gfx950 permlane swaps that exchange a lane's value
// with lane ^ 16 or lane ^ 32 (each returns the pair; either order of the
// two operands gives the same combination, so every lane of a pair holds
// the same result).
template <int ROR>
__device__ __forceinline__ float row_ror_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x120 + ROR, 0xf, 0xf, false));
}
template <bool MAX>
__device__ __forceinline__ float comb(float a, float b) { return MAX ? fmaxf(a, b) : a + b; }
template <bool MAX>
__device__ __forceinline__ float with_lane_xor16(float x) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return comb<MAX>(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
template <bool MAX>
__device__ __forceinline__ float with_lane_xor32(float x) {
  const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return comb<MAX>(__uint_as_float(a[0]), __uint_as_float(a[1]));
}
// Max / sum over the wave, the result in every lane.
template <bool MAX>
__device__ __forceinline__ float wave_all(float x) {
  x = comb<MAX>(x, row_ror_f<8>(x));
  x = comb<MAX>(x, row_ror_f<4>(x));
  x = comb<MAX>(x, row_ror_f<2>(x));
  x = comb<MAX>(x, row_ror_f<1>(x));
  return with_lane_xor32<MAX>(with_lane_xor16<MAX>(x));
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
  // (b, g, h) < 2^26: decode_validate refuses larger launches
  const unsigned qh = blockIdx.x * kWavesPerBlock + wave;
  const unsigned pair = qh / (unsigned)a.rq;
  const int h = (int)(qh - pair * (unsigned)a.rq);
  if (pair >= (unsigned)a.batch * (unsigned)a.kvh) return;
  const int b = (int)(pair / (unsigned)a.kvh);
  const int g = (int)(pair - (unsigned)b * (unsigned)a.kvh);
  const int BS = 1 << a.bs_log2;
  const size_t pstride_ml = kMlFloats;       // floats between partitions
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
  // the attended keys, as the main kernel lays them out
  const int ctx = clamp_ctx(a, attended_len(a, b, ctx_raw), BS);
  const int n_parts = part_count(ctx, a.pt_log2, a.sub_log2);
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
  M = wave_all<true>(M);
  float L = lane < n_parts ? fast_exp2(m0 - M) * l0 : 0.0f;
  for (int p0 = kWave; p0 < n_parts; p0 += kWave) {
    const int pp = p0 + lane;
    if (pp < n_parts) {
      const float* e = mlb + (size_t)pp * pstride_ml;
      L += fast_exp2(e[0] - M) * e[1];
    }
  }
  L = wave_all<false>(L);

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
  // sum the row groups: lanes c, c + LPR, ... hold one 16-byte chunk
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (LPR <= 16) acc[i] = with_lane_xor16<false>(acc[i]);
    if constexpr (LPR <= 32) acc[i] = with_lane_xor32<false>(acc[i]);
  }
  if (lane >= LPR) return;

  const float inv = 1.0f / L;
  // chunk c of a partial row holds elements (c % CH) EPL + 4 (c / CH) ..
  // (the main kernel's store order; CH = HD / EPL 16-byte chunks of a row)
  const int epl = dt == PKV_F32 ? 4 : 8;
  const int chs = HD / epl;
  const size_t eo = ((size_t)b * a.kvh * a.rtot + g * a.rtot + a.h0 + h) * HD +
                    (c % chs) * epl + 4 * (c / chs);
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

// Block sizes below 16 take the kernels with per-lane block ids.
template <int DT, int HD, int R>
hipError_t launch_t(const DecodeKArgs& k, long long items, hipStream_t s) {
  unsigned grid = (unsigned)((items + kWavesPerBlock - 1) / kWavesPerBlock);
  const bool sb = k.bs_log2 < 4;
  if (k.rope_cos) {
    if (sb) decode_kernel<DT, HD, R, true, true><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
    else decode_kernel<DT, HD, R, true, false><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
  } else {
    if (sb) decode_kernel<DT, HD, R, false, true><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
    else decode_kernel<DT, HD, R, false, false><<<grid, kWavesPerBlock * kWave, 0, s>>>(k);
  }
  return hipGetLastError();
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

int group_width(int r) {
  int w = 1;
  while (w < r && w < 16) w <<= 1;
  return w;
}

bool decode_supported(const pkv_pool* p, int n_head) {
  if (n_head <= 0 || n_head % p->n_kv_head != 0) return false;
  return p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256;
}

void decode_plan(const pkv_pool* p, int batch, int n_head, int max_context_len,
                 int* part_tokens, int* max_parts, int* sub_tokens) {
  (void)n_head;
  long long pairs = (long long)batch * p->n_kv_head;
  const long long mc = max_context_len > 0 ? max_context_len : 1;
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
  int mp = (int)((mc + pt - 1) / pt);  // <= 2^25 for max_context_len < 2^31
  // Work-list launches of full-length partitions cut each context's last pt
  // tokens in two (block-aligned while block_size <= pt / 2): the final
  // round of waves then holds items of at most pt / 2 tokens instead of
  // 0 .. pt.
  // Measured on the Llama-3-8B layer shape (ctx U[512, 4096], bf16), both
  // plans launched on one pool (one HBM placement), alternating: 205-211
  // against 225 us per launch at B = 128 (4096 items); 0.5-1.4 % faster at
  // B = 256 (8192 items; four processes), and on the Llama-3-70B stage
  // (B = 128, 8192 items) -1.0 to +0.5 %; 1.0 % slower at B = 384 and 2.6 %
  // at B = 512, where the extra partial writes and merge reads outweigh the
  // shorter tail.  So only lists of up to PKV_DECODE_SUB_SPLIT_MAX_ITEMS
  // full-length items are split.
  int sub = pt;
  if (pt == PKV_DECODE_PART_MAX && pairs * mp > kDirectMaxItems &&
      pairs * mp <= PKV_DECODE_SUB_SPLIT_MAX_ITEMS &&
      p->block_size <= pt / PKV_DECODE_SUB_SPLIT) {
    sub = pt / PKV_DECODE_SUB_SPLIT;
    mp += PKV_DECODE_SUB_SPLIT - 1;
  }
  *part_tokens = pt;
  *max_parts = mp;
  if (sub_tokens) *sub_tokens = sub;
}

size_t decode_workspace_bytes(const pkv_pool* p, int batch, int n_head,
                              int max_context_len) {
  int pt = 0, mp = 0;
  decode_plan(p, batch, n_head, max_context_len, &pt, &mp);
  size_t pairs = (size_t)batch * p->n_kv_head;
  size_t R = (size_t)group_width(n_head / p->n_kv_head);  // partial heads per partition
  if (mp <= 1) return 256;
  size_t ml = ((pairs * mp * kMlFloats * 4 + 255) / 256) * 256;
  size_t po = pairs * mp * R * (size_t)p->head_dim * 4;
  return ml + po;
}

DecodeKArgs decode_kargs(const pkv_pool* p, int layer, const DecodeArgs& a, char* partials,
                         int h0, long long* items) {
  int pt = 0, mp = 0, sub = 0;
  decode_plan(p, a.batch, a.n_head, a.max_context_len, &pt, &mp, &sub);
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
  k.sub_tokens = sub;
  k.pt_log2 = ilog2i(pt);
  k.sub_log2 = ilog2i(sub);
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
  size_t ml_bytes = ((pairs * mp * kMlFloats * 4 + 255) / 256) * 256;
  k.part_ml = reinterpret_cast<float*>(partials);
  k.part_o = reinterpret_cast<float*>(partials + ml_bytes);
  k.err = p->err;
  k.h0 = h0;
  k.rq = rtot - h0 < R ? rtot - h0 : R;
  k.store_new = h0 == 0;  // the first slice stores the new token, every slice attends to it
  *items = (long long)pairs * mp;
  return k;
}

hipError_t launch_decode_merge(const pkv_pool* p, const DecodeKArgs& k, hipStream_t stream) {
  if (k.max_parts <= 1) return hipSuccess;
  const int R = group_width(k.rtot);
  const size_t pairs = (size_t)k.batch * k.kvh;
  unsigned grid = (unsigned)((pairs * k.rq + kWavesPerBlock - 1) / kWavesPerBlock);
  switch (p->head_dim) {
    case 64: decode_merge_kernel<64><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
    case 128: decode_merge_kernel<128><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
    default: decode_merge_kernel<256><<<grid, kWavesPerBlock * kWave, 0, stream>>>(k, R, p->dtype); break;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const pkv_pool* p, int layer, const DecodeArgs& a, char* partials,
                         hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  const int rtot = a.n_head / p->n_kv_head;
  const int R = group_width(rtot);
  hipError_t e = hipSuccess;
  // Slices of at most 16 query heads per group, each a main launch and its
  // merge (stream-ordered, so the slices share the workspace).
  for (int h0 = 0; h0 < rtot; h0 += 16) {
    long long items = 0;
    const DecodeKArgs k = decode_kargs(p, layer, a, partials, h0, &items);
    const bool timed = h0 == 0;  // the profile events bracket the first slice
    if (timed && ev_begin && (e = hipEventRecord(ev_begin, stream)) != hipSuccess) return e;
    switch (p->dtype) {
      case PKV_F32: e = launch_hd<PKV_F32>(p->head_dim, R, k, items, stream); break;
      case PKV_F16: e = launch_hd<PKV_F16>(p->head_dim, R, k, items, stream); break;
      default: e = launch_hd<PKV_BF16>(p->head_dim, R, k, items, stream); break;
    }
    if (e != hipSuccess) return e;
    if (timed && ev_end && (e = hipEventRecord(ev_end, stream)) != hipSuccess) return e;
    if ((e = launch_decode_merge(p, k, stream)) != hipSuccess) return e;
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
