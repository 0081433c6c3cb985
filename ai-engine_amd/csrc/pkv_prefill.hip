// pkv_prefill.hip -- chunked-prefill attention over the paged pool (gfx950).
//
// Replaces the attention of Transformer::prefill_seq
// (crates/ai-engine-candle/src/paged/transformer.rs:139-148,179-196: causal
// mask j > i -> -inf, GQA expand, q k^T * scale, softmax, att v) and
// generalises it to a prompt chunk with a prior context already in the pool:
// sequence s has q_len queries at positions ctx - q_len + i, each attending
// keys 0 .. its position.  The chunk's own K/V rows are stored first with
// pkv_append (the reference's per-token KvPool::write loop, :173-177).
//
// Work decomposition: one wavefront per (sequence, kv head, tile of 32 rows),
// a row being a (query token, GQA head) pair, heads consecutive -- so K/V
// tiles are shared by the whole query group.  Key tiles of 32 keys stream
// from the pool through the block table.
//
//   S^T = K Q^T on MFMA (K fragments straight from HBM as the A operand, the
//   rows' Q as the B operand).  The accumulator layout puts, in each lane,
//   the scores of 8 keys (two 16-key tiles x 4) of ONE row (lane % 16):
//   exactly the per-lane k-slice of the B operand of O^T = V^T P^T under a
//   consistent permutation of the key index, so P never leaves registers.
//   V^T is the A operand, gathered from a padded LDS copy of the V tile
//   (16-bit gathers, conflict-free).  P is split into a 16-bit high part and
//   a 16-bit residual, two MFMAs, so the weights keep ~16 significant bits
//   (f32 pools use v_mfma_f32_16x16x4f32 with exact fp32 P).  Online softmax
//   per row in the exp2 domain; fp32 accumulation throughout.
#include <type_traits>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kPWaves = 4;  // waves per workgroup (independent items)
constexpr int kKT = 32;     // keys per tile (two 16-key MFMA tiles)

template <int DT, int HD, int R>
struct PCfg {
  static constexpr int E = DT == PKV_F32 ? 4 : 2;
  static constexpr int RB = HD * E;                 // row bytes
  static constexpr int NF = RB / 64;                // 16-B fragments per lane per row
  static constexpr int NR = (HD <= 128 && DT != PKV_F32) ? 2 : 1;  // 16-row tiles per wave
  static constexpr int ROWS = 16 * NR;
  static constexpr int ND = HD / 16;                // 16-dim tiles of O^T
  static constexpr int CH = RB / 16;                // 16-B chunks per row
  static constexpr int VPITCH = RB + (DT == PKV_F32 ? 16 : 8);  // LDS row pitch (bytes)
  static constexpr int TPL = 64 / CH;               // keys per V load
  static constexpr int NVL = kKT / TPL;             // V loads per key tile
};

struct PrefillKArgs {
  const char* k_pool;
  const char* v_pool;
  const char* q;
  void* out;
  int out_f32;
  const int32_t* cu_q_lens;
  const int32_t* context_lens;
  const int32_t* block_tables;
  int mbps;
  int n_seqs;
  int kvh;
  int num_blocks;
  int bs_log2;
  int max_q_len;
  int max_context_len;
  int row_tiles;  // ceil(max_q_len * R / ROWS): grid stride per (seq, head)
  float scale_log2;
  uint32_t* err;
};

template <int DT>
__device__ __forceinline__ uint32_t to16(float x) {
  return DT == PKV_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
}
template <int DT>
__device__ __forceinline__ float from16(uint32_t h) {
  return DT == PKV_BF16 ? bf16lo(h) : f16lo(h);
}

template <int DT, int HD, int R>
__global__ void __launch_bounds__(kPWaves * kWave) prefill_kernel(PrefillKArgs a) {
  using C = PCfg<DT, HD, R>;
  __shared__ __attribute__((aligned(16))) char v_lds_all[kPWaves][kKT * C::VPITCH];

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  char* v_lds = v_lds_all[wave];
  const int G = lane >> 4;
  const int col = lane & 15;

  // item = (seq, kv head, row tile); row tiles in descending order so the
  // tiles that see the most keys are dispatched first
  const long long item = (long long)blockIdx.x * kPWaves + wave;
  const int rt = a.row_tiles - 1 - (int)(item % a.row_tiles);
  const long long sg = item / a.row_tiles;
  const int g = (int)(sg % a.kvh);
  const int s = (int)(sg / a.kvh);
  if (s >= a.n_seqs) return;

  const int q0 = a.cu_q_lens[s];
  const int q_len_raw = a.cu_q_lens[s + 1] - q0;
  const int q_len = min(q_len_raw, a.max_q_len);
  if (q_len_raw > a.max_q_len && lane == 0 && rt == 0 && g == 0) atomicOr(a.err, PKV_EBIT_LENGTH);
  const int BS = 1 << a.bs_log2;
  int ctx = a.context_lens[s];
  if (ctx > a.max_context_len || ctx > a.mbps * BS || ctx < q_len || q_len < 0) {
    if (lane == 0 && rt == 0 && g == 0) atomicOr(a.err, PKV_EBIT_LENGTH);
    return;
  }
  const int row0 = rt * C::ROWS;
  if (row0 >= q_len * R) return;
  const int prior = ctx - q_len;
  const int H = a.kvh * R;
  const int tmask = BS - 1;
  const size_t slot_stride = (size_t)a.kvh * C::RB;
  const size_t blk_stride = (size_t)BS * slot_stride;
  const char* kh = a.k_pool + (size_t)g * C::RB;
  const char* vh = a.v_pool + (size_t)g * C::RB;
  const int32_t* table = a.block_tables + (size_t)s * a.mbps;

  // Rows of this lane (B operand / output): row n = 16 * rn + col.
  int tok_of[C::NR];
  u32x4 qf[C::NR][C::NF];
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    const int r = row0 + 16 * rn + col;
    const int rc = min(r, q_len * R - 1);
    tok_of[rn] = rc / R;
    const char* qrow = a.q + ((size_t)(q0 + rc / R) * H + g * R + rc % R) * C::RB;
#pragma unroll
    for (int f = 0; f < C::NF; ++f) qf[rn][f] = ld16(qrow + 64 * f + 16 * G);
  }
  // Keys needed: 0 .. prior + last token of the tile.
  const int last_tok = min((row0 + C::ROWS - 1) / R, q_len - 1);
  const int n_keys = prior + last_tok + 1;
  const int n_tiles = (n_keys + kKT - 1) / kKT;

  auto block_of = [&](int key) {
    int blk = table[key >> a.bs_log2];
    if (blk < 0 || blk >= a.num_blocks) {
      atomicOr(a.err, PKV_EBIT_BLOCK);
      blk = 0;
    }
    return blk;
  };

  float m[C::NR], lsum[C::NR];
  f32x4 o[C::ND][C::NR];
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    m[rn] = -INFINITY;
    lsum[rn] = 0.0f;
#pragma unroll
    for (int dm = 0; dm < C::ND; ++dm) o[dm][rn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  const int vtok = lane / C::CH;  // V load mapping: key, 16-B chunk
  const int vch = lane % C::CH;

  for (int t = 0; t < n_tiles; ++t) {
    const int k0 = t * kKT;
    // ---- V tile -> LDS (coalesced loads; keys past n_keys clamped) ----
    u32x4 vreg[C::NVL];
#pragma unroll
    for (int i = 0; i < C::NVL; ++i) {
      const int key = min(k0 + i * C::TPL + vtok, n_keys - 1);
      const char* base = vh + (size_t)block_of(key) * blk_stride;
      vreg[i] = ld16(base + (size_t)(key & tmask) * slot_stride + 16 * vch);
    }
    // ---- K fragments (A operand): key = k0 + 16 km + col ----
    u32x4 kf[2][C::NF];
#pragma unroll
    for (int km = 0; km < 2; ++km) {
      const int key = min(k0 + 16 * km + col, n_keys - 1);
      const char* r = kh + (size_t)block_of(key) * blk_stride +
                      (size_t)(key & tmask) * slot_stride + 16 * G;
#pragma unroll
      for (int f = 0; f < C::NF; ++f) kf[km][f] = ld16(r + 64 * f);
    }
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < C::NVL; ++i) {
      char* dst = v_lds + (i * C::TPL + vtok) * C::VPITCH + 16 * vch;
      *reinterpret_cast<uint64_t*>(dst) = (uint64_t)vreg[i][0] | ((uint64_t)vreg[i][1] << 32);
      *reinterpret_cast<uint64_t*>(dst + 8) = (uint64_t)vreg[i][2] | ((uint64_t)vreg[i][3] << 32);
    }

    // ---- S^T = K Q^T: acc[km][rn][j] = S[key k0 + 16 km + 4 G + j][row] ----
    f32x4 sacc[2][C::NR];
#pragma unroll
    for (int km = 0; km < 2; ++km)
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn) {
        sacc[km][rn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int f = 0; f < C::NF; ++f) mfma_frag<DT>(kf[km][f], qf[rn][f], sacc[km][rn]);
      }

    // ---- causal mask + online softmax per row (rows along lane % 16) ----
    float p[2][C::NR][4];
#pragma unroll
    for (int rn = 0; rn < C::NR; ++rn) {
      const int lim = prior + tok_of[rn];  // last key this row may see
      float tmax = -INFINITY;
#pragma unroll
      for (int km = 0; km < 2; ++km)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int key = k0 + 16 * km + 4 * G + j;
          const float sv = key <= lim ? sacc[km][rn][j] * a.scale_log2 : -INFINITY;
          p[km][rn][j] = sv;
          tmax = fmaxf(tmax, sv);
        }
      tmax = fmaxf(tmax, shfl_xor_f(tmax, 16));
      tmax = fmaxf(tmax, shfl_xor_f(tmax, 32));
      const float mnew = fmaxf(m[rn], tmax);
      const float alpha = fast_exp2(m[rn] - mnew);
      m[rn] = mnew;
      float ssum = 0.0f;
#pragma unroll
      for (int km = 0; km < 2; ++km)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[km][rn][j] = fast_exp2(p[km][rn][j] - mnew);
          ssum += p[km][rn][j];
        }
      lsum[rn] = lsum[rn] * alpha + ssum;  // lane-partial over its 8 keys
#pragma unroll
      for (int dm = 0; dm < C::ND; ++dm) o[dm][rn] *= alpha;
    }
    __builtin_amdgcn_wave_barrier();

    // ---- O^T += V^T P^T ----
    if constexpr (DT == PKV_F32) {
      // k-step (km, j): lane group G supplies key 16 km + 4 G + j.
#pragma unroll
      for (int dm = 0; dm < C::ND; ++dm)
#pragma unroll
        for (int km = 0; km < 2; ++km)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int kl = 16 * km + 4 * G + j;
            const float va = *reinterpret_cast<const float*>(
                v_lds + kl * C::VPITCH + (16 * dm + col) * 4);
#pragma unroll
            for (int rn = 0; rn < C::NR; ++rn)
              o[dm][rn] = __builtin_amdgcn_mfma_f32_16x16x4f32(va, p[km][rn][j], o[dm][rn], 0, 0, 0);
          }
    } else {
      // one 16x16x32 step: lane group G supplies keys {4G..4G+3, 16+4G..16+4G+3}
      u32x4 phi[C::NR], plo[C::NR];
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float x0 = p[w >> 1][rn][(w & 1) * 2];
          const float x1 = p[w >> 1][rn][(w & 1) * 2 + 1];
          const uint32_t h0 = to16<DT>(x0), h1 = to16<DT>(x1);
          phi[rn][w] = h0 | (h1 << 16);
          plo[rn][w] = to16<DT>(x0 - from16<DT>(h0)) | (to16<DT>(x1 - from16<DT>(h1)) << 16);
        }
#pragma unroll
      for (int dm = 0; dm < C::ND; ++dm) {
        u32x4 va;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int kla = (w >> 1) * 16 + 4 * G + (w & 1) * 2;
          const uint16_t* p0 = reinterpret_cast<const uint16_t*>(
              v_lds + kla * C::VPITCH + (16 * dm + col) * 2);
          const uint16_t* p1 = reinterpret_cast<const uint16_t*>(
              v_lds + (kla + 1) * C::VPITCH + (16 * dm + col) * 2);
          va[w] = (uint32_t)*p0 | ((uint32_t)*p1 << 16);
        }
#pragma unroll
        for (int rn = 0; rn < C::NR; ++rn) {
          mfma_frag<DT>(va, phi[rn], o[dm][rn]);
          mfma_frag<DT>(va, plo[rn], o[dm][rn]);
        }
      }
    }
    __builtin_amdgcn_wave_barrier();
  }

  // ---- epilogue: lane holds O^T[dims 16 dm + 4 G + j][row 16 rn + col] ----
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    float l = lsum[rn];
    l += shfl_xor_f(l, 16);
    l += shfl_xor_f(l, 32);
    const int r = row0 + 16 * rn + col;
    if (r >= q_len * R) continue;
    const float inv = 1.0f / l;
    const size_t base = ((size_t)(q0 + r / R) * H + g * R + r % R) * HD;
#pragma unroll
    for (int dm = 0; dm < C::ND; ++dm) {
      const size_t eo = base + 16 * dm + 4 * G;
      if (a.out_f32) {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + eo) = o[dm][rn] * inv;
      } else {
        uint32_t w0 = to16<DT>(o[dm][rn][0] * inv) | (to16<DT>(o[dm][rn][1] * inv) << 16);
        uint32_t w1 = to16<DT>(o[dm][rn][2] * inv) | (to16<DT>(o[dm][rn][3] * inv) << 16);
        *reinterpret_cast<uint64_t*>(reinterpret_cast<uint16_t*>(a.out) + eo) =
            (uint64_t)w0 | ((uint64_t)w1 << 32);
      }
    }
  }
}

template <int DT, int HD, int R>
hipError_t plaunch(PrefillKArgs k, hipStream_t s) {
  using C = PCfg<DT, HD, R>;
  k.row_tiles = (k.max_q_len * R + C::ROWS - 1) / C::ROWS;
  long long items = (long long)k.n_seqs * k.kvh * k.row_tiles;
  if (items <= 0) return hipSuccess;
  unsigned grid = (unsigned)((items + kPWaves - 1) / kPWaves);
  prefill_kernel<DT, HD, R><<<grid, kPWaves * kWave, 0, s>>>(k);
  return hipGetLastError();
}

template <int DT, int HD>
hipError_t plaunch_r(int R, const PrefillKArgs& k, hipStream_t s) {
  switch (R) {
    case 1: return plaunch<DT, HD, 1>(k, s);
    case 2: return plaunch<DT, HD, 2>(k, s);
    case 4: return plaunch<DT, HD, 4>(k, s);
    case 8: return plaunch<DT, HD, 8>(k, s);
    default: return hipErrorInvalidValue;
  }
}

template <int DT>
hipError_t plaunch_hd(int HD, int R, const PrefillKArgs& k, hipStream_t s) {
  switch (HD) {
    case 64: return plaunch_r<DT, 64>(R, k, s);
    case 128: return plaunch_r<DT, 128>(R, k, s);
    case 256:
      if constexpr (DT != PKV_F32) return plaunch_r<DT, 256>(R, k, s);
      return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
  }
}

int ilog2p(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

}  // namespace

bool prefill_supported(const pkv_pool* p, int n_head) {
  if (n_head <= 0 || n_head % p->n_kv_head != 0) return false;
  int R = n_head / p->n_kv_head;
  if (R != 1 && R != 2 && R != 4 && R != 8) return false;
  if (p->dtype == PKV_F32 && p->head_dim > 128) return false;  // register budget
  return p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256;
}

hipError_t launch_prefill(const pkv_pool* p, int layer, const PrefillArgs& a,
                          hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  PrefillKArgs k{};
  k.k_pool = p->layer_k(layer);
  k.v_pool = p->layer_v(layer);
  k.q = reinterpret_cast<const char*>(a.q);
  k.out = a.out;
  k.out_f32 = a.out_dtype == PKV_F32;
  k.cu_q_lens = a.cu_q_lens;
  k.context_lens = a.context_lens;
  k.block_tables = a.block_tables;
  k.mbps = a.max_blocks_per_seq;
  k.n_seqs = a.n_seqs;
  k.kvh = p->n_kv_head;
  k.num_blocks = p->num_blocks;
  k.bs_log2 = ilog2p(p->block_size);
  k.max_q_len = a.max_q_len;
  k.max_context_len = a.max_context_len;
  k.scale_log2 = a.scale * 1.4426950408889634f;
  k.err = p->err;
  int R = a.n_head / p->n_kv_head;
  hipError_t e = hipSuccess;
  if (ev_begin) e = hipEventRecord(ev_begin, stream);
  if (e != hipSuccess) return e;
  switch (p->dtype) {
    case PKV_F32: e = plaunch_hd<PKV_F32>(p->head_dim, R, k, stream); break;
    case PKV_F16: e = plaunch_hd<PKV_F16>(p->head_dim, R, k, stream); break;
    default: e = plaunch_hd<PKV_BF16>(p->head_dim, R, k, stream); break;
  }
  if (e == hipSuccess && ev_end) e = hipEventRecord(ev_end, stream);
  return e;
}

}  // namespace pkv
