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
// Work decomposition: one workgroup of 4 waves per (sequence, kv head, block
// of ROWS rows), a row being a (query token, GQA head) pair with the group's
// heads consecutive, so every K/V tile serves the whole query group.  Each
// wave owns 16 * NR rows.  Key tiles of KT keys stream from the pool through
// the block table into double-buffered LDS, K and V row-major (V of f32
// pools transposed); the PV operand of 16-bit pools comes from
// ds_read_b64_tr_b16 transposing reads.  Global loads for the next tiles and
// the block ids after them are in flight while a tile is computed.
//
//   S^T = K Q^T on MFMA (K from LDS as the A operand, the rows' Q, held in
//   registers, as B).  The accumulator puts in each lane the scores of 4
//   keys per 16-key tile of ONE row (lane % 16): the per-lane k-slice of the
//   B operand of O^T = V^T P^T, so P never leaves registers.  Online softmax
//   per row in the exp2 domain, fp32 accumulation throughout; for 16-bit
//   pools the row sums come from the P.V MFMA with an all-ones V^T tile (the
//   same rounded P as the numerator, no VALU adds).  P enters the
//   PV product as f16 for f16 pools (relative rounding 2^-12); for bf16 pools
//   as a bf16 high part plus a bf16 residual (two MFMAs, ~16 significant
//   bits); for f32 pools exactly, on v_mfma_f32_16x16x4f32.
//
// Workgroups are mapped XCD-aware: with at least 8 (sequence, kv head) pairs,
// XCD x (= blockIdx % 8) serves the pairs congruent to x mod 8, so the row
// blocks that share a pair's K/V share one L2.  Within an XCD the pairs run
// longest context first, each pair's row blocks last (longest) first, and
// the second round of workgroups per CU runs in reverse order, so the CU
// that holds a heavy workgroup gets a light one beside it; a workgroup's
// time is its chain of key tiles, and the older workgroup of a CU issues
// first.
#include <type_traits>

#include "pkv_prefill_dev.h"

namespace pkv {
namespace {

template <int DT, int HD, int RT, bool FUSED, bool SB>
__global__ void __launch_bounds__(kPT) prefill_kernel(PrefillKArgs a) {
  __shared__ __attribute__((aligned(16))) char lds[2 * PCfg<DT, HD, RT>::STAGE];
  prefill_body<DT, HD, RT, FUSED, SB>(a, blockIdx.x, lds);
}

// Merge of a split row block (sequence s, kv head g, row block rb): per row,
// M = max_p m_p, L = sum_p l_p 2^(m_p - M), O = sum_p O_p 2^(m_p - M) / L
// (exp2 domain of the main kernel), four output elements per thread.  The
// validity checks repeat the main kernel's (which reports the errors).
template <int HD>
__global__ void __launch_bounds__(256)
    prefill_merge_kernel(PrefillKArgs a, int R, int rows_per_block, int out_dt) {
  const int sg = (int)blockIdx.x / a.row_blocks;
  const int rb = (int)blockIdx.x % a.row_blocks;
  if (sg >= a.n_seqs * a.kvh) return;
  const int g = sg % a.kvh, s = sg / a.kvh;
  const int q0 = a.cu_q_lens[s];
  const int q_len = min(a.cu_q_lens[s + 1] - q0, a.max_q_len);
  const int ctx = a.context_lens[s];
  if (ctx > a.max_context_len || ctx > a.mbps * (1 << a.bs_log2) || ctx < q_len || q_len < 0)
    return;
  const int nparts = n_parts_of(ctx - q_len, a.part_keys);
  const int n_rows = q_len * R;
  const int row0 = rb * rows_per_block;
  if (nparts <= 1 || row0 >= n_rows) return;
  const int nr = min(rows_per_block, n_rows - row0);
  const size_t item0 = ((size_t)sg * a.row_blocks + rb) * a.max_parts;
  const size_t pstride = (size_t)rows_per_block;  // rows between parts
  const int H = a.kvh * R;
  constexpr int Q4 = HD / 4;
  for (int task = threadIdx.x; task < nr * Q4; task += 256) {
    const int rr = task / Q4;
    const int d4 = (task - rr * Q4) * 4;
    const size_t pr0 = item0 * pstride + rr;
    float M = -INFINITY;
    for (int j = 0; j < nparts; ++j) M = fmaxf(M, a.part_ml[2 * (pr0 + j * pstride)]);
    float L = 0.0f;
    f32x4 acc = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < nparts; ++j) {
      const size_t pr = pr0 + j * pstride;
      const float w = fast_exp2(a.part_ml[2 * pr] - M);
      L = fmaf(w, a.part_ml[2 * pr + 1], L);
      const f32x4 ov = *reinterpret_cast<const f32x4*>(a.part_o + pr * HD + d4);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(w, ov[i], acc[i]);
    }
    const float inv = 1.0f / L;
    const int r = row0 + rr;
    const size_t eo = ((size_t)(q0 + r / R) * H + g * R + r % R) * HD + d4;
    if (a.out_f32) {
      *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(a.out) + eo) =
          f32x4{acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    } else {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = out_dt == PKV_BF16 ? f32_to_bf16_bits(acc[i] * inv) : f32_to_f16_bits(acc[i] * inv);
      *reinterpret_cast<uint64_t*>(reinterpret_cast<uint16_t*>(a.out) + eo) =
          (uint64_t)(w[0] | (w[1] << 16)) | ((uint64_t)(w[2] | (w[3] << 16)) << 32);
    }
  }
}

template <int DT, int HD, int RT>
hipError_t plaunch(PrefillKArgs k, hipStream_t s) {
  const long long grid = prefill_grid<DT, HD, RT>(k);
  if (grid <= 0) return hipSuccess;
  if (!grid_fits(grid, kPT)) return hipErrorInvalidValue;
  if (k.k_new)
    prefill_kernel<DT, HD, RT, true, false><<<(unsigned)grid, kPT, 0, s>>>(k);
  else
    prefill_kernel<DT, HD, RT, false, false><<<(unsigned)grid, kPT, 0, s>>>(k);
  return hipGetLastError();
}

// Block sizes below a wave-load's key span: the kernels with per-lane block
// ids, built once per dtype and head_dim with the GQA ratio at run time.
template <int DT, int HD>
hipError_t plaunch_sb(PrefillKArgs k, hipStream_t s) {
  const long long grid = prefill_grid<DT, HD, 0>(k);
  if (grid <= 0) return hipSuccess;
  if (!grid_fits(grid, kPT)) return hipErrorInvalidValue;
  if (k.k_new)
    prefill_kernel<DT, HD, 0, true, true><<<(unsigned)grid, kPT, 0, s>>>(k);
  else
    prefill_kernel<DT, HD, 0, false, true><<<(unsigned)grid, kPT, 0, s>>>(k);
  return hipGetLastError();
}

template <int DT, int HD>
hipError_t plaunch_r(int R, const PrefillKArgs& k, hipStream_t s) {
  if ((1 << k.bs_log2) < prefill_wave_keys<DT, HD>()) return plaunch_sb<DT, HD>(k, s);
  switch (R) {
    case 1: return plaunch<DT, HD, 1>(k, s);
    case 2: return plaunch<DT, HD, 2>(k, s);
    case 4: return plaunch<DT, HD, 4>(k, s);
    case 8: return plaunch<DT, HD, 8>(k, s);
    default: return plaunch<DT, HD, 0>(k, s);  // any other ratio, at run time
  }
}

template <int DT>
hipError_t plaunch_hd(int HD, int R, const PrefillKArgs& k, hipStream_t s) {
  switch (HD) {
    case 64: return plaunch_r<DT, 64>(R, k, s);
    case 128: return plaunch_r<DT, 128>(R, k, s);
    case 256: return plaunch_r<DT, 256>(R, k, s);
    default: return hipErrorInvalidValue;
  }
}

template <int HD>
hipError_t pmerge(const PrefillKArgs& k, int R, int rows, int out_dt, hipStream_t s) {
  const long long blocks = (long long)k.n_seqs * k.kvh * k.row_blocks;
  if (blocks <= 0) return hipSuccess;
  if (!grid_fits(blocks, 256)) return hipErrorInvalidValue;
  prefill_merge_kernel<HD><<<(unsigned)blocks, 256, 0, s>>>(k, R, rows, out_dt);
  return hipGetLastError();
}

int ilog2p(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

// Keys per tile and rows per workgroup of the kernel instantiated for a
// pool's dtype and head_dim (host mirror of PCfg).
void prefill_shape(int dt, int hd, int* kt, int* rows) {
  const int rbytes = hd * (dt == PKV_F32 ? 4 : 2);
  *kt = rbytes >= 512 ? 32 : (rbytes >= 256 ? 64 : PKV_PREFILL_KT);
  *rows = kPW * 16 * ((dt != PKV_F32 && hd <= 128) ? PKV_PREFILL_NR : 1);
}

constexpr long long kSplitMaxItems = 4096;  // partial items at most

}  // namespace

void prefill_plan(const pkv_pool* p, int n_seqs, int n_head, int max_q_len, int max_context_len,
                  int* part_keys, int* max_parts, size_t* ws_bytes) {
  int kt = 0, rows = 0;
  prefill_shape(p->dtype, p->head_dim, &kt, &rows);
  const long long R = n_head / p->n_kv_head;
  const long long blocks =
      (long long)n_seqs * p->n_kv_head * (((long long)max_q_len * R + rows - 1) / rows);
  const int mcl = max_context_len > 0 ? max_context_len : 1;
  const int unit = 2 * kt;
  auto round_up = [&](long long x) { return (int)((x + unit - 1) / unit * unit); };
  int pk = round_up(PKV_PREFILL_PART_KEYS);
  int mp = 1 + (mcl - 1) / pk;
  if (blocks >= PKV_PREFILL_SPLIT_MAX_BLOCKS || blocks <= 0) {
    // enough row blocks to fill the GPU: no split
    pk = round_up(mcl);
    mp = 1;
  } else {
    while (mp > 1 && blocks * mp > kSplitMaxItems) {
      pk = round_up(2LL * pk);
      mp = 1 + (mcl - 1) / pk;
    }
  }
  *part_keys = pk;
  *max_parts = mp;
  size_t bytes = 0;
  if (mp > 1) {
    const size_t n = (size_t)blocks * mp * rows;  // partial rows
    bytes = ((n * 2 * 4 + 255) / 256) * 256 + n * (size_t)p->head_dim * 4;
  }
  if (ws_bytes) *ws_bytes = bytes;
}

bool prefill_supported(const pkv_pool* p, int n_head) {
  if (n_head <= 0 || n_head % p->n_kv_head != 0) return false;
  return p->head_dim == 64 || p->head_dim == 128 || p->head_dim == 256;
}

PrefillKArgs prefill_kargs(const pkv_pool* p, int layer, const PrefillArgs& a, char* partials) {
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
  k.k_new = reinterpret_cast<const char*>(a.k_new);
  k.v_new = reinterpret_cast<const char*>(a.v_new);
  k.rq = a.n_head / p->n_kv_head;
  k.cpx = p->n_cu >= kXcd && p->n_cu % kXcd == 0 ? p->n_cu / kXcd : 0;
  prefill_plan(p, a.n_seqs, a.n_head, a.max_q_len, a.max_context_len, &k.part_keys,
               &k.max_parts, nullptr);
  if (k.max_parts > 1) {
    int kt = 0, rows = 0;
    prefill_shape(p->dtype, p->head_dim, &kt, &rows);
    const int R = k.rq;
    const size_t n = (size_t)a.n_seqs * p->n_kv_head *
                     (((size_t)a.max_q_len * R + rows - 1) / rows) * k.max_parts * rows;
    k.part_ml = reinterpret_cast<float*>(partials);
    k.part_o = reinterpret_cast<float*>(partials + ((n * 2 * 4 + 255) / 256) * 256);
  }
  return k;
}

hipError_t launch_prefill_merge(const pkv_pool* p, const PrefillKArgs& k0, hipStream_t stream) {
  if (k0.max_parts <= 1) return hipSuccess;
  PrefillKArgs k = k0;
  int kt = 0, rows = 0;
  prefill_shape(p->dtype, p->head_dim, &kt, &rows);
  const int R = k.rq;
  k.row_blocks = (k.max_q_len * R + rows - 1) / rows;
  switch (p->head_dim) {
    case 64: return pmerge<64>(k, R, rows, p->dtype, stream);
    case 128: return pmerge<128>(k, R, rows, p->dtype, stream);
    default: return pmerge<256>(k, R, rows, p->dtype, stream);
  }
}

hipError_t launch_prefill(const pkv_pool* p, int layer, const PrefillArgs& a,
                          hipStream_t stream, hipEvent_t ev_begin, hipEvent_t ev_end) {
  // the split's partials live in the pool workspace (sized by the caller)
  size_t ws = 0;
  {
    int pk = 0, mp = 0;
    prefill_plan(p, a.n_seqs, a.n_head, a.max_q_len, a.max_context_len, &pk, &mp, &ws);
  }
  if (ws && (!p->ws || p->ws_bytes < ws)) return hipErrorInvalidValue;
  const PrefillKArgs k = prefill_kargs(p, layer, a, p->ws);
  const int R = k.rq;
  hipError_t e = hipSuccess;
  if (ev_begin) e = hipEventRecord(ev_begin, stream);
  if (e != hipSuccess) return e;
  switch (p->dtype) {
    case PKV_F32: e = plaunch_hd<PKV_F32>(p->head_dim, R, k, stream); break;
    case PKV_F16: e = plaunch_hd<PKV_F16>(p->head_dim, R, k, stream); break;
    default: e = plaunch_hd<PKV_BF16>(p->head_dim, R, k, stream); break;
  }
  if (e == hipSuccess && ev_end) e = hipEventRecord(ev_end, stream);
  if (e != hipSuccess) return e;
  return launch_prefill_merge(p, k, stream);
}

}  // namespace pkv
