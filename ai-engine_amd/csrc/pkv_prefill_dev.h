// pkv_prefill_dev.h -- the chunked-prefill attention kernel body (gfx950),
// shared by the prefill launch (pkv_prefill.hip) and the mixed prefill +
// decode launch (pkv_mixed.hip).  Design notes: pkv_prefill.hip.
#pragma once

#include <type_traits>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {


// Waves per workgroup (each owns 16 * NR rows).
#ifndef PKV_PREFILL_WAVES
#define PKV_PREFILL_WAVES 4
#endif
constexpr int kPW = PKV_PREFILL_WAVES;
constexpr int kPT = kPW * 64;  // threads per workgroup

// 16-row MFMA tiles per wave for 16-bit pools of head_dim <= 128.
#ifndef PKV_PREFILL_NR
#define PKV_PREFILL_NR 2
#endif
// Keys per tile for rows of at most 256 bytes.
#ifndef PKV_PREFILL_KT
#define PKV_PREFILL_KT 64
#endif
// Keys per part of a long key range: row blocks whose prior context exceeds
// it are split into parts that run as separate workgroups and are merged
// afterwards (when the launch has few row blocks; see prefill_plan).
#ifndef PKV_PREFILL_PART_KEYS
#define PKV_PREFILL_PART_KEYS 1024
#endif
// Splitting stops at this many row blocks (enough to fill the GPU), and
// parts are lengthened to keep at most kSplitMaxItems partial items.
#ifndef PKV_PREFILL_SPLIT_MAX_BLOCKS
#define PKV_PREFILL_SPLIT_MAX_BLOCKS 256
#endif
// 16-bit pools: softmax row sums taken by the P.V MFMA from an all-ones
// operand instead of VALU adds.
#ifndef PKV_PREFILL_MFMA_ROWSUM
#define PKV_PREFILL_MFMA_ROWSUM 1
#endif
constexpr int kXcd = 8;  // XCDs; workgroups go round-robin over them

template <int DT, int HD, int R>
struct PCfg {
  static constexpr int E = DT == PKV_F32 ? 4 : 2;
  static constexpr int RB = HD * E;                                // row bytes
  static constexpr int NF = RB / 64;                               // 16-B fragments per lane per row
  static constexpr int NR = (DT != PKV_F32 && HD <= 128) ? PKV_PREFILL_NR : 1;  // 16-row tiles per wave
  static constexpr int RW = 16 * NR;                               // rows per wave
  static constexpr int ROWS = kPW * RW;                            // rows per workgroup
  static constexpr int ND = HD / 16;                               // 16-dim tiles of O^T
  static constexpr int KT = RB >= 512 ? 32 : (RB >= 256 ? 64 : PKV_PREFILL_KT);  // keys per tile
  static constexpr int NKM = KT / 16;                              // 16-key MFMA tiles
  static constexpr int CH = RB / 16;                               // 16-B chunks per row
  static constexpr int EPC = 16 / E;                               // elements per chunk
  static constexpr int KPITCH = RB + 16;                           // K row pitch in LDS
  static constexpr int VTP = KT * E + 16;                          // f32: V^T row pitch in LDS
  static constexpr int VP = RB + 32;                               // 16-bit: V row pitch in LDS
  static constexpr int KLDS = KT * KPITCH;
  static constexpr int STAGE = KLDS + (DT == PKV_F32 ? HD * VTP : KT * VP);
  static constexpr int NKL = KT * CH / kPT;                        // K chunks per thread
  // V key-pair chunks per thread (f32 pools; 16-bit pools load V like K and
  // keep NKL chunks in NVP x 2 registers)
  static constexpr int NVP = DT == PKV_F32 ? (KT / 2) * CH / kPT : (NKL + 1) / 2;
  // register sets for tiles in flight: loads run NSET + 1 tiles ahead
  static constexpr int NSET = (NKL + 2 * NVP) <= 4 ? 2 : 1;
  static constexpr int D = NSET + 1;
  static_assert(NKL >= 1 && NVP >= 1, "tile too small for the workgroup");
  static_assert(KT * CH % kPT == 0 && (DT != PKV_F32 || (KT / 2) * CH % kPT == 0), "");
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
  int row_blocks;  // ceil(max_q_len * R / ROWS)
  int part_keys;   // keys per part: a multiple of two tiles
  int max_parts;   // parts per row block at most (1 + (max_context_len - 1) / part_keys)
  int per_xcd;     // workgroup slots per XCD (affinity mapping), 0 = plain order
  int cpx;         // compute units per XCD (pairing of the affinity mapping), 0 = none
  int rq;          // GQA ratio n_head / n_kv_head (kernels built for a fixed ratio ignore it)
  float scale_log2;
  float* part_ml;  // split key ranges: (m, l) per (item, row)
  float* part_o;   //   and the unnormalised O row
  uint32_t* err;
  // Fused store of the prompt's own K/V ([total_q][kvh][hd], pool dtype),
  // or null: keys at or past a sequence's prior context are read from these
  // rows, and each workgroup stores its own tokens' rows into the pool.
  const char* k_new;
  const char* v_new;
};

// Host side (pkv_prefill.hip): kernel arguments of a prefill launch whose
// split partials (if any) go to `partials`, and the merge of a split launch
// (nothing when the launch does not split).
PrefillKArgs prefill_kargs(const pkv_pool* p, int layer, const PrefillArgs& a, char* partials);
hipError_t launch_prefill_merge(const pkv_pool* p, const PrefillKArgs& k, hipStream_t stream);

// Workgroups of the launch; sets the row-block count and the XCD affinity
// mapping of k for the kernel instantiated as PCfg<DT, HD, RT>.
template <int DT, int HD, int RT>
long long prefill_grid(PrefillKArgs& k) {
  using C = PCfg<DT, HD, RT>;
  k.row_blocks = (int)(((long long)k.max_q_len * k.rq + C::ROWS - 1) / C::ROWS);
  const long long n_sg = (long long)k.n_seqs * k.kvh;
  const long long items = n_sg * k.row_blocks * k.max_parts;
  if (items <= 0) return 0;
  long long grid = items;
  k.per_xcd = 0;
  if (n_sg >= kXcd) {
    const long long per = ((n_sg + kXcd - 1) / kXcd) * k.row_blocks * k.max_parts;
    k.per_xcd = (int)per;
    grid = per * kXcd;
  }
  return grid;
}


namespace {


// Parts of a row block whose rows have prior context `prior`: every part but
// the last covers part_keys keys below the prior (visible to all rows, no
// mask, at least one key per row); the last one runs from there to the
// block's last key.
__device__ __forceinline__ int n_parts_of(int prior, int part_keys) {
  return 1 + prior / part_keys;
}

template <int DT>
__device__ __forceinline__ uint32_t to16(float x) {
  return DT == PKV_BF16 ? f32_to_bf16_bits(x) : f32_to_f16_bits(x);
}

constexpr float kTau = 8.0f;  // lazy-rescale threshold (log2 units): weights <= 256

// Max over the four lane groups (rows of 16 lanes) holding one score row:
// permlane16_swap pairs rows 0/1 and 2/3, permlane32_swap the two halves.
__device__ __forceinline__ float row_group_max(float x) {
  auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  x = fmaxf(__uint_as_float(a[0]), __uint_as_float(a[1]));
  auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

// Two floats to packed 16-bit (round to nearest even, v_cvt_pk_*_f32).
template <int DT>
__device__ __forceinline__ uint32_t cvt_pk16(float x0, float x1) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  const f2 v = {x0, x1};
  if constexpr (DT == PKV_BF16) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
  } else {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
  }
}

// Keys one wave's share of a tile load spans (K chunks; f32 pools load V in
// key pairs, twice as many).  Block sizes at least this large give every
// wave-load one block id.
template <int DT, int HD>
constexpr int prefill_wave_keys() {
  return (DT == PKV_F32 ? 2 : 1) * kWave / PCfg<DT, HD, 1>::CH;
}

// RT: the GQA ratio the kernel is built for, or 0 for any ratio (a.rq); the
// ratio only enters the row <-> (token, head) index arithmetic.
// SB (block_size below prefill_wave_keys): a wave-load's keys span several
// blocks, so each lane reads its own key's block id from the table where it
// loads the key (a vector load in the tile's load phase) instead of taking
// the wave-uniform id prefetched by scalar loads.
template <int DT, int HD, int RT, bool FUSED, bool SB = false>
__device__ __forceinline__ void prefill_body(const PrefillKArgs& a, int bid,
                                             char (&lds)[2 * PCfg<DT, HD, RT>::STAGE]) {
  using C = PCfg<DT, HD, RT>;
  const int R = RT > 0 ? RT : a.rq;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int G = lane >> 4;
  const int col = lane & 15;

  // ---- work item: (sequence, kv head) pair sg, row block rb, key part ----
  // Row blocks run last (longest) first, each with its parts in order.
  const int n_sg = a.n_seqs * a.kvh;
  const int rbp = a.row_blocks * a.max_parts;
  int sg, rb, part;
  int q0 = 0, q1 = 0, ctx = 0;  // cu_q_lens[s], cu_q_lens[s + 1], context_lens[s]
  bool have_lens = false;
  {
    int u;
    if (a.per_xcd > 0) {
      const int x = bid % kXcd;
      int slot = bid / kXcd;
      const int nx = (n_sg - x + kXcd - 1) / kXcd;  // pairs of this XCD
      if (slot >= nx * rbp) return;
      if (nx <= 64) {
        // Heaviest first, paired per CU.  The XCD's pairs are ranked by
        // context length (the key count of their last row; ties by index)
        // and their items taken pair-major, last row block first.  The
        // XCD's workgroups fill its CUs in rounds of cpx (one per CU per
        // round); every other full round runs in reverse, so a CU holding
        // the k-th heaviest item of one round holds the k-th lightest of
        // the next.  A CU's older workgroup issues first, and here it is
        // the heavier one.
        if (a.cpx > 0) {
          const int round = slot / a.cpx;
          if ((round & 1) && (round + 1) * a.cpx <= nx * rbp)
            slot = round * a.cpx + (a.cpx - 1 - slot % a.cpx);
        }
        // lane j: the j-th pair of the XCD, with its sequence's lengths
        const int ln = threadIdx.x & 63;
        const int sj = ln < nx ? (x + kXcd * ln) / a.kvh : 0;
        const int w = ln < nx ? a.context_lens[sj] : -1;
        const int c0 = a.cu_q_lens[sj], c1 = a.cu_q_lens[sj + 1];
        int rank = 0;
        for (int j = 0; j < nx; ++j) {
          const int wj = __builtin_amdgcn_readlane(w, j);
          rank += (wj > w) | ((wj == w) & (j < ln));
        }
        const int want = slot / rbp;
        const int jw = (int)__builtin_ctzll(__builtin_amdgcn_ballot_w64(ln < nx && rank == want));
        sg = x + kXcd * jw;
        ctx = __builtin_amdgcn_readlane(w, jw);
        q0 = __builtin_amdgcn_readlane(c0, jw);
        q1 = __builtin_amdgcn_readlane(c1, jw);
        have_lens = true;
        u = slot % rbp;
      } else {
        u = slot / nx;
        sg = x + kXcd * (slot % nx);
      }
    } else {
      if (bid >= n_sg * rbp) return;
      u = bid / n_sg;
      sg = bid % n_sg;
    }
    rb = a.row_blocks - 1 - u / a.max_parts;
    part = u % a.max_parts;
  }
  const int g = sg % a.kvh;
  const int s = sg / a.kvh;

  if (!have_lens) {
    q0 = a.cu_q_lens[s];
    q1 = a.cu_q_lens[s + 1];
    ctx = a.context_lens[s];
  }
  const int q_len_raw = q1 - q0;
  const int q_len = min(q_len_raw, a.max_q_len);
  const bool reporter = tid == 0 && rb == 0 && g == 0;
  if (q_len_raw > a.max_q_len && reporter) atomicOr(a.err, PKV_EBIT_LENGTH);
  const int BS = 1 << a.bs_log2;
  if (ctx > a.max_context_len || ctx > a.mbps * BS || ctx < q_len || q_len < 0) {
    if (reporter) atomicOr(a.err, PKV_EBIT_LENGTH);
    return;
  }
  const int n_rows = q_len * R;
  const int row0 = rb * C::ROWS;
  if (row0 >= n_rows) return;  // uniform over the workgroup
  const int prior = ctx - q_len;
  const int H = a.kvh * R;
  const int tmask = BS - 1;
  const size_t slot_stride = (size_t)a.kvh * C::RB;
  const size_t blk_stride = (size_t)BS * slot_stride;
  const char* kh = a.k_pool + (size_t)g * C::RB;
  const char* vh = a.v_pool + (size_t)g * C::RB;
  const int32_t* table = a.block_tables + (size_t)s * a.mbps;

  // keys the workgroup needs: 0 .. prior + its last token, in parts
  const int n_keys = prior + min(row0 + C::ROWS - 1, n_rows - 1) / R + 1;
  const int nparts = n_parts_of(prior, a.part_keys);
  if (part >= nparts) return;  // uniform over the workgroup

  // Fused store of the K/V rows of the chunk's tokens at positions prior + i.
  // Row blocks partition the tokens: token j belongs to the row block of its
  // first row, j R / ROWS, so row block r owns tokens tok_lo(r) ..
  // tok_lo(r + 1) - 1 with tok_lo(r) = ceil(r ROWS / R).  The store's load
  // round trip must not lengthen the heaviest row blocks (the last ones,
  // which see the most keys): row block rb of the sequence's nrb stores its
  // own tokens and those of its mirror nrb - 1 - rb when rb is the lighter of
  // the two, nothing when it is the heavier; only the last part of a row
  // block stores.  No workgroup of this launch reads these rows from the
  // pool: keys >= prior come from k_new / v_new.
  const char* kin = FUSED ? a.k_new + (size_t)g * C::RB : nullptr;
  const char* vin = FUSED ? a.v_new + (size_t)g * C::RB : nullptr;
  const int nrb = (n_rows + C::ROWS - 1) / C::ROWS;
  const int mirror = nrb - 1 - rb;
  if (FUSED && part == nparts - 1 && rb <= mirror) {
    auto tok_lo = [&](int r) { return min((r * C::ROWS + R - 1) / R, q_len); };
    const int own0 = tok_lo(rb), own = tok_lo(rb + 1) - own0;
    const int mir0 = tok_lo(mirror), mir = rb < mirror ? tok_lo(mirror + 1) - mir0 : 0;
    const int nch = (own + mir) * C::CH;
    for (int idx = tid; idx < nch; idx += kPT) {
      const int j = idx / C::CH, c16 = 16 * (idx % C::CH);
      const int tok = j < own ? own0 + j : mir0 + (j - own);
      const int pos = prior + tok;
      const int blk = table[pos >> a.bs_log2];
      if ((unsigned)blk >= (unsigned)a.num_blocks) {
        atomicOr(a.err, PKV_EBIT_BLOCK);
        continue;
      }
      const size_t off = (size_t)blk * blk_stride + (size_t)(pos & tmask) * slot_stride + c16;
      const size_t src = (size_t)(q0 + tok) * a.kvh * C::RB + c16;
      const u32x4 kx = ld16(kin + src), vx = ld16(vin + src);
      st16(const_cast<char*>(kh) + off, kx);
      st16(const_cast<char*>(vh) + off, vx);
    }
  }
  const int k_hi = part + 1 < nparts ? (part + 1) * a.part_keys : n_keys;
  const int t_lo = part * (a.part_keys / C::KT);
  const int n_tiles = (k_hi + C::KT - 1) / C::KT;  // tiles t_lo .. n_tiles - 1

  // ---- this wave's rows (B operand / output): row 16 rn + col ----
  const int roww = row0 + wave * C::RW;
  const bool has_rows = roww < n_rows;
  const int klim_lo = prior + min(roww, n_rows - 1) / R;              // smallest row limit
  const int klim_hi = prior + min(roww + C::RW - 1, n_rows - 1) / R;  // largest row limit
  int lim[C::NR];
  u32x4 qf[C::NR][C::NF];
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    const int rc = min(roww + 16 * rn + col, n_rows - 1);
    lim[rn] = prior + rc / R;
    const char* qrow = a.q + ((size_t)(q0 + rc / R) * H + g * R + rc % R) * C::RB;
#pragma unroll
    for (int f = 0; f < C::NF; ++f) qf[rn][f] = ld16(qrow + 64 * f + 16 * G);
  }

  // ---- cooperative tile loads.  K chunk i of a thread: key
  //      (tid + kPT i) / CH, bytes 16 (tid % CH); V pair chunk v: keys
  //      2 ((tid + kPT v) / CH) and +1 (kPT = threads per workgroup).  CH divides 64, so one wave's share
  //      of a load covers at most 16 aligned keys -- one block when
  //      block_size >= prefill_wave_keys: its block id is wave-uniform (a
  //      scalar load) and a lane adds a 32-bit offset (smaller blocks: SB,
  //      an id per lane).  Keys past n_keys are clamped to n_keys - 1.
  //      Block ids are checked where they are used; a bad one reads block 0
  //      and is reported once at the end. ----
  const int wkey = (wave * kWave) / C::CH;  // wave's first key within a load
  const int lkey = lane / C::CH;            // lane's key within the wave's share
  const uint32_t lbyte = 16 * (lane % C::CH);
  bool bad_block = false;
  auto table_at = [&](int key) __attribute__((always_inline)) {
    const int k = min(key, n_keys - 1) >> a.bs_log2;
    typedef const __attribute__((address_space(4))) int32_t cint;  // read-only: scalar load
    return *(cint*)(table + k);
  };
  auto checked = [&](int blk) __attribute__((always_inline)) {
    const bool bad = (unsigned)blk >= (unsigned)a.num_blocks;
    bad_block |= bad;
    return bad ? 0 : blk;
  };
  int kb[2][C::NKL], vb[2][C::NVP];  // raw block ids, two sets by tile parity
  auto ids = [&](int t, int (&kbs)[C::NKL], int (&vbs)[C::NVP]) __attribute__((always_inline)) {
    if constexpr (SB) return;  // per-lane ids are read in the load phase
#pragma unroll
    for (int i = 0; i < C::NKL; ++i) kbs[i] = table_at(t * C::KT + wkey + kPT * i / C::CH);
    if constexpr (DT == PKV_F32) {  // 16-bit pools load V with K's keys and block ids
#pragma unroll
      for (int v = 0; v < C::NVP; ++v) vbs[v] = table_at(t * C::KT + 2 * (wkey + kPT * v / C::CH));
    }
  };
  // SB: the block of this lane's key (clamped like the keys themselves)
  auto lane_block = [&](int key) __attribute__((always_inline)) {
    return table[min(key, n_keys - 1) >> a.bs_log2];
  };
  u32x4 kreg[C::NSET][C::NKL], vreg[C::NSET][C::NVP][2];
  // A tile's K/V rows: from the pool, or (fused store) from the prompt's
  // rows for keys >= prior.  MODE 0: every key from the pool; 1: every key
  // from the prompt (keys past n_keys are clamped to n_keys - 1 >= prior);
  // 2: the one tile that straddles the prior, chosen per key.
  auto loads_m = [&](int t, u32x4 (&kr)[C::NKL], u32x4 (&vr)[C::NVP][2],
                     const int (&kbs)[C::NKL], const int (&vbs)[C::NVP], auto mode_c)
                     __attribute__((always_inline)) {
    constexpr int MODE = decltype(mode_c)::value;
    auto src = [&](const char* pool_row_base, const char* in, int key) __attribute__((always_inline)) {
      if constexpr (MODE == 1) return in + (size_t)(q0 + key - prior) * a.kvh * C::RB + lbyte;
      const char* pr = pool_row_base + ((uint32_t)((key & tmask) * slot_stride) + lbyte);
      if constexpr (MODE == 0) return pr;
      return key < prior ? pr : in + (size_t)(q0 + key - prior) * a.kvh * C::RB + lbyte;
    };
#pragma unroll
    for (int i = 0; i < C::NKL; ++i) {
      const int key = min(t * C::KT + wkey + kPT * i / C::CH + lkey, n_keys - 1);
      const int blk = SB ? lane_block(key) : kbs[i];
      kr[i] = ld16(src(kh + (size_t)checked(blk) * blk_stride, kin, key));
    }
    if constexpr (DT == PKV_F32) {
#pragma unroll
      for (int v = 0; v < C::NVP; ++v) {
        const int k0 = t * C::KT + 2 * (wkey + kPT * v / C::CH + lkey);
        const int b0 = SB ? lane_block(k0) : vbs[v];
        const int b1 = SB ? lane_block(k0 + 1) : vbs[v];
        vr[v][0] = ld16(src(vh + (size_t)checked(b0) * blk_stride, vin, min(k0, n_keys - 1)));
        vr[v][1] = ld16(src(vh + (size_t)checked(b1) * blk_stride, vin, min(k0 + 1, n_keys - 1)));
      }
    } else {  // V chunk 2 v + h: the same key and bytes as K chunk 2 v + h
#pragma unroll
      for (int i = 0; i < C::NKL; ++i) {
        const int key = min(t * C::KT + wkey + kPT * i / C::CH + lkey, n_keys - 1);
        const int blk = SB ? lane_block(key) : kbs[i];
        vr[i >> 1][i & 1] = ld16(src(vh + (size_t)checked(blk) * blk_stride, vin, key));
      }
    }
  };
  auto loads = [&](int t, u32x4 (&kr)[C::NKL], u32x4 (&vr)[C::NVP][2],
                   const int (&kbs)[C::NKL], const int (&vbs)[C::NVP]) __attribute__((always_inline)) {
    if constexpr (!FUSED) {
      loads_m(t, kr, vr, kbs, vbs, std::integral_constant<int, 0>{});
    } else {
      const int tk0 = t * C::KT;  // wave-uniform choice of path
      if (tk0 + C::KT <= prior)
        loads_m(t, kr, vr, kbs, vbs, std::integral_constant<int, 0>{});
      else if (tk0 >= prior)
        loads_m(t, kr, vr, kbs, vbs, std::integral_constant<int, 1>{});
      else
        loads_m(t, kr, vr, kbs, vbs, std::integral_constant<int, 2>{});
    }
  };
  auto store = [&](int stage, const u32x4 (&kr)[C::NKL], const u32x4 (&vr)[C::NVP][2]) __attribute__((always_inline)) {
    char* kl = lds + stage * C::STAGE;
    char* vl = kl + C::KLDS;
#pragma unroll
    for (int i = 0; i < C::NKL; ++i) {
      const int idx = tid + kPT * i;
      st16(kl + (idx / C::CH) * C::KPITCH + 16 * (idx % C::CH), kr[i]);
    }
    if constexpr (DT == PKV_F32) {  // V^T: dim-major rows, keys in natural order
#pragma unroll
      for (int v = 0; v < C::NVP; ++v) {
        const int idx = tid + kPT * v;
        char* dst = vl + C::EPC * (idx % C::CH) * C::VTP + 2 * (idx / C::CH) * 4;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          *reinterpret_cast<uint64_t*>(dst + e * C::VTP) =
              (uint64_t)vr[v][0][e] | ((uint64_t)vr[v][1][e] << 32);
      }
    } else {  // V row-major like K; read transposed by ds_read_b64_tr_b16
#pragma unroll
      for (int i = 0; i < C::NKL; ++i) {
        const int idx = tid + kPT * i;
        st16(vl + (idx / C::CH) * C::VP + 16 * (idx % C::CH), vr[i >> 1][i & 1]);
      }
    }
  };

  // Row sums: lane-partial VALU sums, or (16-bit pools) the P.V MFMA against
  // an all-ones V^T tile, which leaves the full sum of row 16 rn + col in
  // every register of lacc[rn].
  constexpr bool kRowSum = PKV_PREFILL_MFMA_ROWSUM && DT != PKV_F32;
  const uint32_t one2 = DT == PKV_BF16 ? 0x3F803F80u : 0x3C003C00u;
  const u32x4 ones = u32x4{one2, one2, one2, one2};
  f32x4 lacc[C::NR];
  float m[C::NR], lsum[C::NR];
  f32x4 o[C::ND][C::NR];
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    m[rn] = -INFINITY;
    lsum[rn] = 0.0f;
    lacc[rn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int dm = 0; dm < C::ND; ++dm) o[dm][rn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  }

  // A operand of O^T += V^T P^T for 16-bit pools, from row-major V in LDS:
  // lane (dim 16 dm + col, group G) needs keys 32 ks + 4 G + {0..3} and
  // 32 ks + 16 + 4 G + {0..3}.  ds_read_b64_tr_b16 gives lane i of a 16-lane
  // group, element j, the (i & 3)-th 16-bit value at the address of lane
  // 4 j + (i >> 2); so lane s of the group points at key 4 G + (s >> 2),
  // dims 4 (s & 3) .. +3 of the 16-dim tile.
  auto v_frag = [&](const char* vl, int ks, int dm) __attribute__((always_inline)) {
    typedef short s4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) s4 lds_s4;
    const int src = lane & 15;
    const char* b = vl + (32 * ks + 4 * G + (src >> 2)) * C::VP + (16 * dm + 4 * (src & 3)) * 2;
    const s4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(b));
    const s4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4*)(b + 16 * C::VP));
    const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
    return u32x4{l2.x, l2.y, h2.x, h2.y};
  };
  // ---- S^T = K Q^T: sacc[km][rn][j] = S[key k0 + 16 km + 4 G + j][row] ----
  typedef f32x4 STile[C::NKM][C::NR];
  auto qk = [&](const char* kl, STile& sacc) __attribute__((always_inline)) {
#pragma unroll
    for (int km = 0; km < C::NKM; ++km) {
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn) sacc[km][rn] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int f = 0; f < C::NF; ++f) {
        const u32x4 kf = ld16(kl + (16 * km + col) * C::KPITCH + 64 * f + 16 * G);
#pragma unroll
        for (int rn = 0; rn < C::NR; ++rn) mfma_frag<DT>(kf, qf[rn][f], sacc[km][rn]);
      }
    }
  };
  // Causal mask: scores of keys past a row's position become -inf in place,
  // so the shared softmax below gives them weight exactly 0 and a row's
  // arithmetic does not depend on which rows share its wave or workgroup.
  auto mask = [&](int k0, STile& sacc) __attribute__((always_inline)) {
#pragma unroll
    for (int km = 0; km < C::NKM; ++km)
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (k0 + 16 * km + 4 * G + j > lim[rn]) sacc[km][rn][j] = -INFINITY;
  };
  // Online softmax per row (rows along lane % 16) with a lazily raised
  // reference max m (log2 domain): m moves only when a tile's row max exceeds
  // it by more than kTau, so weights stay <= 2^kTau and the O/l rescale is
  // skipped whenever no row of the wave moved.  Scores enter the exponent
  // through one fma; the weights replace the scores in sacc.  Returns
  // whether this lane's rows moved (alpha: their rescale factors).
  auto softmax = [&](STile& sacc, float (&alpha)[C::NR]) __attribute__((always_inline)) {
    bool moved = false;
    // A row's max over the tile exceeds m + kTau iff one of its lane
    // groups' partial maxima does (scale > 0, checked by the host, and
    // rounding is monotone), so the cross-lane reduction runs only when some
    // row of the wave can move -- after the first tiles, rarely.
    float lmax[C::NR];
    bool over = false;
#pragma unroll
    for (int rn = 0; rn < C::NR; ++rn) {
      lmax[rn] = -INFINITY;
#pragma unroll
      for (int km = 0; km < C::NKM; ++km)
#pragma unroll
        for (int j = 0; j < 4; ++j) lmax[rn] = fmaxf(lmax[rn], sacc[km][rn][j]);
      over |= lmax[rn] * a.scale_log2 > m[rn] + kTau;
      alpha[rn] = 1.0f;
    }
    if (__builtin_amdgcn_ballot_w64(over)) {  // wave-uniform
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn) {
        const float tmax = row_group_max(lmax[rn]) * a.scale_log2;
        if (tmax > m[rn] + kTau) {  // always in tile 0: m starts at -inf, key 0 is visible
          alpha[rn] = fast_exp2(m[rn] - tmax);
          m[rn] = tmax;
          moved = true;
        }
      }
    }
#pragma unroll
    for (int rn = 0; rn < C::NR; ++rn) {
      const float nm = -m[rn];
      float ssum = 0.0f;
#pragma unroll
      for (int km = 0; km < C::NKM; ++km)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          sacc[km][rn][j] = fast_exp2(fmaf(sacc[km][rn][j], a.scale_log2, nm));
          if constexpr (!kRowSum) ssum += sacc[km][rn][j];
        }
      if constexpr (!kRowSum) lsum[rn] = fmaf(lsum[rn], alpha[rn], ssum);  // lane-partial
    }
    return moved;
  };
  auto rescale = [&](bool moved, const float (&alpha)[C::NR]) __attribute__((always_inline)) {
    if (__builtin_amdgcn_ballot_w64(moved)) {  // wave-uniform
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn) {
#pragma unroll
        for (int dm = 0; dm < C::ND; ++dm) o[dm][rn] *= alpha[rn];
        if constexpr (kRowSum) lacc[rn] *= alpha[rn];
      }
    }
  };
  // 16-bit pools: the weights as the B operand of the P.V MFMA, k-step ks
  // (32 keys): lane group G supplies keys 32 ks + {4G..4G+3, 16+4G..16+4G+3};
  // bf16 as a high part plus the bf16 residual (two MFMAs).
  constexpr int NKS = C::KT / 32;
  typedef u32x4 PTile[NKS][C::NR];
  auto pack = [&](const STile& p, PTile& phi, PTile& plo) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int rn = 0; rn < C::NR; ++rn)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const float x0 = p[2 * ks + (w >> 1)][rn][(w & 1) * 2];
          const float x1 = p[2 * ks + (w >> 1)][rn][(w & 1) * 2 + 1];
          phi[ks][rn][w] = cvt_pk16<DT>(x0, x1);
          if constexpr (DT == PKV_BF16)
            plo[ks][rn][w] = cvt_pk16<DT>(x0 - bf16lo(phi[ks][rn][w]), x1 - bf16hi(phi[ks][rn][w]));
        }
  };
  // ---- O^T += V^T P^T ----
  auto pv16 = [&](const char* vl, const PTile& phi, const PTile& plo) __attribute__((always_inline)) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
      for (int dm = 0; dm < C::ND; ++dm) {
        const u32x4 va = v_frag(vl, ks, dm);
#pragma unroll
        for (int rn = 0; rn < C::NR; ++rn) {
          mfma_frag<DT>(va, phi[ks][rn], o[dm][rn]);
          if constexpr (DT == PKV_BF16) mfma_frag<DT>(va, plo[ks][rn], o[dm][rn]);
        }
      }
      if constexpr (kRowSum) {
        // every row of the all-ones operand sums the row's weights
#pragma unroll
        for (int rn = 0; rn < C::NR; ++rn) {
          mfma_frag<DT>(ones, phi[ks][rn], lacc[rn]);
          if constexpr (DT == PKV_BF16) mfma_frag<DT>(ones, plo[ks][rn], lacc[rn]);
        }
      }
    }
  };
  auto pv32 = [&](const char* vl, const STile& p) __attribute__((always_inline)) {
    // k-step (km, j): lane group G supplies key 16 km + 4 G + j
#pragma unroll
    for (int dm = 0; dm < C::ND; ++dm)
#pragma unroll
      for (int km = 0; km < C::NKM; ++km) {
        const u32x4 va = ld16(vl + (16 * dm + col) * C::VTP + (16 * km + 4 * G) * 4);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int rn = 0; rn < C::NR; ++rn)
            o[dm][rn] = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(va[j]),
                                                             p[km][rn][j], o[dm][rn], 0, 0, 0);
      }
  };
  auto compute = [&](int t, bool masked) __attribute__((always_inline)) {
    const char* kl = lds + (t & 1) * C::STAGE;
    const char* vl = kl + C::KLDS;
    STile sacc;
    qk(kl, sacc);
    if (masked) mask(t * C::KT, sacc);  // wave-uniform branch
    float alpha[C::NR];
    const bool moved = softmax(sacc, alpha);
    rescale(moved, alpha);
    if constexpr (DT == PKV_F32) {
      pv32(vl, sacc);
    } else {
      PTile phi, plo;
      pack(sacc, phi, plo);
      pv16(vl, phi, plo);
    }
  };

  // ---- pipeline: tile t is computed from LDS stage t & 1 while the data
  //      of tiles t + 1 .. t + D sit in registers or in flight and the block
  //      ids of tile t + D + 1 resolve.  Loads return in issue order, so
  //      each tile's block ids are issued before the previous tile's data:
  //      waiting for them never waits for data still needed in flight. ----
  // Loads and block ids past the last tile are clamped to key n_keys - 1
  // (valid, unused) and stores past it fill an LDS stage nobody reads, so the
  // memory operations run unconditionally: the in-order wait counts stay
  // exact across the loop.  Iterations run in pairs (register sets and LDS
  // stages alternate); a tile past the end computes nothing.
  // Tile indices are absolute (keys t * KT ..); a part starts at an even
  // tile (part_keys is a multiple of two tiles), so parities, LDS stages and
  // register sets follow t as in a whole range.
  constexpr int NS = C::NSET, D = C::D;
  ids(t_lo, kb[0], vb[0]);
  loads(t_lo, kreg[0], vreg[0], kb[0], vb[0]);
  if constexpr (D > 2) {
    ids(t_lo + 1, kb[1], vb[1]);
    loads(t_lo + 1, kreg[1 % NS], vreg[1 % NS], kb[1], vb[1]);
  }
  store(0, kreg[0], vreg[0]);
  ids(t_lo + D - 1, kb[(D - 1) & 1], vb[(D - 1) & 1]);
  ids(t_lo + D, kb[D & 1], vb[D & 1]);
  loads(t_lo + D - 1, kreg[(D - 1) % NS], vreg[(D - 1) % NS], kb[(D - 1) & 1], vb[(D - 1) & 1]);
  __syncthreads();

  auto iter = [&](int t, auto parity) __attribute__((always_inline)) {
    constexpr int P = decltype(parity)::value;  // t & 1
    const int k0 = t * C::KT;
    // wave-uniform: the tile is in this part and some row sees one of its keys
    if (has_rows && k0 < k_hi && k0 <= klim_hi)
      compute(t, k0 + C::KT - 1 > klim_lo);
    store((P + 1) & 1, kreg[(P + 1) % NS], vreg[(P + 1) % NS]);
    ids(t + D + 1, kb[(P + D + 1) & 1], vb[(P + D + 1) & 1]);
    loads(t + D, kreg[(P + D) % NS], vreg[(P + D) % NS], kb[(P + D) & 1], vb[(P + D) & 1]);
    __syncthreads();
  };
  for (int t = t_lo; t < n_tiles; t += 2) {
    iter(t, std::integral_constant<int, 0>{});
    iter(t + 1, std::integral_constant<int, 1>{});
  }
  if (bad_block && lane == 0) atomicOr(a.err, PKV_EBIT_BLOCK);
  if (!has_rows) return;

  if (nparts > 1) {
    // ---- partial result of this part: (m, l) and the unnormalised O row
    //      (lane holds O^T[dims 16 dm + 4 G + j][row 16 rn + col]) ----
    const size_t item = ((size_t)sg * a.row_blocks + rb) * a.max_parts + part;
#pragma unroll
    for (int rn = 0; rn < C::NR; ++rn) {
      float l;
      if constexpr (kRowSum) {
        l = lacc[rn][0];
      } else {
        l = lsum[rn];
        l += shfl_xor_f(l, 16);
        l += shfl_xor_f(l, 32);
      }
      const int r = roww + 16 * rn + col;
      if (r >= n_rows) continue;
      const size_t pr = item * C::ROWS + (r - row0);
      float* po = a.part_o + pr * HD;
#pragma unroll
      for (int dm = 0; dm < C::ND; ++dm)
        *reinterpret_cast<f32x4*>(po + 16 * dm + 4 * G) = o[dm][rn];
      if (G == 0) {
        a.part_ml[2 * pr] = m[rn];
        a.part_ml[2 * pr + 1] = l;
      }
    }
    return;
  }

  // ---- epilogue: lane holds O^T[dims 16 dm + 4 G + j][row 16 rn + col] ----
#pragma unroll
  for (int rn = 0; rn < C::NR; ++rn) {
    float l;
    if constexpr (kRowSum) {
      l = lacc[rn][0];
    } else {
      l = lsum[rn];
      l += shfl_xor_f(l, 16);
      l += shfl_xor_f(l, 32);
    }
    const int r = roww + 16 * rn + col;
    if (r >= n_rows) continue;
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

}  // namespace
}  // namespace pkv
