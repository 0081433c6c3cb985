// pkv_sample.hip -- token selection on the device: argmax and sample() of
// crates/ai-engine-runtime/src/sample.rs:12-55, which the paged engine runs
// on every logits row it copies to the host (engine.rs:145-162, 226) with
// SamplingConfig {temperature of the request, top_p: None, top_k: None,
// seed: 42} (engine.rs:58-60).  Selecting on the device leaves one int32
// per row to copy back instead of the whole row.
//
// Greedy rows (temperature 0, or at most one logit) take the first maximum;
// a NaN is never chosen and a row with no value above -inf gives 0
// (argmax's fold from (0, -inf), sample.rs:50-55).
//
// Other rows: the reference sorts y = logit / temperature (stable,
// descending), keeps the first top_k, takes p = softmax, keeps the shortest
// prefix whose cumulative p reaches top_p, renormalises, and returns the
// first token at which the cumulative p reaches r, the first f32 of
// StdRng::seed_from_u64(seed) -- one fixed value for a fixed seed.  All of
// that only needs the sorted position where a running mass crosses a
// threshold, which a radix selection finds without sorting: y maps to an
// order-preserving 32-bit key, and three passes over the row (key bits
// 31..20, 19..10, 9..0) histogram the mass of the tokens that share the
// digits chosen so far, walking the buckets from the largest y down until
// the threshold is reached.  Masses are exp(y - max y) in 2^-40 fixed point,
// so the LDS histograms add integers: the sums are exact and the result does
// not depend on the order of the atomics.  Tokens with equal y are ordered
// by index, as the stable sort leaves them.  The selected token equals the
// reference's except where the reference's own f32 running sums land within
// their rounding (~1e-6) of r or top_p.
//
// One workgroup of 1024 threads per row.  The row is read once per pass --
// max; the first digit, whose histogram also gives the total mass and is
// shared by the top_p and r selections; two more digits per selection (the
// last one records each bucket's size and smallest index, which settles a
// tie without another pass unless several tied tokens are needed; three more
// passes for top_k) -- and stays in L2 / the Infinity Cache between passes.
// Batches of at most 128 rows without top_k / top_p split each row over
// several workgroups instead (one launch per pass, partial histograms in a
// stream-ordered allocation), which gives the same tokens.
#include <algorithm>
#include <climits>
#include <cmath>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {

float sample_draw(uint64_t seed) {
  // rand_core 0.6.4 SeedableRng::seed_from_u64: a PCG32 stream fills the
  // 32-byte ChaCha key, eight little-endian words.
  uint32_t s[16] = {0x61707865u, 0x3320646eu, 0x79622d32u, 0x6b206574u};
  uint64_t st = seed;
  for (int i = 0; i < 8; ++i) {
    st = st * 6364136223846793005ull + 11634580027462260723ull;
    const uint32_t xs = (uint32_t)(((st >> 18) ^ st) >> 27);
    const uint32_t rot = (uint32_t)(st >> 59);
    s[4 + i] = (xs >> rot) | (xs << ((32u - rot) & 31u));
  }
  // words 12..15: block counter 0 and stream 0 (rand_chacha 0.3.1)
  uint32_t x[16];
  for (int i = 0; i < 16; ++i) x[i] = s[i];
  auto rotl = [](uint32_t v, int n) { return (v << n) | (v >> (32 - n)); };
  auto qr = [&](int a, int b, int c, int d) {
    x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 16);
    x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 12);
    x[a] += x[b]; x[d] = rotl(x[d] ^ x[a], 8);
    x[c] += x[d]; x[b] = rotl(x[b] ^ x[c], 7);
  };
  for (int r = 0; r < 12; r += 2) {  // StdRng = ChaCha12
    qr(0, 4, 8, 12); qr(1, 5, 9, 13); qr(2, 6, 10, 14); qr(3, 7, 11, 15);
    qr(0, 5, 10, 15); qr(1, 6, 11, 12); qr(2, 7, 8, 13); qr(3, 4, 9, 14);
  }
  const uint32_t w0 = x[0] + s[0];
  // rand 0.8 Standard for f32: the top 24 bits times 2^-24, in [0, 1)
  return (float)(w0 >> 8) * (1.0f / 16777216.0f);
}

namespace {

constexpr int kST = 1024;                 // threads per row
constexpr int kSW = kST / 64;             // waves per row
constexpr int kB1 = 4096;                 // first digit: key bits 31..20
constexpr int kB2 = 1024;                 // second / third: bits 19..10, 9..0
constexpr float kFix = 1099511627776.0f;  // 2^40
constexpr unsigned long long kOne = 1ull << 40;
constexpr int kSplitMinChunk = 4096;      // split path: elements per workgroup at least

struct SampleArgs {
  const char* logits;
  long long stride_bytes;
  int vocab;
  const float* temps;
  int top_k;
  float top_p;
  float r;
  int32_t* tokens;
};

struct SampleSmem {
  unsigned long long h1[kB1];  // first-digit histogram, kept between selections
  unsigned long long h[kB2];   // histogram of the later digits
  unsigned int cnt[kB2];       // last digit: tokens per bucket
  int minidx[kB2];             // last digit: smallest index per bucket
  unsigned long long red_u[kSW];
  float red_f[kSW];
  int red_i[kSW];
  int red_j[kSW];
  unsigned int sel_bucket;
  unsigned long long sel_rem;
  int found;
};

template <int DT>
__device__ __forceinline__ float logit(const char* row, int i) {
  if constexpr (DT == PKV_F32) {
    return reinterpret_cast<const float*>(row)[i];
  } else if constexpr (DT == PKV_BF16) {
    return __uint_as_float((uint32_t)reinterpret_cast<const uint16_t*>(row)[i] << 16);
  } else {
    return (float)reinterpret_cast<const _Float16*>(row)[i];
  }
}

// Vectors a thread of the exact path's row scans loads before it processes
// them: one memory round trip per kRowBatch vectors instead of one per
// vector (a 128k row is 16 vectors per thread).
constexpr int kRowBatch = 8;

// Calls f(i, logit) for this thread's elements of row[lo, hi), in
// increasing i: 16-byte vectors (VEC: the row is 16-byte aligned and lo is
// a multiple of a vector's elements), loaded U at a time, then the tail
// past the last vector.
template <int DT, bool VEC, int U = 1, class F>
__device__ __forceinline__ void for_range(const char* row, int lo, int hi, F&& f) {
  int done = lo;
  if constexpr (VEC) {
    constexpr int E = DT == PKV_F32 ? 4 : 8;
    const int vend = hi / E;
    for (int v0 = lo / E + (int)threadIdx.x; v0 < vend; v0 += U * kST) {
      u32x4 wb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = v0 + u * kST;
        wb[u] = v < vend ? ld16(row + (size_t)v * 16) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = v0 + u * kST;
        if (v >= vend) continue;  // (no break: wb stays statically indexed)
        const u32x4 w = wb[u];
        if constexpr (DT == PKV_F32) {
#pragma unroll
          for (int j = 0; j < 4; ++j) f(v * 4 + j, __uint_as_float(w[j]));
        } else {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float lo16 = DT == PKV_BF16 ? bf16lo(w[j]) : f16lo(w[j]);
            const float hi16 = DT == PKV_BF16 ? bf16hi(w[j]) : f16hi(w[j]);
            f(v * 8 + 2 * j, lo16);
            f(v * 8 + 2 * j + 1, hi16);
          }
        }
      }
    }
    done = max(lo, vend * E);
  }
  for (int i = done + (int)threadIdx.x; i < hi; i += kST) f(i, logit<DT>(row, i));
}
template <int DT, bool VEC, int U = 1, class F>
__device__ __forceinline__ void for_each(const char* row, int V, F&& f) {
  for_range<DT, VEC, U>(row, 0, V, static_cast<F&&>(f));
}

// Larger y -> larger key; -0.0 and +0.0 compare equal, as partial_cmp has them.
__device__ __forceinline__ uint32_t order_key(float y) {
  uint32_t b = __float_as_uint(y);
  if (y == 0.0f) b = 0u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// The float whose order_key is k (keys of +0 map back to +0).
__device__ __forceinline__ float key_value(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// Logits x whose y = fl(x / T) can have a key in [kmin, kmax]: y then lies
// within one ulp of [ya, yb], so x / T does too, and x lies in the product of
// that range with T (exact in double), rounded outwards to float.  A test
// against the interval rejects other elements without the division; the
// few it admits are checked exactly.
struct XRange {
  float lo, hi;
};
__device__ __forceinline__ XRange x_range(uint32_t kmin, uint32_t kmax, float T) {
  const float ya = nextafterf(key_value(kmin), -INFINITY);
  const float yb = nextafterf(key_value(kmax), INFINITY);
  double a = (double)ya * (double)T, b = (double)yb * (double)T;
  if (a > b) {
    const double t = a;
    a = b;
    b = t;
  }
  return XRange{nextafterf((float)a, -INFINITY), nextafterf((float)b, INFINITY)};
}

// exp(d) for d = y - max y <= 0, in 2^-40 units.
__device__ __forceinline__ unsigned long long mass_of(float d) {
  const float e = expf(d);
  if (!(e > 0.0f)) return 0ull;
  if (e >= 1.0f) return kOne;
  return (unsigned long long)(e * kFix);
}

// Wave-wide steps without LDS round trips.  Reductions leave the result in
// every lane: DPP rotations within each 16-lane row, then the gfx950
// permlane16/32 swaps, which exchange values between lane and lane ^ 16
// (lane ^ 32) and return both (in either order, so any combination that
// does not depend on the order gives every lane the same result).  The
// inclusive scan shifts within rows, then broadcasts the row sums (lanes
// shifted in from outside a row read 0).  Every combination used here is
// exact (integer sums, max, min, argmax), so the order is immaterial.
template <int ROR>
__device__ __forceinline__ uint32_t ror_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x120 + ROR, 0xf, 0xf, false);
}
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t shr_u32(uint32_t x) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xf, false);
}
struct Pair32 { uint32_t a, b; };
__device__ __forceinline__ Pair32 swap16_u32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return {r[0], r[1]};
}
__device__ __forceinline__ Pair32 swap32_u32(uint32_t x) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return {r[0], r[1]};
}
__device__ __forceinline__ unsigned long long u64_of(uint32_t lo, uint32_t hi) {
  return ((unsigned long long)hi << 32) | lo;
}

// f(own, other) applied over the wave (f commutative and associative).
template <typename T, typename F>
__device__ __forceinline__ T wave_reduce32(T v, F f) {
  auto u = [](T x) { return __builtin_bit_cast(uint32_t, x); };
  auto t = [](uint32_t x) { return __builtin_bit_cast(T, x); };
  v = f(v, t(ror_u32<8>(u(v))));
  v = f(v, t(ror_u32<4>(u(v))));
  v = f(v, t(ror_u32<2>(u(v))));
  v = f(v, t(ror_u32<1>(u(v))));
  Pair32 p = swap16_u32(u(v));
  v = f(t(p.a), t(p.b));
  p = swap32_u32(u(v));
  return f(t(p.a), t(p.b));
}
__device__ __forceinline__ unsigned long long wave_sum_u64(unsigned long long v) {
  auto step = [&](uint32_t lo, uint32_t hi) { v += u64_of(lo, hi); };
  step(ror_u32<8>((uint32_t)v), ror_u32<8>((uint32_t)(v >> 32)));
  step(ror_u32<4>((uint32_t)v), ror_u32<4>((uint32_t)(v >> 32)));
  step(ror_u32<2>((uint32_t)v), ror_u32<2>((uint32_t)(v >> 32)));
  step(ror_u32<1>((uint32_t)v), ror_u32<1>((uint32_t)(v >> 32)));
  Pair32 lo = swap16_u32((uint32_t)v), hi = swap16_u32((uint32_t)(v >> 32));
  v = u64_of(lo.a, hi.a) + u64_of(lo.b, hi.b);
  lo = swap32_u32((uint32_t)v);
  hi = swap32_u32((uint32_t)(v >> 32));
  return u64_of(lo.a, hi.a) + u64_of(lo.b, hi.b);
}
// Inclusive prefix sum in lane order.
__device__ __forceinline__ unsigned long long wave_incl_u64(unsigned long long v) {
  auto step = [&](uint32_t lo, uint32_t hi) { v += u64_of(lo, hi); };
  step(shr_u32<0x111, 0xf>((uint32_t)v), shr_u32<0x111, 0xf>((uint32_t)(v >> 32)));  // row_shr:1
  step(shr_u32<0x112, 0xf>((uint32_t)v), shr_u32<0x112, 0xf>((uint32_t)(v >> 32)));  // row_shr:2
  step(shr_u32<0x114, 0xf>((uint32_t)v), shr_u32<0x114, 0xf>((uint32_t)(v >> 32)));  // row_shr:4
  step(shr_u32<0x118, 0xf>((uint32_t)v), shr_u32<0x118, 0xf>((uint32_t)(v >> 32)));  // row_shr:8
  step(shr_u32<0x142, 0xa>((uint32_t)v), shr_u32<0x142, 0xa>((uint32_t)(v >> 32)));  // row_bcast:15
  step(shr_u32<0x143, 0xc>((uint32_t)v), shr_u32<0x143, 0xc>((uint32_t)(v >> 32)));  // row_bcast:31
  return v;
}

__device__ float block_max(SampleSmem& sm, float v) {
  v = wave_reduce32(v, [](float x, float y) { return fmaxf(x, y); });
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) sm.red_f[wv] = v;
  __syncthreads();
  float r = sm.red_f[0];
  for (int w = 1; w < kSW; ++w) r = fmaxf(r, sm.red_f[w]);
  __syncthreads();
  return r;
}

__device__ unsigned long long block_sum_u64(SampleSmem& sm, unsigned long long v) {
  v = wave_sum_u64(v);
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) sm.red_u[wv] = v;
  __syncthreads();
  unsigned long long r = 0;
  for (int w = 0; w < kSW; ++w) r += sm.red_u[w];
  __syncthreads();
  return r;
}

__device__ int block_min_i(SampleSmem& sm, int v) {
  v = wave_reduce32(v, [](int x, int y) { return min(x, y); });
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  if (lane == 0) sm.red_i[wv] = v;
  __syncthreads();
  int r = sm.red_i[0];
  for (int w = 1; w < kSW; ++w) r = min(r, sm.red_i[w]);
  __syncthreads();
  return r;
}

// Finds in hist[0..nb) (nb = 4096 or 1024), walking from the top bucket
// down, the first bucket where the running total reaches rem, and records
// it in sm.sel_bucket and what is still needed inside it in sm.sel_rem.
// Thread t owns the nb / kST buckets from nb-1-t*per down; a block-wide
// inclusive scan of the threads' sums finds the first thread whose running
// total reaches rem, and that thread walks its buckets in order.  The
// histograms always hold at least rem below the digits chosen so far; if
// that ever failed, the smallest non-empty bucket is taken so that the row
// still ends with a token.  Call from all threads; ends with a barrier.
__device__ void scan_buckets(SampleSmem& sm, const unsigned long long* hist, int nb,
                             unsigned long long rem) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int per = nb / kST;
  const int hi = nb - 1 - tid * per;
  unsigned long long seg = 0;
  for (int j = 0; j < per; ++j) seg += hist[hi - j];
  unsigned long long incl = wave_incl_u64(seg);  // inclusive scan over the wave
  if (lane == 63) sm.red_u[wv] = incl;
  __syncthreads();
  for (int w = 0; w < wv; ++w) incl += sm.red_u[w];
  const unsigned long long reach = __ballot(incl >= rem);
  const unsigned long long nonempty = __ballot(seg != 0ull);
  if (lane == 0) {
    sm.red_i[wv] = reach ? __builtin_ctzll(reach) : -1;                   // first reaching lane
    sm.red_j[wv] = nonempty ? 63 - __builtin_clzll(nonempty) : -1;        // last non-empty lane
  }
  __syncthreads();
  int chosen_t = -1, last_t = -1;
  for (int w = 0; w < kSW; ++w) {
    if (chosen_t < 0 && sm.red_i[w] >= 0) chosen_t = w * 64 + sm.red_i[w];
    if (sm.red_j[w] >= 0) last_t = w * 64 + sm.red_j[w];
  }
  const int ft = chosen_t >= 0 ? chosen_t : (last_t >= 0 ? last_t : 0);
  if (tid == ft) {
    unsigned long long acc = incl - seg;
    int chosen = -1, last_nonempty = hi;
    for (int j = 0; j < per; ++j) {
      const unsigned long long h = hist[hi - j];
      if (h) last_nonempty = hi - j;
      if (h && acc + h >= rem) {
        chosen = hi - j;
        break;
      }
      acc += h;
    }
    unsigned long long r2 = rem - acc;
    if (chosen < 0) {
      chosen = last_nonempty;
      r2 = hist[chosen] ? hist[chosen] : 1ull;
    }
    sm.sel_bucket = (uint32_t)chosen;
    sm.sel_rem = r2;
  }
  __syncthreads();
}

// Per-row context of the temperature path.
template <int DT, bool VEC>
struct Row {
  const char* x;
  int V;
  float T, ymax;
  bool has_k;
  uint32_t kkey;  // top_k: key of the k-th largest value
  int kcut;       // top_k: last index kept among the tokens with that key
  __device__ bool kept(int i, uint32_t key) const {
    return !has_k || key > kkey || (key == kkey && i <= kcut);
  }
};

struct Sel {
  uint32_t key;             // the selected key (all 32 bits)
  unsigned long long rem;   // what is still needed inside its tie group
  unsigned long long hist;  // the tie group's total (mass, or count)
  unsigned long long cnt;   // the tie group's size
  int minidx;               // its smallest index
};

// One digit of a selection over row[lo, hi): sm.h gets the histogram of
// key bits shift..shift+9 among the tokens whose key equals `prefix` under
// `pmask` (COUNT: every token; otherwise kept tokens' mass) and, for the
// last digit, sm.cnt / sm.minidx each bucket's size and smallest index.
// Elements whose logit lies outside the prefix's logit interval are
// rejected before the division.  Call from all threads; ends with a barrier.
template <bool COUNT, int DT, bool VEC>
__device__ void digit_pass(SampleSmem& sm, const Row<DT, VEC>& rw, int lo, int hi,
                           uint32_t prefix, uint32_t pmask, int shift, bool last) {
  for (int b = threadIdx.x; b < kB2; b += kST) {
    sm.h[b] = 0ull;
    sm.cnt[b] = 0u;
    sm.minidx[b] = INT_MAX;
  }
  __syncthreads();
  const XRange xr = x_range(prefix, prefix | ~pmask, rw.T);
  for_range<DT, VEC>(rw.x, lo, hi, [&](int i, float x) {
    if (!(x >= xr.lo && x <= xr.hi)) return;
    const float y = x / rw.T;
    const uint32_t key = order_key(y);
    if ((key & pmask) != prefix) return;
    const uint32_t b = (key >> shift) & (uint32_t)(kB2 - 1);
    if constexpr (COUNT) {
      atomicAdd(&sm.h[b], 1ull);
    } else {
      if (!rw.kept(i, key)) return;
      const unsigned long long m = mass_of(y - rw.ymax);
      if (m == 0ull) return;
      atomicAdd(&sm.h[b], m);
    }
    if (last) {
      atomicAdd(&sm.cnt[b], 1u);
      atomicMin(&sm.minidx[b], i);
    }
  });
  __syncthreads();
}

// Second and third digits of a selection whose first-digit histogram is
// sm.h1: COUNT counts every token, otherwise kept tokens' mass.
template <bool COUNT, int DT, bool VEC>
__device__ Sel select_low(SampleSmem& sm, const Row<DT, VEC>& rw, unsigned long long target) {
  scan_buckets(sm, sm.h1, kB1, target);
  uint32_t prefix = sm.sel_bucket << 20;
  unsigned long long rem = sm.sel_rem;
  Sel out{};
  for (int pass = 0; pass < 2; ++pass) {
    const int shift = pass == 0 ? 10 : 0;
    const uint32_t pmask = pass == 0 ? 0xfff00000u : 0xfffffc00u;
    const bool last = pass == 1;
    __syncthreads();  // every thread has read sm.sel_* before it is reused
    digit_pass<COUNT>(sm, rw, 0, rw.V, prefix, pmask, shift, last);
    scan_buckets(sm, sm.h, kB2, rem);
    const uint32_t b = sm.sel_bucket;
    rem = sm.sel_rem;
    prefix |= b << shift;
    if (last) {
      out.hist = sm.h[b];
      out.cnt = sm.cnt[b];
      out.minidx = sm.minidx[b];
    }
  }
  __syncthreads();
  out.key = prefix;
  out.rem = rem;
  return out;
}

// Index of the n-th (1-based) token, in index order, whose key is `key` and
// that the top_k filter keeps (FILTER); V - 1 if there is none.  Only used
// when more than one token of a tie group is needed.  Each step gives every
// thread a contiguous chunk of kTE elements (64 bytes: four 16-byte loads
// when the row is aligned), marks the matches in a bit mask (the logit
// interval of the key rejects most elements before the division), and a
// block-wide exclusive scan of the per-thread counts, in index order, finds
// the thread holding the n-th match.
template <bool FILTER, int DT, bool VEC>
__device__ __forceinline__ int nth_tied(SampleSmem& sm, const Row<DT, VEC>& rw, uint32_t key,
                        unsigned long long n, int lo = 0, int hi = -1) {
  if (hi < 0) hi = rw.V;  // the walk covers [lo, hi); lo is a multiple of 8
  constexpr int E = DT == PKV_F32 ? 4 : 2;  // element bytes
  constexpr int kTE = 64 / E;               // elements per thread per step
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const XRange xr = x_range(key, key, rw.T);
  if (tid == 0) sm.found = rw.V - 1;
  __syncthreads();
  unsigned long long base = 0;
  for (int c = lo; c < hi; c += kST * kTE) {
    const int i0 = c + tid * kTE;
    float xs[kTE];
    if (VEC && i0 + kTE <= hi) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const u32x4 w = ld16(rw.x + (size_t)i0 * E + 16 * q);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          if constexpr (DT == PKV_F32) {
            xs[4 * q + j] = __uint_as_float(w[j]);
          } else {
            xs[8 * q + 2 * j] = DT == PKV_BF16 ? bf16lo(w[j]) : f16lo(w[j]);
            xs[8 * q + 2 * j + 1] = DT == PKV_BF16 ? bf16hi(w[j]) : f16hi(w[j]);
          }
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < kTE; ++e) xs[e] = i0 + e < hi ? logit<DT>(rw.x, i0 + e) : NAN;
    }
    uint32_t mask = 0u;
#pragma unroll
    for (int e = 0; e < kTE; ++e) {
      const float x = xs[e];  // NaN (past the end) fails the interval test
      if (!(x >= xr.lo && x <= xr.hi)) continue;
      const uint32_t k = order_key(x / rw.T);
      if (k == key && (!FILTER || rw.kept(i0 + e, k))) mask |= 1u << e;
    }
    const int cnt = __popc(mask);
    int incl = cnt;  // inclusive scan over the wave, in lane (= index) order (DPP)
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x111, 0xf, 0xf, false);  // row_shr:1
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x112, 0xf, 0xf, false);  // row_shr:2
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x114, 0xf, 0xf, false);  // row_shr:4
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x118, 0xf, 0xf, false);  // row_shr:8
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x142, 0xa, 0xf, false);  // row_bcast:15
    incl += __builtin_amdgcn_update_dpp(0, incl, 0x143, 0xc, 0xf, false);  // row_bcast:31
    if (lane == 63) sm.red_i[wv] = incl;
    __syncthreads();
    int off = 0, tot = 0;
    for (int w = 0; w < kSW; ++w) {
      const int cw = sm.red_i[w];
      off += w < wv ? cw : 0;
      tot += cw;
    }
    const unsigned long long before = base + (unsigned long long)(off + incl - cnt);
    if (cnt > 0 && before < n && n <= before + (unsigned long long)cnt) {
      uint32_t m = mask;
      for (unsigned long long k = n - before; k > 1ull; --k) m &= m - 1u;  // drop lower matches
      sm.found = i0 + __builtin_ctz(m);
    }
    __syncthreads();
    base += (unsigned long long)tot;
    if (base >= n) break;
  }
  const int r = sm.found;
  __syncthreads();
  return r;
}

__device__ __forceinline__ unsigned long long clamp_target(double t, unsigned long long hi) {
  unsigned long long v = t >= (double)hi ? hi : (unsigned long long)ceil(t > 0.0 ? t : 0.0);
  return v < 1ull ? 1ull : (v > hi ? hi : v);
}

// How many tokens of the selected tie group the remaining mass needs.
__device__ __forceinline__ unsigned long long ties_needed(const Sel& s) {
  const unsigned long long per = s.cnt ? s.hist / s.cnt : s.hist;
  unsigned long long n = per ? (s.rem + per - 1ull) / per : 1ull;
  if (n > s.cnt) n = s.cnt;
  return n < 1ull ? 1ull : n;
}

// First maximum of row[lo, hi) (strictly greater values only, so the first
// maximum wins; NaN is never taken): (value, index), index INT_MAX when no
// value exceeds -inf.  The result is valid in thread 0.
template <int DT, bool VEC>
__device__ __forceinline__ void block_argmax(SampleSmem& sm, const char* x, int lo, int hi, float& bv, int& bi) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  bv = -INFINITY;
  bi = INT_MAX;
  for_range<DT, VEC>(x, lo, hi, [&](int i, float v) {
    if (v > bv) {
      bv = v;
      bi = i;
    }
  });
  {
    // (value, index) pairs: the larger value, the smaller index on a tie
    auto take = [&](uint32_t ov_bits, uint32_t oi_bits) {
      const float ov = __uint_as_float(ov_bits);
      const int oi = (int)oi_bits;
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    };
    take(ror_u32<8>(__float_as_uint(bv)), ror_u32<8>((uint32_t)bi));
    take(ror_u32<4>(__float_as_uint(bv)), ror_u32<4>((uint32_t)bi));
    take(ror_u32<2>(__float_as_uint(bv)), ror_u32<2>((uint32_t)bi));
    take(ror_u32<1>(__float_as_uint(bv)), ror_u32<1>((uint32_t)bi));
    Pair32 pv = swap16_u32(__float_as_uint(bv)), pi = swap16_u32((uint32_t)bi);
    bv = __uint_as_float(pv.a);
    bi = (int)pi.a;
    take(pv.b, pi.b);
    pv = swap32_u32(__float_as_uint(bv));
    pi = swap32_u32((uint32_t)bi);
    bv = __uint_as_float(pv.a);
    bi = (int)pi.a;
    take(pv.b, pi.b);
  }
  if (lane == 0) {
    sm.red_f[wv] = bv;
    sm.red_i[wv] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kSW; ++w) {
      const float ov = sm.red_f[w];
      const int oi = sm.red_i[w];
      if (ov > bv || (ov == bv && oi < bi)) {
        bv = ov;
        bi = oi;
      }
    }
  }
}

// The largest x (T > 0) or -x (T < 0) of row[lo, hi), in every thread.
// max of fl(x / T) needs no division: correctly rounded division is
// monotone in x, so it is that value divided by T (ymax_of).
template <int DT, bool VEC>
__device__ float block_xmax(SampleSmem& sm, const char* x, int lo, int hi, float T) {
  float xm = -INFINITY;
  if (T > 0.0f)
    for_range<DT, VEC>(x, lo, hi, [&](int, float v) { xm = fmaxf(xm, v); });
  else
    for_range<DT, VEC>(x, lo, hi, [&](int, float v) { xm = fmaxf(xm, -v); });
  return block_max(sm, xm);
}
__device__ __forceinline__ float ymax_of(float xm, float T) { return (T > 0.0f ? xm : -xm) / T; }

// First digit of the mass histogram over row[lo, hi), added to sm.h1.
template <int DT, bool VEC>
__device__ void mass_pass(SampleSmem& sm, const Row<DT, VEC>& rw, int lo, int hi) {
  for_range<DT, VEC>(rw.x, lo, hi, [&](int i, float v) {
    const float y = v / rw.T;
    const uint32_t key = order_key(y);
    if (!rw.kept(i, key)) return;
    const unsigned long long m = mass_of(y - rw.ymax);
    if (m) atomicAdd(&sm.h1[key >> 20], m);
  });
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) sample_kernel(SampleArgs a) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.x;
  const int tid = threadIdx.x;
  const char* x = a.logits + (long long)row * a.stride_bytes;
  const int V = a.vocab;
  const float T = a.temps ? a.temps[row] : 0.0f;

  if (T == 0.0f || V <= 1) {
    float bv;
    int bi;
    block_argmax<DT, VEC>(sm, x, 0, V, bv, bi);
    if (tid == 0) a.tokens[row] = bi == INT_MAX ? 0 : bi;
    return;
  }

  Row<DT, VEC> rw{x, V, T, 0.0f, false, 0u, V};
  rw.ymax = ymax_of(block_xmax<DT, VEC>(sm, x, 0, V, T), T);

  if (a.top_k > 0 && a.top_k < V) {
    // the k-th largest key, and how many of its ties the first k include
    for (int b = tid; b < kB1; b += kST) sm.h1[b] = 0ull;
    __syncthreads();
    for_each<DT, VEC>(x, V, [&](int, float v) { atomicAdd(&sm.h1[order_key(v / T) >> 20], 1ull); });
    __syncthreads();
    const Sel s = select_low<true>(sm, rw, (unsigned long long)a.top_k);
    rw.kkey = s.key;
    rw.kcut = s.rem >= s.cnt ? V : (s.rem <= 1ull ? s.minidx : nth_tied<false>(sm, rw, s.key, s.rem));
    rw.has_k = true;
  }

  // first digit of the mass histogram; its buckets add up to the total mass
  for (int b = tid; b < kB1; b += kST) sm.h1[b] = 0ull;
  __syncthreads();
  mass_pass<DT, VEC>(sm, rw, 0, V);
  __syncthreads();
  unsigned long long part = 0;
  for (int b = tid; b < kB1; b += kST) part += sm.h1[b];
  unsigned long long total = block_sum_u64(sm, part);

  if (a.top_p < 1.0f) {
    // the shortest sorted prefix whose mass reaches top_p of the total
    const unsigned long long tp = clamp_target((double)a.top_p * (double)total, total);
    const Sel s = select_low<false>(sm, rw, tp);
    const unsigned long long per = s.cnt ? s.hist / s.cnt : s.hist;
    total = tp - s.rem + ties_needed(s) * per;
  }
  const unsigned long long tr = clamp_target((double)a.r * (double)total, total);
  const Sel s = select_low<false>(sm, rw, tr);
  const unsigned long long n = ties_needed(s);
  const int tok = n == 1ull ? (s.minidx == INT_MAX ? V - 1 : s.minidx)
                            : nth_tied<true>(sm, rw, s.key, n);
  if (tid == 0) a.tokens[row] = tok;
}

// ---- small batches: each row split over G workgroups -----------------------
// Without top_k / top_p, a row's selection needs its max, the first-digit
// mass histogram and two more digit histograms; each is a sum over the row,
// so G workgroups (blockIdx.x) can each take a contiguous chunk and add
// their part in global memory, one launch per pass (the launch boundary
// orders the passes; no workgroup waits for another).  The masses are the
// same integers as in sample_kernel and integer sums do not depend on their
// order, so the token is the same as sample_kernel's.  Launches: max (which
// also clears the histograms), mass, second digit, third digit, finish (one
// workgroup per row: the last scan, a tie walk when needed, the token).
constexpr int kMaxG = 32;
static_assert(kB1 % kST == 0 && kB2 == kST && kMaxG <= kST, "split-path loads");
static_assert(sizeof(unsigned long long) % alignof(unsigned int) == 0, "");
struct SplitWs {  // per row
  float pmax[kMaxG];  // per workgroup: max x / -x (sampled), max x (greedy)
  int pidx[kMaxG];    // greedy: index of that max (INT_MAX: none)
  unsigned long long h1[kB1];
  unsigned long long h2[kB2];
  unsigned long long h3[kB2];
  unsigned int cnt3[kB2];
  int min3[kB2];
  uint32_t pre1, pre2;            // first one / two digits of the selected key
  unsigned long long rem1, rem2;  // what remains to select inside them
};
// Behind the batch's SplitWs rows: the third digit's tokens per bucket in
// each chunk, [batch][G][kB2] unsigned ints, sized by the call's G.
__device__ __forceinline__ unsigned int* chunk_counts(SplitWs* ws, int batch, int row, int G,
                                                      int g) {
  return reinterpret_cast<unsigned int*>(ws + batch) + ((size_t)row * G + g) * kB2;
}

// Workgroup blockIdx.x's chunk of a row: multiples of 8 elements (whole
// 16-byte vectors for every dtype), the last one ending at V.
__device__ __forceinline__ void chunk_of(int V, int g, int G, int& lo, int& hi) {
  const int ce = (((V + G - 1) / G) + 7) / 8 * 8;
  lo = min(V, g * ce);
  hi = min(V, lo + ce);
}
__device__ __forceinline__ void split_chunk(int V, int& lo, int& hi) {
  chunk_of(V, (int)blockIdx.x, (int)gridDim.x, lo, hi);
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) split_max_kernel(SampleArgs a, SplitWs* ws) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.y, g = blockIdx.x, G = gridDim.x, tid = threadIdx.x;
  SplitWs& w = ws[row];
  for (int i = g * kST + tid; i < kB1; i += G * kST) w.h1[i] = 0ull;
  for (int i = g * kST + tid; i < kB2; i += G * kST) {
    w.h2[i] = 0ull;
    w.h3[i] = 0ull;
    w.cnt3[i] = 0u;
    w.min3[i] = INT_MAX;
  }
  const char* x = a.logits + (long long)row * a.stride_bytes;
  const float T = a.temps ? a.temps[row] : 0.0f;
  int lo, hi;
  split_chunk(a.vocab, lo, hi);
  if (T == 0.0f || a.vocab <= 1) {
    float bv;
    int bi;
    block_argmax<DT, VEC>(sm, x, lo, hi, bv, bi);
    if (tid == 0) {
      w.pmax[g] = bv;
      w.pidx[g] = bi;
    }
    return;
  }
  const float xm = block_xmax<DT, VEC>(sm, x, lo, hi, T);
  if (tid == 0) w.pmax[g] = xm;
}

// The row's global histograms as the later passes read them, loaded with
// one round trip at the start of a launch: thread t's first-digit buckets
// t + kST j, its second- and third-digit bucket t, and the per-workgroup
// maxima (threads below G).
struct SplitLoad {
  unsigned long long h1[kB1 / kST];
  unsigned long long h2, h3;
  unsigned int cnt3;
  int min3;
  float pmax;
};
__device__ __forceinline__ SplitLoad split_load(const SplitWs& w, int G, int digits) {
  const int tid = threadIdx.x;
  SplitLoad l;
#pragma unroll
  for (int j = 0; j < kB1 / kST; ++j) l.h1[j] = digits >= 1 ? w.h1[tid + j * kST] : 0ull;
  l.h2 = digits >= 2 ? w.h2[tid] : 0ull;
  l.h3 = digits >= 3 ? w.h3[tid] : 0ull;
  l.cnt3 = digits >= 3 ? w.cnt3[tid] : 0u;
  l.min3 = digits >= 3 ? w.min3[tid] : INT_MAX;
  l.pmax = tid < G ? w.pmax[tid] : -INFINITY;
  return l;
}

// From the loaded histograms: the selection target r * total and the first
// `digits` (1 or 2) digits chosen so far; sm.h1 holds the first-digit
// histogram afterwards.
__device__ void split_prefix(SampleSmem& sm, const SplitLoad& l, float r, int digits,
                             uint32_t& prefix, unsigned long long& rem) {
  const int tid = threadIdx.x;
  unsigned long long part = 0;
#pragma unroll
  for (int j = 0; j < kB1 / kST; ++j) {
    sm.h1[tid + j * kST] = l.h1[j];
    part += l.h1[j];
  }
  if (digits == 2) sm.h[tid] = l.h2;
  const unsigned long long total = block_sum_u64(sm, part);  // barriers: LDS complete
  scan_buckets(sm, sm.h1, kB1, clamp_target((double)r * (double)total, total));
  prefix = sm.sel_bucket << 20;
  rem = sm.sel_rem;
  if (digits == 2) {
    __syncthreads();  // every thread has read sm.sel_*
    scan_buckets(sm, sm.h, kB2, rem);
    prefix |= sm.sel_bucket << 10;
    rem = sm.sel_rem;
  }
  __syncthreads();  // every thread has read sm.sel_*
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) split_mass_kernel(SampleArgs a, SplitWs* ws) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.y, tid = threadIdx.x;
  const SplitWs& w = ws[row];
  const float pm = tid < (int)gridDim.x ? w.pmax[tid] : -INFINITY;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || a.vocab <= 1) return;
  const char* x = a.logits + (long long)row * a.stride_bytes;
  for (int b = tid; b < kB1; b += kST) sm.h1[b] = 0ull;
  Row<DT, VEC> rw{x, a.vocab, T, ymax_of(block_max(sm, pm), T), false, 0u, a.vocab};
  int lo, hi;
  split_chunk(a.vocab, lo, hi);
  mass_pass<DT, VEC>(sm, rw, lo, hi);
  __syncthreads();
  for (int b = tid; b < kB1; b += kST)
    if (sm.h1[b]) atomicAdd(&ws[row].h1[b], sm.h1[b]);
}

template <int DT, bool VEC, bool LAST>
__global__ void __launch_bounds__(kST) split_digit_kernel(SampleArgs a, SplitWs* ws) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.y, tid = threadIdx.x;
  const SplitLoad l = split_load(ws[row], gridDim.x, LAST ? 2 : 1);
  const uint32_t pre1 = LAST ? ws[row].pre1 : 0u;  // issued with the histogram loads
  const unsigned long long rem1 = LAST ? ws[row].rem1 : 0ull;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || a.vocab <= 1) return;
  const char* x = a.logits + (long long)row * a.stride_bytes;
  Row<DT, VEC> rw{x, a.vocab, T, ymax_of(block_max(sm, l.pmax), T), false, 0u, a.vocab};
  uint32_t prefix;
  unsigned long long rem;
  if constexpr (LAST) {
    // the first digit was selected by the second digit pass (workgroup 0
    // stored it): only the second digit's scan is left
    sm.h[tid] = l.h2;
    __syncthreads();
    scan_buckets(sm, sm.h, kB2, rem1);
    prefix = pre1 | (sm.sel_bucket << 10);
    rem = sm.sel_rem;
    __syncthreads();  // every thread has read sm.sel_*
  } else {
    split_prefix(sm, l, a.r, 1, prefix, rem);
  }
  if (blockIdx.x == 0 && tid == 0) {  // for the next launch
    if (LAST) {
      ws[row].pre2 = prefix;
      ws[row].rem2 = rem;
    } else {
      ws[row].pre1 = prefix;
      ws[row].rem1 = rem;
    }
  }
  int lo, hi;
  split_chunk(a.vocab, lo, hi);
  digit_pass<false>(sm, rw, lo, hi, prefix, LAST ? 0xfffffc00u : 0xfff00000u, LAST ? 0 : 10,
                    LAST);
  SplitWs& w = ws[row];
  if (LAST) {  // every bucket, zeros included: no clearing needed
    unsigned int* cc = chunk_counts(ws, (int)gridDim.y, row, (int)gridDim.x, (int)blockIdx.x);
    for (int b = tid; b < kB2; b += kST) cc[b] = sm.cnt[b];
  }
  for (int b = tid; b < kB2; b += kST) {
    if (!sm.h[b]) continue;
    atomicAdd(LAST ? &w.h3[b] : &w.h2[b], sm.h[b]);
    if (LAST) {
      atomicAdd(&w.cnt3[b], sm.cnt[b]);
      atomicMin(&w.min3[b], sm.minidx[b]);
    }
  }
}

template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) split_finish_kernel(SampleArgs a, SplitWs* ws, int G) {
  __shared__ SampleSmem sm;
  const int row = blockIdx.x, tid = threadIdx.x;
  const SplitWs& w = ws[row];
  const int V = a.vocab;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || V <= 1) {
    if (tid == 0) {  // chunks in index order: strictly greater keeps the first maximum
      float bv = -INFINITY;
      int bi = INT_MAX;
      for (int g = 0; g < G; ++g) {
        if (w.pmax[g] > bv) {
          bv = w.pmax[g];
          bi = w.pidx[g];
        }
      }
      a.tokens[row] = bi == INT_MAX ? 0 : bi;
    }
    return;
  }
  // The first two digits were selected by the third digit pass (the same
  // scans in every one of its workgroups; workgroup 0 stored the result).
  const uint32_t prefix = w.pre2;
  const unsigned long long rem = w.rem2;
  sm.h[tid] = w.h3[tid];
  sm.cnt[tid] = w.cnt3[tid];
  sm.minidx[tid] = w.min3[tid];
  const char* x = a.logits + (long long)row * a.stride_bytes;
  Row<DT, VEC> rw{x, V, T, 0.0f, false, 0u, V};  // the tie walk reads no ymax
  __syncthreads();
  scan_buckets(sm, sm.h, kB2, rem);
  const uint32_t b = sm.sel_bucket;
  Sel s;
  s.key = prefix | b;
  s.rem = sm.sel_rem;
  s.hist = sm.h[b];
  s.cnt = sm.cnt[b];
  s.minidx = sm.minidx[b];
  __syncthreads();
  const unsigned long long n = ties_needed(s);
  int tok;
  if (n == 1ull) {
    tok = s.minidx == INT_MAX ? V - 1 : s.minidx;
  } else {
    // The chunks' counts of the selected key, in index order, locate the
    // chunk holding the n-th tied token; only that chunk is walked.
    if (tid < kWave) {
      const unsigned long long c =
          tid < G ? (unsigned long long)chunk_counts(ws, (int)gridDim.x, row, G, tid)[b] : 0ull;
      const unsigned long long incl = wave_incl_u64(c);
      const unsigned long long hit = __ballot(incl >= n);
      if (tid == 0 && !hit) sm.red_i[0] = -1;  // counts inconsistent: walk the row
      if (hit && tid == __ffsll((long long)hit) - 1) {
        sm.red_i[0] = tid;
        sm.red_u[0] = n - (incl - c);
      }
    }
    __syncthreads();
    const int gs = sm.red_i[0];
    const unsigned long long nn = gs < 0 ? n : sm.red_u[0];
    __syncthreads();  // nth_tied reuses sm.red_i
    int lo = 0, hi = V;
    if (gs >= 0) chunk_of(V, gs, G, lo, hi);
    tok = nth_tied<true>(sm, rw, s.key, nn, lo, hi);
  }
  if (tid == 0) a.tokens[row] = tok;
}

// ---- bit-exact sample(): the reference's own f32 arithmetic -----------------
// sample.rs:16-47 sorts y = x / T (stable, descending), keeps the first
// top_k, takes p_i = (y_i - max).exp() with f32::exp, adds the p_i in sorted
// order in f32, divides each by that sum, (top_p: adds them again in f32
// until the running sum reaches top_p, truncates there and divides by the
// truncated sum), and returns the first token at which the f32 running sum
// reaches r.  sample_exact_kernel reproduces every one of those values bit
// for bit, so the token is the reference's on every input, including rows
// where f32 rounding alone moves the pick:
//  * exp: f32::exp is the C library's expf on the reference's host (on
//    x86-64 Linux, glibc).  expf_glibc restates glibc's expf (the algorithm
//    of Arm's Optimized Routines, glibc >= 2.28, as built for x86-64 with
//    FMA); it was checked against the host libm on every float <= 0, the
//    only arguments it gets here (y - max <= 0).
//  * order: a stable LSD radix sort of the order keys (four passes of 8 bits)
//    keeps equal y in index order, as the reference's stable sort does.
//  * f32 running sums: f32_run (below) gives the exact sequence of
//    rounded sums without a 128k-long serial chain.
// The token of the selected sorted position is found with the fast path's
// tie walk (the n-th token of that value in index order).

// glibc expf's table: 2^(i/32) rounded to double, minus i << 47 (so that
// adding k << 47 scales it by 2^(k/32 - i/32)).
__constant__ unsigned long long kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// glibc's expf: x N / ln2 = k + r (N = 32, k rounded to nearest by adding
// 1.5 * 2^52), exp(x) = 2^(k/N) * 2^(r/N), the second factor a cubic in r
// with the published minimax coefficients, evaluated in double and rounded
// once to float.  Algorithm, table values and coefficients: Arm Optimized
// Routines (math/expf.c, exp2f_data.c; Copyright (c) Arm Limited, MIT OR
// Apache-2.0 WITH LLVM-exception), the expf glibc has used since 2.28.  The reduction r = x N / ln2 - k is one fused multiply-add
// (as GCC contracts it when glibc is built for FMA hardware); every other
// operation is a separately rounded double operation, in glibc's order.
// The main path (x not NaN, -0x1.9fe368p6 <= x <= 0x1.62e42ep6), the table
// at tab (kExp2Tab, or a copy in LDS).
__device__ __forceinline__ float expf_glibc_main(float x, const unsigned long long* tab) {
#pragma clang fp contract(off)
  constexpr double kN = 32.0;
  constexpr double kInvLn2N = 0x1.71547652b82fep0 * kN;
  constexpr double kShift = 0x1.8p52;
  constexpr double kC0 = 0x1.c6af84b912394p-5 / kN / kN / kN;
  constexpr double kC1 = 0x1.ebfce50fac4f3p-3 / kN / kN;
  constexpr double kC2 = 0x1.62e42ff0c52d6p-1 / kN;
  const double xd = (double)x;
  const double z = kInvLn2N * xd;
  double kd = z + kShift;
  const unsigned long long ki = (unsigned long long)__double_as_longlong(kd);
  kd -= kShift;
  const double r = __builtin_fma(kInvLn2N, xd, -kd);
  const unsigned long long t = tab[ki % 32] + (ki << 47);
  const double s = __longlong_as_double((long long)t);
  const double zz = __builtin_fma(kC0, r, kC1);
  const double r2 = r * r;
  double y = __builtin_fma(kC2, r, 1.0);
  y = __builtin_fma(zz, r2, y);
  y = y * s;
  return (float)y;
}
__device__ __forceinline__ float expf_glibc(float x) {
  if (x != x) return x + x;
  if (x == -INFINITY) return 0.0f;
  if (x > 0x1.62e42ep6f) return INFINITY;  // overflow (arguments here are <= 0)
  if (x < -0x1.9fe368p6f) return 0.0f;     // below half the smallest subnormal
  return expf_glibc_main(x, kExp2Tab);
}

constexpr int kXBits = 8;             // radix sort: bits per pass
constexpr int kXR = 1 << kXBits;      // buckets per pass
constexpr int kNoDelta = INT_MIN;     // f32_run: chunk without a precomputed delta
constexpr int kDeltaCap = (1 << 24) + 1;  // deltas this large always leave the binade
constexpr int kRunChunks = 2048;      // f32_run: chunks at most
constexpr int kXU = 8;                // 64-element batches of loads in flight per wave

struct ExactSmem {
  unsigned int off[kSW][kXR];       // radix pass: per-wave digit counts, then positions
  unsigned int wtot[kSW];
  float wsum[kSW];
  float csum[kRunChunks];           // f32_run: chunk sums, then exclusive prefixes
  int ce[kRunChunks];               // binade the chunk's delta assumes (kNoDelta: none)
  int cd0[kRunChunks], cd1[kRunChunks];  // its delta for an even / odd start
  float s;                          // f32_run result: the sum reached
  int pos;                          //   and the number of elements it took
  int flag;
};

// Inclusive prefix sums across the wave in lane order on DPP: row shifts
// within the 16-lane rows, then the row broadcasts of the lane-15 and
// lane-31 partials (no LDS round trips).  The float version adds in a
// different order than a serial sum (its callers use it for estimates only).
__device__ __forceinline__ unsigned int wave_incl_add_u32(unsigned int x) {
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x111, 0xf, 0xf, false);
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x112, 0xf, 0xf, false);
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x114, 0xf, 0xf, false);
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x118, 0xf, 0xf, false);
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x142, 0xa, 0xf, false);
  x += (unsigned int)__builtin_amdgcn_update_dpp(0, (int)x, 0x143, 0xc, 0xf, false);
  return x;
}
__device__ __forceinline__ float wave_incl_add_f32(float x) {
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x111, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x112, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x114, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x118, 0xf, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x142, 0xa, 0xf, false));
  x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x143, 0xc, 0xf, false));
  return x;
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
  return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xf, 0xf, false);
}
// Sums over the wave; every lane receives the total (DPP row rotations, then
// the gfx950 permlane swaps across rows).
__device__ __forceinline__ int wsum_i32(int x) {
  x += dpp_i<0x128>(x);
  x += dpp_i<0x124>(x);
  x += dpp_i<0x122>(x);
  x += dpp_i<0x121>(x);
  const auto a = __builtin_amdgcn_permlane16_swap((unsigned)x, (unsigned)x, false, false);
  x = (int)(a[0] + a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap((unsigned)x, (unsigned)x, false, false);
  return (int)(b[0] + b[1]);
}
__device__ __forceinline__ float wsum_f32(float x) { return swap32_sum(swap16_sum(row_sum16(x))); }

// Lanes of the batch whose key has this lane's digit d (valid lanes only).
__device__ __forceinline__ unsigned long long digit_match(uint32_t d, bool valid) {
  unsigned long long match = __ballot(valid);
#pragma unroll
  for (int b = 0; b < kXBits; ++b) {
    const bool bit = (d >> b) & 1u;
    const unsigned long long bal = __ballot(bit);
    match &= bit ? bal : ~bal;
  }
  return match;
}

// One stable pass of the LSD radix sort: src[0, n) -> dst by key bits
// [shift, shift + 8).  Wave w owns a contiguous segment, read 64 keys at a
// time in order.  Within a batch, the keys sharing a digit are found with
// eight ballots: the group's highest lane adds the group's size to the
// wave's count for the digit (no contended atomics), and in the scatter a
// key's rank in its group plus the wave's running position for the digit
// (counts scanned digit-major, wave-minor) gives its place.  When every key
// has the same digit the pass would move nothing: it returns false and
// leaves dst alone.  Ends with a barrier.
__device__ __forceinline__ bool radix_pass(ExactSmem& xs, const uint32_t* src, uint32_t* dst, int n, int shift) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int seg = ((n + kSW - 1) / kSW + 63) / 64 * 64;
  const int w0 = min(n, wv * seg), w1 = min(n, w0 + seg);
  for (int i = tid; i < kSW * kXR; i += kST) (&xs.off[0][0])[i] = 0u;
  if (tid == 0) xs.flag = 0;
  __syncthreads();
  for (int i0 = w0; i0 < w1; i0 += 64 * kXU) {
    uint32_t kk[kXU];
#pragma unroll
    for (int u = 0; u < kXU; ++u) {
      const int i = i0 + 64 * u + lane;
      kk[u] = i < w1 ? src[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kXU; ++u) {
      const bool valid = i0 + 64 * u + lane < w1;
      const uint32_t d = (kk[u] >> shift) & (kXR - 1);
      const unsigned long long match = digit_match(d, valid);
      if (valid && (match >> lane) == 1ull) xs.off[wv][d] += (unsigned int)__popcll(match);
    }
  }
  __syncthreads();
  unsigned int c = 0, incl = 0;
  if (tid < kXR) {  // digit tid: prefix over the waves, then over the digits
    for (int w = 0; w < kSW; ++w) {
      const unsigned int h = xs.off[w][tid];
      xs.off[w][tid] = c;
      c += h;
    }
    incl = wave_incl_add_u32(c);
    if (lane == 63) xs.wtot[wv] = incl;
    if (c == (unsigned int)n) xs.flag = 1;
  }
  __syncthreads();
  const bool uniform = xs.flag;
  __syncthreads();  // every thread has read the flag before the next pass clears it
  if (uniform) return false;
  if (tid < kXR) {
    unsigned int base = incl - c;
    for (int w = 0; w < wv; ++w) base += xs.wtot[w];
    for (int w = 0; w < kSW; ++w) xs.off[w][tid] += base;
  }
  __syncthreads();
  for (int i0 = w0; i0 < w1; i0 += 64 * kXU) {
    uint32_t kk[kXU];
#pragma unroll
    for (int u = 0; u < kXU; ++u) {
      const int i = i0 + 64 * u + lane;
      kk[u] = i < w1 ? src[i] : 0u;
    }
#pragma unroll
    for (int u = 0; u < kXU; ++u) {
      const bool valid = i0 + 64 * u + lane < w1;
      const uint32_t k = kk[u];
      const uint32_t d = (k >> shift) & (kXR - 1);
      const unsigned long long match = digit_match(d, valid);
      const unsigned int rank = (unsigned int)__popcll(match & ((1ull << lane) - 1ull));
      const unsigned int base = xs.off[wv][d];
      if (valid) {
        dst[base + rank] = k;
        if ((match >> lane) == 1ull) xs.off[wv][d] = base + rank + 1u;
      }
    }
  }
  __syncthreads();
  return true;
}

// Sorts the keys in a[0, n) ascending by their low `bits` bits (the others
// are zero); b is scratch of n keys.  Returns the array holding the result.
__device__ __forceinline__ uint32_t* radix_sort(ExactSmem& xs, uint32_t* a, uint32_t* b, int n, int bits) {
  for (int shift = 0; shift < bits; shift += kXBits) {
    if (radix_pass(xs, a, b, n, shift)) {
      uint32_t* t = a;
      a = b;
      b = t;
    }
  }
  return a;
}

// In binade e (sums s in [2^e, 2^(e+1)), spacing u = 2^(e-23)), adding v >= 0
// to s = n u gives (n + a + rnd) u, or for a tie (v / u = a + 1/2 exactly)
// the even one of (n + a) u and (n + a + 1) u, while the result stays below
// 2^(e+1).  a is capped at kDeltaCap (such a step always leaves the binade).
__device__ __forceinline__ void split_at(float v, int e, int& a, int& rnd, bool& tie) {
  const uint32_t b = __float_as_uint(v);
  const int E = (int)((b >> 23) & 255u);
  const uint32_t mant = E ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
  const int k = (E ? E - 150 : -149) - e + 23;  // v / u = mant * 2^k
  // k >= 0: a = mant 2^k (capped); k < 0: a = mant >> -k, the bits shifted
  // out deciding the rounding.  Selects, no branches: a shift of 31 leaves
  // a = 0 and a remainder below half for every 24-bit mant, as any k < -25
  // (v < u / 4) must.
  const int sh = min(max(-k, 1), 31);
  const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1);
  const uint32_t up = k >= 7 ? (uint32_t)kDeltaCap : min(mant << max(k, 0), (uint32_t)kDeltaCap);
  a = (int)(k >= 0 ? up : mant >> sh);
  rnd = k < 0 && rem > half;
  tie = k < 0 && rem == half;
}

// (d0, d1) then (b0, b1): the deltas of two consecutive runs composed, for
// an even / odd start (the second run starts at the parity the first left).
__device__ __forceinline__ void compose(int& d0, int& d1, int b0, int b1) {
  const int n0 = d0 + ((d0 & 1) ? b1 : b0);
  const int n1 = d1 + ((d1 & 1) ? b0 : b1);
  d0 = min(n0, kDeltaCap);
  d1 = min(n1, kDeltaCap);
}

// The earlier partial of a scan step: lane i gets lane i's source under DPP
// control CTRL (rows outside ROW_MASK, and lanes without a source, get
// (0, 0), the identity of compose).
template <int CTRL, int ROW_MASK = 0xf>
__device__ __forceinline__ void dpp_compose(int& a0, int& a1) {
  int b0 = __builtin_amdgcn_update_dpp(0, a0, CTRL, ROW_MASK, 0xf, false);
  int b1 = __builtin_amdgcn_update_dpp(0, a1, CTRL, ROW_MASK, 0xf, false);
  compose(b0, b1, a0, a1);
  a0 = b0;
  a1 = b1;
}

// Inclusive composition scan across the wave in lane order: lane i ends with
// the deltas of lanes 0 .. i composed, earlier first.  Row shifts within the
// 16-lane rows, then the row broadcasts of the lane-15 and lane-31 partials
// (VALU data movement, no LDS round trips).
__device__ __forceinline__ void compose_scan(int& a0, int& a1) {
  dpp_compose<0x111>(a0, a1);        // row_shr:1
  dpp_compose<0x112>(a0, a1);        // row_shr:2
  dpp_compose<0x114>(a0, a1);        // row_shr:4
  dpp_compose<0x118>(a0, a1);        // row_shr:8
  dpp_compose<0x142, 0xa>(a0, a1);   // row_bcast:15 into rows 1 and 3
  dpp_compose<0x143, 0xc>(a0, a1);   // row_bcast:31 into rows 2 and 3
}

// The f32 running sum s_{i+1} = fl(s_i + v_i), s_0 = 0, over v[0, len) (in
// global memory, written before the call), up to and including the first i
// with s_{i+1} >= thr (use_thr).  Result in xs.s (the sum reached) and
// xs.pos (elements taken: that i + 1, or len).
//
// While the sum stays in one binade e, every step is an integer addition in
// units of u = 2^(e-23) (split_at), so a run of steps is the sum of their
// increments -- except at exact ties, where round-half-even makes the step
// depend on the parity of the running count; a run is therefore described
// by two deltas, one per start parity, and such deltas compose.  The
// sequence is cut into chunks of C consecutive elements (C a multiple of
// 64, at most kRunChunks chunks), each handled by one wave with coalesced
// loads: a first sweep sums the chunks (float, only for guesses), a scan
// gives each chunk a guess of the binade its running sum starts in, and a
// second sweep computes the chunk's deltas for that binade (a wave sum of
// the increments per 64 elements; a composition scan across the lanes when
// the 64 hold a tie).  Wave 0 then walks the chunks in order, applying runs
// of chunks whose guess matches the actual sum by a composition scan across
// lanes, provided the result stays in the binade and below thr; any other
// chunk (the first, a wrong guess, a binade crossing or the threshold inside
// it, a value that is not finite) is walked element by element with real
// f32 additions.  The guesses only decide the speed: every delta used is
// checked against the actual running sum.  Call from all threads; ends with
// a barrier.
__device__ __forceinline__ void f32_run(ExactSmem& xs, const float* v, int len, bool use_thr, float thr) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int C = max(64, ((len + kRunChunks - 1) / kRunChunks + 63) / 64 * 64);
  const int nch = (len + C - 1) / C;
  // Wave w owns the contiguous chunks [cw0, cw1) and streams them kXU
  // batches of 64 at a time; batch b of the range belongs to chunk
  // cw0 + b / (C / 64).
  const int cpw = (nch + kSW - 1) / kSW;
  const int cw0 = min(nch, wv * cpw), cw1 = min(nch, cw0 + cpw);
  const int bpc = C / 64;  // batches per chunk
  const int nb = (cw1 - cw0) * bpc;
  // sweep 1: chunk sums (-1: the chunk holds a value that is not finite)
  {
    float acc = 0.0f;
    bool fin = true;
    for (int b0 = 0; b0 < nb; b0 += kXU) {
      float xv[kXU];
#pragma unroll
      for (int u = 0; u < kXU; ++u) {
        const int i = cw0 * C + (b0 + u) * 64 + lane;
        xv[u] = b0 + u < nb && i < len ? v[i] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kXU; ++u) {
        if (b0 + u >= nb) break;  // uniform
        fin &= xv[u] >= 0.0f && xv[u] <= 3.402823466e38f;
        acc += xv[u];
        if ((b0 + u + 1) % bpc == 0) {  // the chunk's last batch
          const float t = wsum_f32(acc);
          if (lane == 0) xs.csum[cw0 + (b0 + u) / bpc] = __ballot(!fin) ? -1.0f : t;
          acc = 0.0f;
          fin = true;
        }
      }
    }
  }
  __syncthreads();
  // exclusive prefix over the chunks (a non-finite chunk poisons the rest:
  // their guesses become -1, i.e. no delta)
  {
    const int c0 = 2 * tid;
    const float x0 = c0 < nch ? xs.csum[c0] : 0.0f, x1 = c0 + 1 < nch ? xs.csum[c0 + 1] : 0.0f;
    const float mine = (x0 < 0.0f || x1 < 0.0f) ? -INFINITY : x0 + x1;
    const float in = wave_incl_add_f32(mine);
    if (lane == 63) xs.wsum[wv] = in;
    __syncthreads();
    float pre = in - mine;
    for (int w = 0; w < wv; ++w) pre += xs.wsum[w];
    if (!(mine > -INFINITY)) pre = -INFINITY;
    if (c0 < nch) xs.csum[c0] = pre;
    if (c0 + 1 < nch) xs.csum[c0 + 1] = x0 < 0.0f ? -INFINITY : pre + x0;
    __syncthreads();
  }
  // sweep 2: each chunk's deltas for its guessed binade (chunks past the
  // threshold, by a margin far above any f32 drift, are never reached
  // before the walk stops: no delta)
  {
    int e = kNoDelta, d0 = 0, d1 = 0;
    for (int b0 = 0; b0 < nb; b0 += kXU) {
      float xv[kXU];
#pragma unroll
      for (int u = 0; u < kXU; ++u) {
        const int i = cw0 * C + (b0 + u) * 64 + lane;
        xv[u] = b0 + u < nb && i < len ? v[i] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kXU; ++u) {
        const int b = b0 + u;
        if (b >= nb) break;  // uniform
        const int c = cw0 + b / bpc;
        if (b % bpc == 0) {  // the chunk's first batch: its guess
          const float pre = xs.csum[c];
          e = pre > 0.0f && pre < 3.402823466e38f && !(use_thr && pre > thr * 1.0625f)
                  ? (int)((__float_as_uint(pre) >> 23) & 255u) - 127
                  : kNoDelta;
          d0 = d1 = 0;
        }
        if (e != kNoDelta && d0 < kDeltaCap && d1 < kDeltaCap) {
          int a, rnd;
          bool tie;
          split_at(xv[u], e, a, rnd, tie);
          int q0, q1;
          if (!__ballot(tie)) {
            q0 = q1 = min(wsum_i32(a + rnd), kDeltaCap);  // 64 (2^24 + 2) < 2^31
          } else {  // composition scan across the lanes: lane 63 holds the batch
            int p0 = tie ? a + (a & 1) : a + rnd;
            int p1 = tie ? a + ((a + 1) & 1) : a + rnd;
            compose_scan(p0, p1);
            q0 = readlane_i(p0, 63);
            q1 = readlane_i(p1, 63);
          }
          compose(d0, d1, q0, q1);
        }
        if ((b + 1) % bpc == 0 && lane == 0) {  // the chunk's last batch
          xs.ce[c] = (d0 >= kDeltaCap || d1 >= kDeltaCap) ? kNoDelta : e;
          xs.cd0[c] = d0;
          xs.cd1[c] = d1;
        }
      }
    }
  }
  __syncthreads();

  if (wv == 0) {
    float s = 0.0f;
    int pos = len;
    bool done = false;
    // element-by-element walk of chunk c (wave-uniform)
    auto walk = [&](int c) {
      const int clo = c * C, chi = min(len, clo + C);
      for (int i0 = clo; i0 < chi && !done; i0 += 64) {
        const float x = i0 + lane < chi ? v[i0 + lane] : 0.0f;
        const int m = min(64, chi - i0);
        for (int j = 0; j < m; ++j) {
          s = s + readlane_f(x, j);
          if (use_thr && s >= thr) {
            pos = i0 + j + 1;
            done = true;
            break;
          }
        }
      }
    };
    for (int g = 0; g < nch && !done; g += 64) {
      const bool have = g + lane < nch;
      const int ec = have ? xs.ce[g + lane] : kNoDelta;
      const int c0 = have ? xs.cd0[g + lane] : 0, c1 = have ? xs.cd1[g + lane] : 0;
      const int gend = min(64, nch - g);
      int start = 0;
      while (start < gend && !done) {
        const uint32_t sb = __float_as_uint(s);
        const int sE = (int)((sb >> 23) & 255u);
        const bool s_normal = sE >= 1 && sE <= 254 && !(sb >> 31);
        const int es = sE - 127;
        const unsigned long long rm = __ballot(s_normal && lane >= start && ec == es) >> start;
        const int run = ~rm ? __builtin_ctzll(~rm) : 64;
        if (run == 0) {
          walk(g + start);
          ++start;
          continue;
        }
        // composed deltas of chunks start .. lane (identity outside the run)
        const bool in = lane >= start && lane < start + run;
        int a0 = in ? c0 : 0, a1 = in ? c1 : 0;
        compose_scan(a0, a1);
        const int n = (int)((sb & 0x7fffffu) | 0x800000u);
        const long long nend = (long long)n + ((n & 1) ? a1 : a0);
        const float send = nend < (1ll << 24) ? ldexpf((float)nend, es - 23) : INFINITY;
        const unsigned long long bad =
            __ballot(in && (nend >= (1ll << 24) || (use_thr && send >= thr)));
        if (!bad) {
          s = readlane_f(send, start + run - 1);
          start += run;
          continue;
        }
        const int l = __builtin_ctzll(bad);
        if (l > start) s = readlane_f(send, l - 1);
        walk(g + l);
        start = l + 1;
      }
    }
    if (lane == 0) {
      xs.s = s;
      xs.pos = pos;
    }
  }
  __syncthreads();
}

// Sort key of a logit for the exact path (the logit negated when T < 0, so
// that larger keys give larger y = x / T): larger value -> larger key, -0
// and +0 equal; 16 significant bits for 16-bit logits.
template <int DT>
__device__ __forceinline__ uint32_t xkey(float x) {
  if constexpr (DT == PKV_F32) {
    return order_key(x);
  } else {
    uint32_t b = DT == PKV_BF16 ? (__float_as_uint(x) >> 16)
                                : (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x);
    if ((b & 0x7fffu) == 0u) b = 0u;
    return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
  }
}
template <int DT>
__device__ __forceinline__ float xkey_value(uint32_t k) {
  if constexpr (DT == PKV_F32) {
    return key_value(k);
  } else {
    const uint32_t b = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
    return DT == PKV_BF16 ? __uint_as_float(b << 16)
                          : (float)__builtin_bit_cast(_Float16, (uint16_t)b);
  }
}

struct ExactArgs {
  const char* logits;
  long long stride_bytes;
  int vocab;
  const float* temps;
  int top_k;         // 0: None
  float top_p;       // NaN: None
  float r;
  int32_t* tokens;
  uint32_t* scratch;  // 2 * vocab keys per row of the launch
  int row0;           // first row of this launch
  // f32 logits: per row, 0 once a kernel has selected its token, 1 while it
  // is left to the next kernel (buckets, then runs of equal values, then the
  // sort); null: the exact kernel samples every row
  int32_t* fallback;
  int32_t* route;  // optional, per row: the kernel that selected it (kRoute*)
};

// Which kernel selected a row's token (pkv_sample_exact_routes).
constexpr int32_t kRouteArgmax = 0, kRouteBuckets = 1, kRouteRuns = 2, kRouteSort = 3;

template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) sample_exact_kernel(ExactArgs a) {
  __shared__ SampleSmem sm;
  __shared__ ExactSmem xs;
  const int row = a.row0 + blockIdx.x;
  const int tid = threadIdx.x;
  if (a.fallback && a.fallback[row] == 0) return;  // selected by an earlier kernel
  const char* x = a.logits + (long long)row * a.stride_bytes;
  const int V = a.vocab;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || V <= 1) {  // sample.rs:13-15
    float bv;
    int bi;
    block_argmax<DT, VEC>(sm, x, 0, V, bv, bi);
    if (tid == 0) {
      a.tokens[row] = bi == INT_MAX ? 0 : bi;
      if (a.route) a.route[row] = kRouteArgmax;
    }
    return;
  }
  uint32_t* ka = a.scratch + (size_t)blockIdx.x * 2 * (size_t)V;
  uint32_t* kb = ka + V;
  // The logits sorted descending (ascending complemented keys; negated for
  // T < 0).  y = fl(x / T) is monotone in x, so the sorted logits give the
  // reference's sequence of y values (equal y adjacent), and only the values
  // enter the sums; no division is needed to sort.
  constexpr int kBits = DT == PKV_F32 ? 32 : 16;
  constexpr uint32_t kMask = DT == PKV_F32 ? 0xffffffffu : 0xffffu;
  const bool neg = T < 0.0f;
  for_each<DT, VEC, kRowBatch>(x, V, [&](int i, float v) { ka[i] = kMask & ~xkey<DT>(neg ? -v : v); });
  __syncthreads();
  const uint32_t* sk = radix_sort(xs, ka, kb, V, kBits);
  float* p = reinterpret_cast<float*>(sk == ka ? kb : ka);
  auto y_at = [&](int i) {
    const float xp = xkey_value<DT>(kMask & ~sk[i]);
    return (neg ? -xp : xp) / T;
  };

  int len = a.top_k > 0 && a.top_k < V ? a.top_k : V;  // probs.truncate(k)
  const float max_x = y_at(0);
  for (int i0 = tid; i0 < len; i0 += kXU * kST) {
    uint32_t kk[kXU];
#pragma unroll
    for (int u = 0; u < kXU; ++u) kk[u] = i0 + u * kST < len ? sk[i0 + u * kST] : 0u;
#pragma unroll
    for (int u = 0; u < kXU; ++u) {
      if (i0 + u * kST >= len) break;
      const float xp = xkey_value<DT>(kMask & ~kk[u]);
      p[i0 + u * kST] = expf_glibc((neg ? -xp : xp) / T - max_x);
    }
  }
  __syncthreads();
  f32_run(xs, p, len, false, 0.0f);  // sum += p
  // p /= divisor over [0, n), kXU loads in flight per thread
  auto divide = [&](int n, float divisor) {
    for (int i0 = tid; i0 < n; i0 += kXU * kST) {
      float pv[kXU];
#pragma unroll
      for (int u = 0; u < kXU; ++u) pv[u] = i0 + u * kST < n ? p[i0 + u * kST] : 0.0f;
#pragma unroll
      for (int u = 0; u < kXU; ++u)
        if (i0 + u * kST < n) p[i0 + u * kST] = pv[u] / divisor;
    }
    __syncthreads();
  };
  divide(len, xs.s);
  if (a.top_p == a.top_p) {  // Some(top_p)
    f32_run(xs, p, len, true, a.top_p);
    len = xs.pos;     // cutoff
    divide(len, xs.s);  // xs.s equals the f32 sum of the kept probabilities
  }
  f32_run(xs, p, len, true, a.r);  // acc += prob until r <= acc
  const int j = xs.pos - 1;  // xs.pos = len when acc never reaches r: probs.last()
  // the token at sorted position j: the first sorted position of its y,
  // then that many tokens further among the equal ones, in index order
  const uint32_t kj = order_key(y_at(j));
  int lo = 0, hi = j;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (order_key(y_at(mid)) > kj) lo = mid + 1;
    else hi = mid;
  }
  Row<DT, VEC> rw{x, V, T, 0.0f, false, 0u, V};
  const int tok = nth_tied<false>(sm, rw, kj, (unsigned long long)(j - lo + 1));
  if (tid == 0) {
    a.tokens[row] = tok;
    if (a.route) a.route[row] = kRouteSort;
  }
}

// ---- 16-bit logits: the sorted sequence as runs of equal values -------------
// A 16-bit logit takes one of 65,536 values, so the descending sequence the
// reference sorts is, without sorting, the list of distinct values (an LDS
// histogram of the 16-bit sort keys, read from the largest key down), each
// repeated as often as it occurs: a run.  Everything after the sort is a
// function of that sequence: the maximum, p = exp(y - max) once per run, and
// the f32 running sums, where c copies of one value added while the sum stays
// in one binade are c equal integer steps (for a tie, a first step that
// depends on the parity of the running count, then c - 1 equal even steps),
// so a run has closed-form deltas (run_delta) and its binade crossings and
// its threshold crossing are found by arithmetic (run_step).  f32_runs walks
// runs as f32_run walks elements.  A bf16 row of N(0, 9) logits has ~3k
// runs for 128k logits.

constexpr int kHalfKeys = 32768;  // histogram: one half of the 16-bit key space per pass
constexpr int kMaxRuns = 65536;

struct RunSmem {
  float csum[kRunChunks];  // chunk sums, then exclusive prefixes (guesses)
  int ce[kRunChunks];      // binade the chunk's delta assumes (kNoDelta: none)
  int cd0[kRunChunks], cd1[kRunChunks];
  float wsum[kSW];
  float s;    // f32_runs result: the sum reached,
  int r_end;  //   the run where the threshold stopped it (R: not reached)
  int k_end;  //   and how many copies of that run it took
  int R;
};
// Rows of at most kLdsRuns runs keep their runs in LDS after the histogram
// (the running-sum walks read them one at a time, in order).
constexpr int kLdsRuns = 4096;

union RunLds {
  unsigned int hist[kHalfKeys];
  struct {
    SampleSmem sm;
    RunSmem rs;
    uint32_t key[kLdsRuns], cnt[kLdsRuns], start[kLdsRuns];
    float val[kLdsRuns];
  } x;
};

// A row's runs in descending order of value (global scratch, kMaxRuns each).
struct RunArrays {
  uint32_t* key;    // 16-bit order key of the (sign-adjusted) logit
  uint32_t* cnt;    // copies
  uint32_t* start;  // position of the first copy in the sorted sequence
  float* val;       // what the current running sum adds per copy
};

// Exclusive prefix of one value per thread over the workgroup; wtmp: kSW
// scratch words outside any buffer the caller is using.  Ends with a barrier.
__device__ __forceinline__ unsigned int block_excl_scan(unsigned int v, unsigned int* wtmp,
                                                        unsigned int& total) {
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const unsigned int in = wave_incl_add_u32(v);
  if (lane == 63) wtmp[wv] = in;
  __syncthreads();
  unsigned int pre = in - v;
  total = 0;
  for (int w = 0; w < kSW; ++w) {
    const unsigned int t = wtmp[w];
    if (w < wv) pre += t;
    total += t;
  }
  __syncthreads();
  return pre;
}

// Exclusive prefix of the chunk sums csum[0, nch) (nch <= 2 kST), in place;
// a negative entry (a chunk that is not finite) makes every later prefix
// -inf (no guess).  Ends with a barrier.
__device__ __forceinline__ void chunk_prefix(float* csum, float* wsum, int nch) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int c0 = 2 * tid;
  const float x0 = c0 < nch ? csum[c0] : 0.0f, x1 = c0 + 1 < nch ? csum[c0 + 1] : 0.0f;
  const float mine = (x0 < 0.0f || x1 < 0.0f) ? -INFINITY : x0 + x1;
  const float in = wave_incl_add_f32(mine);
  if (lane == 63) wsum[wv] = in;
  __syncthreads();
  float pre = in - mine;
  for (int w = 0; w < wv; ++w) pre += wsum[w];
  if (!(mine > -INFINITY)) pre = -INFINITY;
  if (c0 < nch) csum[c0] = pre;
  if (c0 + 1 < nch) csum[c0 + 1] = x0 < 0.0f ? -INFINITY : pre + x0;
  __syncthreads();
}

// Deltas (even / odd start, units of 2^(e-23)) of c >= 1 copies of v added
// in binade e; kDeltaCap when they leave it.  A tie's first copy rounds the
// count to even, after which every copy adds the even a + (a & 1).
__device__ __forceinline__ void run_delta(float v, unsigned int c, int e, int& d0, int& d1) {
  int a, rnd;
  bool tie;
  split_at(v, e, a, rnd, tie);
  long long x0, x1;
  if (!tie) {
    x0 = x1 = (long long)c * (a + rnd);
  } else {
    const long long rest = (long long)(c - 1u) * (a + (a & 1));
    x0 = a + (a & 1) + rest;
    x1 = a + ((a + 1) & 1) + rest;
  }
  d0 = x0 >= kDeltaCap ? kDeltaCap : (int)x0;
  d1 = x1 >= kDeltaCap ? kDeltaCap : (int)x1;
}

// Adds c copies of v to s with f32 semantics, a binade at a time, stopping
// after the first copy that brings s to thr or beyond (use_thr; s < thr on
// entry).  Returns the copies taken; *hit whether it stopped.  Uniform
// arguments give uniform results (no lane exchange).
__device__ __forceinline__ unsigned int run_step(float& s, float v, unsigned int c, bool use_thr,
                                                 float thr, bool& hit) {
  unsigned int k = 0;
  hit = false;
  while (k < c) {
    const uint32_t sb = __float_as_uint(s);
    const int sE = (int)((sb >> 23) & 255u);
    if (!(sE >= 1 && sE <= 254 && !(sb >> 31)) || !(v >= 0.0f && v <= 3.402823466e38f)) {
      // zero, subnormal, inf or NaN involved: one real addition
      s = s + v;
      ++k;
      if (use_thr && s >= thr) {
        hit = true;
        return k;
      }
      if (s != s) return c;  // NaN: every later sum is NaN and below nothing
      continue;
    }
    const int e = sE - 127;
    long long n = (long long)((sb & 0x7fffffu) | 0x800000u);
    int a, rnd;
    bool tie;
    split_at(v, e, a, rnd, tie);
    long long q = a + rnd;
    if (tie) {
      const long long n1 = n + a + ((n + a) & 1);
      ++k;
      if (n1 >= (1ll << 24)) {
        s = s + v;  // leaves the binade: the real addition
      } else {
        n = n1;
        s = ldexpf((float)n, e - 23);
      }
      if (use_thr && s >= thr) {
        hit = true;
        return k;
      }
      if (n1 >= (1ll << 24) || k >= c) continue;
      q = a + (a & 1);
    }
    if (q == 0) return c;  // the remaining copies change nothing
    long long take = min((long long)(c - k), ((1ll << 24) - 1 - n) / q);
    if (use_thr) {
      // the first copy j with (n + j q) 2^(e-23) >= thr, i.e. n + j q >= ceil(thr / u)
      const long long need =
          max((long long)ceil(ldexp((double)thr, 23 - e)) - n, 1ll);
      const long long j = (need + q - 1) / q;
      if (j <= take) {
        n += j * q;
        k += (unsigned int)j;
        s = ldexpf((float)n, e - 23);
        hit = true;
        return k;
      }
    }
    n += take * q;
    k += (unsigned int)take;
    s = ldexpf((float)n, e - 23);
    if (k < c) {  // the next copy leaves the binade: the real addition
      s = s + v;
      ++k;
      if (use_thr && s >= thr) {
        hit = true;
        return k;
      }
    }
  }
  return c;
}

// The f32 running sum over runs [0, R) of ra (cnt[r] copies of val[r]), the
// way f32_run takes elements: chunks of G consecutive runs (at most
// kRunChunks chunks), a guessed binade per chunk from float prefix sums,
// composed closed-form deltas per chunk, and wave 0 walking the chunks,
// applying runs of chunks whose guess matches the actual sum and stepping
// any other chunk run by run (run_step).  Results in rs.s, rs.r_end and
// rs.k_end.  Call from all threads; ends with a barrier.
__device__ __forceinline__ void f32_runs(RunSmem& rs, const RunArrays& ra, int R, bool use_thr,
                                         float thr) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int G = max(1, (R + kRunChunks - 1) / kRunChunks);
  const int nch = (R + G - 1) / G;
  for (int c = tid; c < nch; c += kST) {
    float acc = 0.0f;
    bool fin = true;
    for (int r = c * G; r < min(R, (c + 1) * G); ++r) {
      const float v = ra.val[r];
      fin &= v >= 0.0f && v <= 3.402823466e38f;
      acc += v * (float)ra.cnt[r];
    }
    rs.csum[c] = fin ? acc : -1.0f;
  }
  __syncthreads();
  chunk_prefix(rs.csum, rs.wsum, nch);
  for (int c = tid; c < nch; c += kST) {
    const float pre = rs.csum[c];
    int e = kNoDelta, d0 = 0, d1 = 0;
    if (pre > 0.0f && pre < 3.402823466e38f && !(use_thr && pre > thr * 1.0625f)) {
      e = (int)((__float_as_uint(pre) >> 23) & 255u) - 127;
      for (int r = c * G; r < min(R, (c + 1) * G) && d0 < kDeltaCap && d1 < kDeltaCap; ++r) {
        int b0, b1;
        run_delta(ra.val[r], ra.cnt[r], e, b0, b1);
        compose(d0, d1, b0, b1);
      }
      if (d0 >= kDeltaCap || d1 >= kDeltaCap) e = kNoDelta;
    }
    rs.ce[c] = e;
    rs.cd0[c] = d0;
    rs.cd1[c] = d1;
  }
  __syncthreads();

  if (wv == 0) {
    float s = 0.0f;
    int r_end = R, k_end = 0;
    bool done = false;
    auto walk = [&](int c) {  // chunk c run by run (wave-uniform)
      for (int r = c * G; r < min(R, (c + 1) * G) && !done; ++r) {
        bool hit;
        const unsigned int k = run_step(s, ra.val[r], ra.cnt[r], use_thr, thr, hit);
        if (hit) {
          done = true;
          r_end = r;
          k_end = (int)k;
        }
      }
    };
    for (int g = 0; g < nch && !done; g += 64) {
      const bool have = g + lane < nch;
      const int ec = have ? rs.ce[g + lane] : kNoDelta;
      const int c0 = have ? rs.cd0[g + lane] : 0, c1 = have ? rs.cd1[g + lane] : 0;
      const int gend = min(64, nch - g);
      int start = 0;
      while (start < gend && !done) {
        const uint32_t sb = __float_as_uint(s);
        const int sE = (int)((sb >> 23) & 255u);
        const bool s_normal = sE >= 1 && sE <= 254 && !(sb >> 31);
        const int es = sE - 127;
        const unsigned long long rm = __ballot(s_normal && lane >= start && ec == es) >> start;
        const int run = ~rm ? __builtin_ctzll(~rm) : 64;
        if (run == 0) {
          walk(g + start);
          ++start;
          continue;
        }
        const bool in = lane >= start && lane < start + run;
        int a0 = in ? c0 : 0, a1 = in ? c1 : 0;
        compose_scan(a0, a1);
        const int n = (int)((sb & 0x7fffffu) | 0x800000u);
        const long long nend = (long long)n + ((n & 1) ? a1 : a0);
        const float send = nend < (1ll << 24) ? ldexpf((float)nend, es - 23) : INFINITY;
        const unsigned long long bad =
            __ballot(in && (nend >= (1ll << 24) || (use_thr && send >= thr)));
        if (!bad) {
          s = readlane_f(send, start + run - 1);
          start += run;
          continue;
        }
        const int l = __builtin_ctzll(bad);
        if (l > start) s = readlane_f(send, l - 1);
        walk(g + l);
        start = l + 1;
      }
    }
    if (lane == 0) {
      rs.s = s;
      rs.r_end = r_end;
      rs.k_end = k_end;
    }
  }
  __syncthreads();
}

// sample_exact_kernel for 16-bit logits, on runs instead of a sorted copy.
// Scratch: 4 kMaxRuns words per row (keys, counts, starts, values).
template <int DT, bool VEC>
__global__ void __launch_bounds__(kST) sample_runs_kernel(ExactArgs a) {
  // Keys are 16-bit: of the logits themselves, or for f32 logits of their
  // bf16 value, which is the logit itself when its low 16 bits are zero (f32
  // logits of a bf16 model); a row with any other f32 logit is left to
  // sample_exact_kernel (a.fallback).
  constexpr int KT = DT == PKV_F32 ? PKV_BF16 : DT;
  __shared__ RunLds u;
  __shared__ unsigned int wtmp[kSW];
  SampleSmem& sm = u.x.sm;
  RunSmem& rs = u.x.rs;
  const int row = a.row0 + blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63;
  if (a.fallback && a.fallback[row] == 0) return;  // selected by sample_bucket_kernel
  const char* x = a.logits + (long long)row * a.stride_bytes;
  const int V = a.vocab;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || V <= 1) {  // sample.rs:13-15
    float bv;
    int bi;
    block_argmax<DT, VEC>(sm, x, 0, V, bv, bi);
    if (tid == 0) {
      a.tokens[row] = bi == INT_MAX ? 0 : bi;
      if (a.fallback) a.fallback[row] = 0;
      if (a.route) a.route[row] = kRouteArgmax;
    }
    return;
  }
  uint32_t* base = a.scratch + (size_t)blockIdx.x * 4 * kMaxRuns;
  RunArrays ra{base, base + kMaxRuns, base + 2 * kMaxRuns,
               reinterpret_cast<float*>(base + 3 * kMaxRuns)};
  const bool neg = T < 0.0f;

  // runs: one histogram of all 65,536 keys as 16-bit counts, two per LDS
  // word; a count past 65,535 would carry into its neighbour (or out of the
  // word), which only lowers the counts' total, so a total below V sends the
  // row to the two-pass 32-bit histogram below (a value held by more than
  // 65,535 logits).
  int R = 0;
  bool two_pass = false;
  {
    for (int b = tid; b < kHalfKeys; b += kST) u.hist[b] = 0u;
    __syncthreads();
    bool inexact = false;
    for_each<DT, VEC, kRowBatch>(x, V, [&](int, float v) {
      if constexpr (DT == PKV_F32) inexact |= (__float_as_uint(v) & 0xffffu) != 0u;
      const uint32_t k = xkey<KT>(neg ? -v : v);
      const unsigned long long act = __ballot(true);
      const uint32_t k0 = __builtin_amdgcn_readfirstlane(k);
      const uint32_t sh = (k & 1u) * 16u;
      if (__ballot(k == k0) == act) {  // one key across the wave: one addition
        if (lane == __builtin_ctzll(act)) atomicAdd(&u.hist[k >> 1], (unsigned)__popcll(act) << sh);
      } else {
        atomicAdd(&u.hist[k >> 1], 1u << sh);
      }
    });
    if constexpr (DT == PKV_F32) {
      const bool leave = __syncthreads_or(inexact);
      if (tid == 0) a.fallback[row] = leave ? 1 : 0;
      if (leave) return;  // uniform: the row needs the f32 sort
    } else {
      __syncthreads();
    }
    const int whi = kHalfKeys - 1 - 32 * tid;  // this thread's 32 words (64 keys), descending
    unsigned int nz = 0, sum = 0;
    for (int j = 0; j < 32; ++j) {
      const unsigned int w = u.hist[whi - j];
      nz += (w >> 16 != 0u) + ((w & 0xffffu) != 0u);
      sum += (w >> 16) + (w & 0xffffu);
    }
    unsigned int total, counted;
    unsigned int at = block_excl_scan(nz, wtmp, total);
    block_excl_scan(sum, wtmp, counted);
    if (counted == (unsigned int)V) {
      for (int j = 0; j < 32; ++j) {
        const unsigned int w = u.hist[whi - j];
        const uint32_t kh = 2u * (uint32_t)(whi - j) + 1u;
        if (w >> 16) {
          ra.key[at] = kh;
          ra.cnt[at] = w >> 16;
          ++at;
        }
        if (w & 0xffffu) {
          ra.key[at] = kh - 1u;
          ra.cnt[at] = w & 0xffffu;
          ++at;
        }
      }
      R = (int)total;
    }
    two_pass = counted != (unsigned int)V;
    __syncthreads();  // every thread has read the histogram before it is cleared or reused
  }
  for (int half = 1; half >= 0 && two_pass; --half) {
    for (int b = tid; b < kHalfKeys; b += kST) u.hist[b] = 0u;
    __syncthreads();
    for_each<DT, VEC, kRowBatch>(x, V, [&](int, float v) {
      const uint32_t k = xkey<KT>(neg ? -v : v);
      const bool mine = (int)(k >> 15) == half;
      const unsigned long long act = __ballot(true);
      const uint32_t k0 = __builtin_amdgcn_readfirstlane(k);
      if (__ballot(k == k0) == act) {  // one key across the wave: one addition
        if (mine && lane == __builtin_ctzll(act)) atomicAdd(&u.hist[k & 0x7fffu], (unsigned)__popcll(act));
      } else if (mine) {
        atomicAdd(&u.hist[k & 0x7fffu], 1u);
      }
    });
    __syncthreads();
    const int bhi = kHalfKeys - 1 - 32 * tid;  // this thread's 32 bins, descending
    unsigned int nz = 0;
    for (int j = 0; j < 32; ++j) nz += u.hist[bhi - j] != 0u;
    unsigned int total;
    unsigned int at = (unsigned int)R + block_excl_scan(nz, wtmp, total);
    for (int j = 0; j < 32; ++j) {
      const unsigned int h = u.hist[bhi - j];
      if (h) {
        ra.key[at] = ((uint32_t)half << 15) | (uint32_t)(bhi - j);
        ra.cnt[at] = h;
        ++at;
      }
    }
    R += (int)total;
    __syncthreads();  // every thread has read the histogram before it is cleared or reused
  }
  // start positions; top_k cuts the sequence at len (probs.truncate(k))
  {
    const int RP = (R + kST - 1) / kST;
    const int r0 = min(R, tid * RP), r1 = min(R, r0 + RP);
    unsigned int sum = 0;
    for (int r = r0; r < r1; ++r) sum += ra.cnt[r];
    unsigned int total;
    unsigned int st = block_excl_scan(sum, wtmp, total);
    const unsigned int len = a.top_k > 0 && a.top_k < V ? (unsigned int)a.top_k : (unsigned int)V;
    if (tid == 0) rs.R = R;
    __syncthreads();
    for (int r = r0; r < r1; ++r) {
      const unsigned int c = ra.cnt[r];
      ra.start[r] = st;
      if (st < len && len <= st + c) {
        ra.cnt[r] = len - st;
        rs.R = r + 1;
      }
      st += c;
    }
    __syncthreads();
    R = rs.R;
  }
  if (R <= kLdsRuns) {  // the runs move to LDS: the walks below read them one by one
    for (int r = tid; r < R; r += kST) {
      u.x.key[r] = ra.key[r];
      u.x.cnt[r] = ra.cnt[r];
      u.x.start[r] = ra.start[r];
    }
    __syncthreads();
    ra = RunArrays{u.x.key, u.x.cnt, u.x.start, u.x.val};
  }
  auto y_of = [&](int r) {
    const float xp = xkey_value<KT>(ra.key[r]);
    return (neg ? -xp : xp) / T;
  };
  const float max_x = y_of(0);
  for (int r = tid; r < R; r += kST) ra.val[r] = expf_glibc(y_of(r) - max_x);
  __syncthreads();
  f32_runs(rs, ra, R, false, 0.0f);  // sum += p
  const float sum = rs.s;
  for (int r = tid; r < R; r += kST) ra.val[r] = ra.val[r] / sum;
  __syncthreads();
  if (a.top_p == a.top_p) {  // Some(top_p): cut after the first copy reaching it
    f32_runs(rs, ra, R, true, a.top_p);
    const float s_top = rs.s;  // the f32 sum of the kept probabilities
    if (rs.r_end < R) {
      const int rc = rs.r_end, kc = rs.k_end;
      __syncthreads();
      if (tid == 0) ra.cnt[rc] = (uint32_t)kc;
      R = rc + 1;
    }
    for (int r = tid; r < R; r += kST) ra.val[r] = ra.val[r] / s_top;
    __syncthreads();
  }
  f32_runs(rs, ra, R, true, a.r);  // acc += prob until r <= acc
  int rj, j;
  if (rs.r_end < R) {
    rj = rs.r_end;
    j = (int)ra.start[rj] + rs.k_end - 1;
  } else {  // probs.last()
    rj = R - 1;
    j = (int)(ra.start[rj] + ra.cnt[rj]) - 1;
  }
  // the token at sorted position j: the first position of its y (runs of
  // different logits can share a y), then that many tokens further among
  // the equal ones, in index order
  const float yj = y_of(rj);
  const uint32_t kj = order_key(yj);
  int rf = rj;
  while (rf > 0 && order_key(y_of(rf - 1)) == kj) --rf;
  Row<DT, VEC> rw{x, V, T, 0.0f, false, 0u, V};
  const int tok = nth_tied<false>(sm, rw, kj, (unsigned long long)(j - (int)ra.start[rf] + 1));
  if (tid == 0) {
    a.tokens[row] = tok;
    if (a.route) a.route[row] = kRouteRuns;
  }
}

// ---- f32 logits: buckets of y instead of a sort -----------------------------
// Only the f32 running sums depend on the sorted order, and only in part.
// While a running sum stays inside one binade, each addition adds an integer
// number of units that depends on the added value alone (split_at), except
// at an exact tie, where round-half-even depends on the count so far; so a
// stretch of the sorted sequence that the sum crosses without leaving its
// binade, without a tie and without reaching a threshold adds the same total
// in any order.
//
// sample_bucket_kernel cuts y into kBk buckets by its distance below max y (a
// monotone function of y: each bucket is a contiguous stretch of the sorted
// sequence, and equal y share a bucket) and counts each bucket's logits and
// approximate mass (integers).  The mass prefix predicts the binade in which
// each running sum (the softmax denominator; top_p's; r's) enters each bucket.
// The keys of the buckets a sum must follow in order are stored and sorted:
// the top of the order (its first kRegionA logits, where large probabilities
// make ties common, kept in LDS with their values), the buckets where top_p
// or r is predicted to be reached (with a margin), and a top_k cut.  Every
// other bucket is only summed: its unit increments for the binade predicted
// for it.  A walk then follows each sum: stored stretches 64 sorted logits at
// a time (a composition scan of the two-parity deltas across the lanes, real
// f32 additions where the sum leaves its binade), other buckets as prefix
// sums of their increments -- checked against the actual sum.  Where the
// actual binade differs from the prediction, one more pass over the row sums
// the following buckets predicted alike again for the actual binade; where a
// bucket holds a tie, or the sum would leave its binade or reach its
// threshold inside it, one more pass stores its keys (and those of the next
// buckets), which are sorted and walked.
//
// Logits kDTail or more below max y have p = expf(y - max y) < 0.84 2^-25.
// Every sum such a p (or p / S, p / S / S2) meets is at least 1 (the
// softmax denominator starts with exp(0) = 1), resp. at least the first
// normalised probability, more than 2^25 times the added value: the addition
// is below half a unit, changes nothing and is never a tie.  These logits
// (most of a typical row) are counted but never stored, sorted or summed.
//
// A row is left to the later kernels (fallback stays 1) when it holds a NaN
// or max y is infinite, when a bucket to sort holds more than kBkSortMax
// logits, or when the running sum never reaches r (sample.rs then takes the
// last kept token).
constexpr int kBk = 4096;              // buckets of y per row (index kBk: the tail)
constexpr int kWaveSortMax = 256;      // largest bucket one wave sorts
constexpr int kBkSortMax = kSW * kWaveSortMax;  // largest bucket the workgroup sorts
constexpr int kRegionA = 4096;         // the top logits, always stored (in LDS)
constexpr int kGatherSpan = 4;         // buckets one extra pass gathers
constexpr float kDTail = 17.5f;        // y - max y <= -kDTail: the tail
constexpr float kMargin = 0x1p-6f;     // relative margin of the predictions
constexpr short kNoBinade = SHRT_MIN;  // no prediction
constexpr unsigned char kStored = 1, kSorted = 2, kGather = 4;
static_assert(kBk == 4 * kST, "four buckets per thread in the scans");

struct BucketSmem {
  unsigned int start[kBk + 2];    // first sorted position of bucket b; [kBk]: the tail's; [kBk+1]: V
  unsigned int cur[kBk + 1];      // logits per bucket, then store cursors
  float pm[kBk + 1];              // approximate mass before bucket b ([kBk]: the total)
  unsigned long long inc[kBk];    // fixed-point mass; then unit increments (bit 63: walk it)
  short eg[kBk];                  // predicted binade of the running sum entering the bucket
  unsigned char flag[kBk];        // kStored, kSorted, kGather
  uint32_t stage[kSW][kWaveSortMax];  // keys being sorted: per wave, or all for one big bucket
  uint32_t topk[kRegionA];        // the keys of the top of the order, sorted,
  uint32_t topi[kRegionA];        //   their logits' indices,
  float topv[kRegionA];           //   and what they add to the current sum
  float ch_sum[kRegionA / 64];    // chunks of 64 of the top: sums (estimates),
  int ch_e[kRegionA / 64];        //   the binade predicted at their start,
  int ch_d0[kRegionA / 64], ch_d1[kRegionA / 64];  // their deltas in it (even / odd start)
  unsigned long long exptab[32];   // kExp2Tab
  unsigned long long wu[kSW];
  unsigned int wtmp[kSW];
  float wf[kSW], wg[kSW];
  int wi[kSW];
  float s;                        // walk: the running sum,
  int b, todo, why, pos, big;     //   next bucket, bucket to see to and why, position reached
  int tok;                        // the token found
};
union BucketLds {
  SampleSmem sm;
  BucketSmem bs;
};

// What a logit adds to a running sum: p = expf(y - max y) (divs 0), p / S
// (1) or (p / S) / S2 (2), each division rounded as the reference's, from
// t = y - max y or from the stored key of x' (y = x' / |T|).
struct BucketValue {
  float aT, ymax, S, S2;
  int divs;
  const unsigned long long* tab;  // kExp2Tab's copy in LDS
  // (t > -kDTail: expf's main path)
  __device__ __forceinline__ float of_t(float t) const {
    float v = expf_glibc_main(t, tab);
    if (divs >= 1) v = v / S;
    if (divs >= 2) v = v / S2;
    return v;
  }
  __device__ __forceinline__ float operator()(uint32_t k) const {
    return of_t(key_value(k) / aT - ymax);
  }
  // an estimate of of_t within 1.3e-6 (relative; see quick_inc)
  __device__ __forceinline__ float approx(float t) const {
    return divs == 0 ? __expf(t) : __expf(t) / (divs == 1 ? S : S * S2);
  }
};

// Binade of a positive normal float (kNoBinade otherwise).
__device__ __forceinline__ short binade_of(float v) {
  const uint32_t b = __float_as_uint(v);
  const int E = (int)(b >> 23);
  return v > 0.0f && E >= 1 && E <= 254 ? (short)(E - 127) : kNoBinade;
}

// The unit increment of a value v in binade e decided from an estimate va:
// round to nearest of v / u (u = 2^(e-23)).  __expf is within 9.9e-7
// (relative) of the exact expf on every float argument of this path (all
// 1.1e9 floats in [-17.5, 0], checked on the device), and each division
// after it adds at most one more rounding, so |va - v| < 1.3e-6 v: when
// va / u lies farther than 1e-5 va / u + 1e-6 from a half-integer, v / u
// lies on the same side of it and is no tie.  Returns false (v is needed
// exactly) otherwise, or from 2^15 units up.
__device__ __forceinline__ bool quick_inc(float va, int e, unsigned& inc) {
  const float z = ldexpf(va, 23 - e);
  inc = 0u;
  if (z < 0.49f) return true;
  if (!(z < 32768.0f)) return false;
  const float fl = floorf(z), f = z - fl;  // exact: z < 2^15
  if (fabsf(f - 0.5f) <= 1e-5f * z + 1e-6f) return false;
  inc = (unsigned)fl + (f > 0.5f ? 1u : 0u);
  return true;
}

// Adds v's unit increment in binade e to bucket b; a tie, or a step that
// alone leaves the binade, marks the bucket to be walked (bit 63).
__device__ __forceinline__ void add_inc(BucketSmem& bs, int b, float v, int e) {
  int a, rnd;
  bool tie;
  split_at(v, e, a, rnd, tie);
  if (tie || a >= kDeltaCap)
    atomicOr(&bs.inc[b], 1ull << 63);
  else if (a + rnd)
    atomicAdd(&bs.inc[b], (unsigned long long)(a + rnd));
}

// Sorts keys[0, n) descending in place, with their indices idx[0, n),
// n <= kWaveSortMax, by one wave: each key's rank among the n (equal keys
// keep their order).
__device__ __forceinline__ void wave_sort_desc(uint32_t* keys, uint32_t* idx, int n,
                                               uint32_t* stg) {
  const int lane = threadIdx.x & 63;
  if (n <= 64) {
    const uint32_t k = lane < n ? keys[lane] : 0u, x = lane < n ? idx[lane] : 0u;
    int r = 0;
    for (int j = 0; j < n; ++j) {
      const uint32_t o = (uint32_t)readlane_i((int)k, j);
      r += o > k || (o == k && j < lane);
    }
    if (lane < n) {
      keys[r] = k;
      idx[r] = x;
    }
    return;
  }
  uint32_t mk[kWaveSortMax / 64], mx[kWaveSortMax / 64];
#pragma unroll
  for (int q = 0; q < kWaveSortMax / 64; ++q) {
    const int i = lane + 64 * q;
    mk[q] = i < n ? keys[i] : 0u;
    mx[q] = i < n ? idx[i] : 0u;
    if (i < n) stg[i] = mk[q];
  }
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int q = 0; q < kWaveSortMax / 64; ++q) {
    const int i = lane + 64 * q;
    if (i >= n) continue;
    int r = 0;
    for (int j = 0; j < n; ++j) {
      const uint32_t o = stg[j];
      r += o > mk[q] || (o == mk[q] && j < i);
    }
    keys[r] = mk[q];
    idx[r] = mx[q];
  }
}

// Calls f(valid, i, x) for every logit x = row[i] with the whole wave
// converged (lanes past the end get valid = false): 16-byte vectors, U in
// flight, when VEC, then the elements past the last vector.
template <bool VEC, int U, class F>
__device__ __forceinline__ void row_converged(const char* row, int V, F&& f) {
  const int lane = threadIdx.x & 63, w0 = (threadIdx.x >> 6) * 64;
  int done = 0;
  if constexpr (VEC) {
    const int nvec = V / 4;
    for (int base = w0; base < nvec; base += U * kST) {
      u32x4 wb[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = base + u * kST + lane;
        wb[u] = v < nvec ? ld16(row + (size_t)v * 16) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int v = base + u * kST + lane;
#pragma unroll
        for (int j = 0; j < 4; ++j) f(v < nvec, 4 * v + j, __uint_as_float(wb[u][j]));
      }
    }
    done = nvec * 4;
  }
  for (int base = done + w0; base < V; base += kST) {
    const int i = base + lane;
    f(i < V, i, i < V ? reinterpret_cast<const float*>(row)[i] : 0.0f);
  }
}

// Wave 0: the f32 running sum s over sorted positions [lo, hi) -- the top of
// the order from bs.topv (positions below nA), the rest from the keys in K --
// stopping at the first sum >= thr (use_thr; *pos gets its position).  Per
// 64 positions: while s is a normal number, the two-parity deltas of the 64
// additions in s's binade, composed across the lanes, give every prefix sum;
// from the first one that leaves the binade or reaches thr, real f32
// additions.
__device__ __forceinline__ void walk_sorted(const BucketSmem& bs, const uint32_t* K, int nA, int lo, int hi,
                            float& s, int& pos, bool use_thr, float thr, const BucketValue vf) {
  const int lane = threadIdx.x & 63;
  for (int i0 = lo; i0 < hi && pos < 0; i0 += 64) {
    const int m = min(64, hi - i0), i = i0 + lane;
    const float v = lane >= m ? 0.0f : i < nA ? bs.topv[i] : vf(K[i]);
    const uint32_t sb = __float_as_uint(s);
    const int sE = (int)((sb >> 23) & 255u);
    int j0 = 0;
    if (sE >= 1 && sE <= 254 && !(sb >> 31)) {
      const int e = sE - 127;
      int a, rnd;
      bool tie;
      split_at(v, e, a, rnd, tie);
      int p0 = tie ? a + (a & 1) : min(a + rnd, kDeltaCap);
      int p1 = tie ? a + ((a + 1) & 1) : min(a + rnd, kDeltaCap);
      compose_scan(p0, p1);
      const long long n = (long long)((sb & 0x7fffffu) | 0x800000u);
      const long long nend = n + ((n & 1) ? p1 : p0);
      const float send = nend < (1ll << 24) ? ldexpf((float)nend, e - 23) : INFINITY;
      const unsigned long long bad =
          __ballot(lane < m && (nend >= (1ll << 24) || (use_thr && send >= thr)));
      if (!bad) {
        s = readlane_f(send, m - 1);
        continue;
      }
      j0 = __builtin_ctzll(bad);
      if (j0 > 0) s = readlane_f(send, j0 - 1);
    }
    for (int j = j0; j < m; ++j) {
      s = s + readlane_f(v, j);
      if (use_thr && s >= thr) {
        pos = i0 + j;
        break;
      }
    }
  }
}

// Wave 0: the sum over the top of the order, positions [0, hi) (values in
// bs.topv; chunk c = positions [64 c, 64 c + 64), with its deltas for the
// binade predicted at its start in bs.ch_*): runs of chunks whose prediction
// holds are applied with a composition scan across the lanes, one chunk a
// lane; any other chunk is walked as walk_sorted walks 64 positions.
__device__ __forceinline__ void walk_top(const BucketSmem& bs, int hi, float& s, int& pos,
                                         bool use_thr, float thr, const BucketValue vf) {
  const int lane = threadIdx.x & 63;
  const int nch = (hi + 63) / 64;  // <= 64
  int c = 0;
  while (c < nch && pos < 0) {
    const uint32_t sb = __float_as_uint(s);
    const int sE = (int)((sb >> 23) & 255u);
    const bool sn = sE >= 1 && sE <= 254 && !(sb >> 31);  // wave-uniform
    const int es = sE - 127;
    const int g = c + lane;
    const unsigned long long okm = __ballot(g < nch && sn && bs.ch_e[g] == es);
    const int run = ~okm ? __builtin_ctzll(~okm) : 64;
    int d0 = lane < run ? bs.ch_d0[g] : 0, d1 = lane < run ? bs.ch_d1[g] : 0;
    compose_scan(d0, d1);
    const long long n = (long long)((sb & 0x7fffffu) | 0x800000u);
    const long long nend = n + ((n & 1) ? d1 : d0);
    const float send = nend < (1ll << 24) ? ldexpf((float)nend, es - 23) : INFINITY;
    const unsigned long long stm =
        __ballot(sn && lane < run && (nend >= (1ll << 24) || (use_thr && send >= thr)));
    const int upto = stm ? __builtin_ctzll(stm) : run;
    if (sn && upto > 0) s = readlane_f(send, upto - 1);
    c += upto;
    if (c >= nch) break;
    walk_sorted(bs, nullptr, hi, 64 * c, min(64 * c + 64, hi), s, pos, use_thr, thr, vf);
    ++c;
  }
}

// Why walk_scan stopped at bucket bs.todo (not stored): the sum is in another
// binade than the one its increments were summed for; or the bucket holds a
// tie, or the sum leaves its binade or reaches thr inside it.
constexpr int kWhyRebin = 1, kWhyStore = 2;

// Wave 0: continues the walk from bucket bs.b with sum bs.s over buckets
// [0, nbk) (`part` kept only below position len).  Stored buckets are walked
// in sorted order; others are applied as prefix sums of their increments
// while the sum stays in their binade and below thr.  Stops at the first
// position where the sum reaches thr (bs.pos), at nbk, or at a bucket that
// needs another pass over the row (bs.todo, bs.why).
__device__ __forceinline__ void walk_scan(BucketSmem& bs, const uint32_t* K, int nA, int bA,
                                          int nbk, int part, int len, bool use_thr, float thr,
                                          const BucketValue vf) {
  const int lane = threadIdx.x & 63;
  float s = bs.s;
  int b = bs.b, todo = -1, why = 0, pos = -1;
  if (b == 0) {  // the top of the order, buckets [0, bA) (nbk <= bA when top_k cuts there)
    walk_top(bs, min(nA, len), s, pos, use_thr, thr, vf);
    b = min(bA, nbk);
  }
  while (b < nbk && pos < 0) {
    if (bs.flag[b] & kStored) {  // the stretch of stored buckets from b
      int e2 = b;
      for (;;) {
        const int g = e2 + lane;
        const unsigned long long st = __ballot(g < nbk && (bs.flag[g] & kStored));
        const int k = ~st ? __builtin_ctzll(~st) : 64;
        e2 += k;
        if (k < 64) break;
      }
      const int hi = e2 - 1 == part ? len : (int)bs.start[e2];
      walk_sorted(bs, K, nA, (int)bs.start[b], hi, s, pos, use_thr, thr, vf);
      b = e2;
      continue;
    }
    const int g = b + lane;
    const bool have = g < nbk;
    const bool stored = have && (bs.flag[g] & kStored);
    const int e = have ? bs.eg[g] : kNoBinade;
    const unsigned c = have ? bs.start[g + 1] - bs.start[g] : 0u;
    const unsigned long long iv = have ? bs.inc[g] : 0ull;
    const unsigned d = (unsigned)min(iv, (unsigned long long)kDeltaCap);
    const uint32_t sb = __float_as_uint(s);
    const int sE = (int)((sb >> 23) & 255u);
    const bool sn = sE >= 1 && sE <= 254 && !(sb >> 31);  // wave-uniform
    const int es = sE - 127;
    // lanes 0 .. run-1: empty buckets, or buckets summed for this binade
    const unsigned long long okm =
        __ballot(have && !stored && (c == 0u || (sn && (iv >> 63) == 0ull && e == es)));
    const int run = ~okm ? __builtin_ctzll(~okm) : 64;
    const long long n = (long long)((sb & 0x7fffffu) | 0x800000u);
    // 64 (2^24 + 1) < 2^32
    const long long nend = n + (long long)wave_incl_add_u32(lane < run && c ? d : 0u);
    const float send = nend < (1ll << 24) ? ldexpf((float)nend, es - 23) : INFINITY;
    const unsigned long long stm = __ballot(sn && lane < run && c != 0u &&
                                            (nend >= (1ll << 24) || (use_thr && send >= thr)));
    const int upto = stm ? __builtin_ctzll(stm) : run;
    if (sn && upto > 0) s = readlane_f(send, upto - 1);
    b += upto;
    if (stm) {
      todo = b;
      why = kWhyStore;
      break;
    }
    if (b >= nbk || run == 64 || readlane_i(stored, run)) continue;
    todo = b;  // bucket b: summed for another binade, or a tie
    why = sn && readlane_i(e, run) != es ? kWhyRebin : kWhyStore;
    break;
  }
  if (lane == 0) {
    bs.s = s;
    bs.b = b;
    bs.todo = todo;
    bs.why = why;
    bs.pos = pos;
  }
}

template <bool VEC>
struct BucketRow {
  const char* x;
  int V;
  bool neg;
  float aT, ymax, scale;
  // bucket of y, from t = y - max y (smaller t: the same or a later bucket)
  __device__ __forceinline__ int bucket(float t) const {
    const float d = -t;
    if (!(d < kDTail)) return kBk;
    const float f = d * scale;
    return f < (float)kBk ? (int)f : kBk - 1;
  }
  template <class F>
  __device__ __forceinline__ void each(F&& f) const {  // f(x', t) for every logit
    for_each<PKV_F32, VEC, 4>(x, V, [&](int, float v) {
      const float xp = neg ? -v : v;
      f(xp, xp / aT - ymax);
    });
  }
};

// Sorts every stored, unsorted bucket in [b0, nbk) (keys in K, indices in
// KI): one wave per bucket, then the workgroup for those over kWaveSortMax.
// Returns false when one holds more than kBkSortMax keys.  All threads; ends
// with a barrier.
__device__ __forceinline__ bool sort_stored(BucketSmem& bs, uint32_t* K, uint32_t* KI, int b0,
                                            int nbk) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  if (tid == 0) bs.big = 0;
  __syncthreads();
  for (int b = b0 + wv; b < nbk; b += kSW) {
    if ((bs.flag[b] & (kStored | kSorted)) != kStored) continue;  // wave-uniform
    const int st = (int)bs.start[b], n = (int)bs.start[b + 1] - st;
    if (n > kWaveSortMax) {
      if (lane == 0) atomicAdd(&bs.big, 1);
      continue;
    }
    wave_sort_desc(K + st, KI + st, n, bs.stage[wv]);
    if (lane == 0) bs.flag[b] |= kSorted;
  }
  __syncthreads();
  if (bs.big == 0) return true;
  uint32_t* stg = &bs.stage[0][0];
  for (int b = b0; b < nbk; ++b) {  // uniform
    if ((bs.flag[b] & (kStored | kSorted)) != kStored) continue;
    const int st = (int)bs.start[b], n = (int)bs.start[b + 1] - st;
    if (n > kBkSortMax) return false;
    uint32_t mx[kBkSortMax / kST];
#pragma unroll
    for (int q = 0; q < kBkSortMax / kST; ++q) {
      const int i = tid + q * kST;
      if (i < n) {
        stg[i] = K[st + i];
        mx[q] = KI[st + i];
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kBkSortMax / kST; ++q) {
      const int i = tid + q * kST;
      if (i >= n) continue;
      const uint32_t k = stg[i];
      int r = 0;
      for (int j = 0; j < n; ++j) {
        const uint32_t o = stg[j];
        r += o > k || (o == k && j < i);
      }
      K[st + r] = k;
      KI[st + r] = mx[q];
    }
    __syncthreads();
    if (tid == 0) bs.flag[b] |= kSorted;
  }
  __syncthreads();
  return true;
}

// The f32 running sum of vf over the kept sorted positions [0, len) --
// buckets [0, nbk), `part` (if >= 0) kept only up to len -- up to and
// including the first sum >= thr (use_thr).  Results: bs.s, and bs.pos the
// position where thr was reached (-1: not reached).  Returns false when a
// bucket to sort is too large (the row is left to the sort kernel).  All
// threads; ends with a barrier.
template <bool VEC>
__device__ __forceinline__ bool bucket_walk(BucketSmem& bs, uint32_t* K, uint32_t* KI,
                                            const BucketRow<VEC>& rw, int nA, int bA, int nbk,
                                            int part, int len, bool use_thr, float thr,
                                            const BucketValue vf) {
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  // the top's values, and per chunk of 64 its deltas in the binade the sum
  // is predicted to enter it with (float prefix sums of the chunks)
  const int hiA = min(nA, len), nch = (hiA + 63) / 64;
  for (int i = tid; i < hiA; i += kST) bs.topv[i] = vf(bs.topk[i]);
  __syncthreads();
  for (int c = wv; c < nch; c += kSW) {
    const int i = 64 * c + lane;
    const float t = wsum_f32(i < hiA ? bs.topv[i] : 0.0f);
    if (lane == 0) bs.ch_sum[c] = t;
  }
  __syncthreads();
  for (int c = wv; c < nch; c += kSW) {
    float pre = 0.0f;
    for (int q = 0; q < c; ++q) pre += bs.ch_sum[q];
    const int e = use_thr && pre > thr * 1.0625f ? kNoBinade : binade_of(pre);
    int d0 = 0, d1 = 0;
    if (e != kNoBinade) {  // wave-uniform
      const int i = 64 * c + lane;
      int a, rnd;
      bool tie;
      split_at(i < hiA ? bs.topv[i] : 0.0f, e, a, rnd, tie);
      d0 = tie ? a + (a & 1) : min(a + rnd, kDeltaCap);
      d1 = tie ? a + ((a + 1) & 1) : min(a + rnd, kDeltaCap);
      compose_scan(d0, d1);
    }
    if (lane == 63) {
      bs.ch_e[c] = e;
      bs.ch_d0[c] = d0;
      bs.ch_d1[c] = d1;
    }
  }
  if (tid == 0) {
    bs.s = 0.0f;
    bs.b = 0;
  }
  __syncthreads();
  for (;;) {
    if (wv == 0) walk_scan(bs, K, nA, bA, nbk, part, len, use_thr, thr, vf);
    __syncthreads();
    const int todo = bs.todo, why = bs.why;
    if (todo < 0) break;  // (every thread reads bs.todo before it changes again)
    if (why == kWhyRebin) {
      // the buckets from todo on that were predicted like todo: the actual
      // binade of the sum, their increments again
      const int wrong = bs.eg[todo];
      const uint32_t sb = __float_as_uint(bs.s);
      const int es = (int)((sb >> 23) & 255u) - 127;
      __syncthreads();
      for (int b = todo + tid; b < nbk; b += kST) {
        if (bs.eg[b] == wrong && !(bs.flag[b] & kStored)) {
          bs.eg[b] = (short)es;
          bs.inc[b] = 0ull;
        }
      }
      __syncthreads();
      rw.each([&](float, float t) {
        const int b = rw.bucket(t);
        if (b < todo || b >= nbk || bs.eg[b] != es || (bs.flag[b] & kStored)) return;
        unsigned qi;
        if (!quick_inc(vf.approx(t), es, qi)) add_inc(bs, b, vf.of_t(t), es);
        else if (qi) atomicAdd(&bs.inc[b], (unsigned long long)qi);
      });
      __syncthreads();
      continue;
    }
    // store the keys of todo and the next buckets not stored
    for (int b = todo + tid; b < min(nbk, todo + kGatherSpan); b += kST)
      if (!(bs.flag[b] & kStored)) bs.flag[b] = kGather;
    __syncthreads();
    row_converged<VEC, 4>(rw.x, rw.V, [&](bool valid, int i, float v) {
      const float xp = rw.neg ? -v : v;
      const int b = valid ? rw.bucket(xp / rw.aT - rw.ymax) : kBk;
      if (b < kBk && (bs.flag[b] & kGather)) {
        const unsigned p = bs.start[b] + atomicAdd(&bs.cur[b], 1u);
        K[p] = order_key(xp);
        KI[p] = (uint32_t)i;
      }
    });
    __syncthreads();
    for (int b = tid; b < kBk; b += kST)
      if (bs.flag[b] & kGather) bs.flag[b] = kStored;
    __syncthreads();
    if (!sort_stored(bs, K, KI, todo, nbk)) return false;
  }
  __syncthreads();
  return true;
}

template <bool VEC>
__global__ void __launch_bounds__(kST) sample_bucket_kernel(ExactArgs a) {
  __shared__ BucketLds u;
  SampleSmem& sm = u.sm;
  BucketSmem& bs = u.bs;
  const int row = a.row0 + blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const char* x = a.logits + (long long)row * a.stride_bytes;
  const int V = a.vocab;
  const float T = a.temps ? a.temps[row] : 0.0f;
  if (T == 0.0f || V <= 1) {  // sample.rs:13-15
    float bv;
    int bi;
    block_argmax<PKV_F32, VEC>(sm, x, 0, V, bv, bi);
    if (tid == 0) {
      a.tokens[row] = bi == INT_MAX ? 0 : bi;
      a.fallback[row] = 0;
      if (a.route) a.route[row] = kRouteArgmax;
    }
    return;
  }
  auto leave = [&]() {
    if (tid == 0) a.fallback[row] = 1;
  };
  const bool neg = T < 0.0f;
  const float aT = fabsf(T);  // y = x / T = x' / |T| with x' = x, or -x when T < 0

  // 1. the largest and smallest x', and whether a logit is NaN
  if (tid < 32) bs.exptab[tid] = kExp2Tab[tid];
  float hi = -INFINITY, lo = INFINITY;
  bool nan = false;
  for_each<PKV_F32, VEC, kRowBatch>(x, V, [&](int, float v) {
    const float xp = neg ? -v : v;
    hi = fmaxf(hi, xp);
    lo = fminf(lo, xp);
    nan |= v != v;
  });
  hi = wave_reduce32(hi, [](float p, float q) { return fmaxf(p, q); });
  lo = wave_reduce32(lo, [](float p, float q) { return fminf(p, q); });
  const bool wnan = __ballot(nan) != 0ull;
  if (lane == 0) {
    bs.wf[wv] = hi;
    bs.wg[wv] = lo;
    bs.wi[wv] = wnan;
  }
  __syncthreads();
  bool anynan = false;
  for (int w = 0; w < kSW; ++w) {
    hi = fmaxf(hi, bs.wf[w]);
    lo = fminf(lo, bs.wg[w]);
    anynan |= bs.wi[w] != 0;
  }
  const float ymax = hi / aT, ymin = lo / aT;
  if (anynan || !(fabsf(ymax) < INFINITY)) {  // uniform
    leave();
    return;
  }
  const float D = fminf(ymax - ymin, kDTail);
  const BucketRow<VEC> rw{x, V, neg, aT, ymax,
                          D > 0.0f ? fminf((float)kBk / D, 0x1p100f) : 0.0f};

  // 2. logits and approximate mass (2^-40 units) per bucket; the tail only
  // counted
  for (int i = tid; i <= kBk; i += kST) bs.cur[i] = 0u;
  for (int i = tid; i < kBk; i += kST) bs.inc[i] = 0ull;
  __syncthreads();
  rw.each([&](float, float t) {
    const int b = rw.bucket(t);
    const unsigned long long tl = __ballot(b == kBk);
    if (tl && lane == __builtin_ctzll(__ballot(true)))
      atomicAdd(&bs.cur[kBk], (unsigned)__popcll(tl));
    if (b < kBk) {
      atomicAdd(&bs.cur[b], 1u);
      atomicAdd(&bs.inc[b], (unsigned long long)(__expf(t) * 0x1p40f));
    }
  });
  __syncthreads();

  // 3. exclusive prefixes: bucket starts (the tail last) and masses
  {
    const int b0 = 4 * tid;
    unsigned c[4];
    unsigned long long m[4];
    unsigned cs = 0u;
    unsigned long long ms = 0ull;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = bs.cur[b0 + j];
      m[j] = bs.inc[b0 + j];
      cs += c[j];
      ms += m[j];
    }
    const unsigned tail = bs.cur[kBk];
    unsigned total;
    unsigned pre = block_excl_scan(cs, bs.wtmp, total);
    const unsigned long long mincl = wave_incl_u64(ms);
    if (lane == 63) bs.wu[wv] = mincl;
    __syncthreads();
    unsigned long long mpre = mincl - ms, mtot = 0ull;
    for (int w = 0; w < kSW; ++w) {
      if (w < wv) mpre += bs.wu[w];
      mtot += bs.wu[w];
    }
    // ... and the denominator's f32 running sum predicted at each bucket's
    // start (into cur, as floats): a bucket of small probabilities adds each
    // rounded to whole units of the sum's binade (its logits are within a
    // factor exp(1 / scale) of its centre), which the mass alone misses
    float est[4], es = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float pmj = (float)mpre * 0x1p-40f, mj = (float)m[j] * 0x1p-40f;
      bs.start[b0 + j] = pre;
      pre += c[j];
      bs.pm[b0 + j] = pmj;
      mpre += m[j];
      const int e = binade_of(pmj);
      const float unit = e == kNoBinade ? 0.0f : ldexpf(1.0f, e - 23);
      const float z = e == kNoBinade ? 1e9f : __expf(-((float)(b0 + j) + 0.5f) / rw.scale) / unit;
      est[j] = z < 256.0f ? (float)c[j] * rintf(z) * unit : mj;
      es += est[j];
    }
    if (tid == kST - 1) {
      bs.start[kBk] = pre;
      bs.start[kBk + 1] = pre + tail;
      bs.pm[kBk] = (float)mtot * 0x1p-40f;
    }
    const float ein = wave_incl_add_f32(es);
    if (lane == 63) bs.wf[wv] = ein;
    __syncthreads();  // (every read of cur as counts is done)
    float epre = ein - es;
    for (int w = 0; w < wv; ++w) epre += bs.wf[w];
    float* pc = reinterpret_cast<float*>(bs.cur);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      pc[b0 + j] = epre;
      epre += est[j];
    }
    if (tid == kST - 1) pc[kBk] = epre;
  }
  __syncthreads();

  // top_k: positions [0, len) are kept; buckets [0, nbk) are in play and
  // `part` is kept only in part (a cut inside the tail drops nothing that
  // matters)
  const int nreg = (int)bs.start[kBk];
  int len = a.top_k > 0 && a.top_k < V ? a.top_k : V;
  int nbk = kBk, part = -1;
  auto cut_at = [&](int n) {
    nbk = kBk;
    part = -1;
    if (n < nreg) {  // the bucket of position n - 1: the last with start < n
      int l = 0, h = kBk - 1;
      while (l < h) {
        const int mid = (l + h + 1) >> 1;
        if ((int)bs.start[mid] < n) l = mid;
        else h = mid - 1;
      }
      nbk = l + 1;
      part = (int)bs.start[l + 1] > n ? l : -1;
    }
  };
  cut_at(len);
  // the top of the order: buckets [0, bA), positions [0, nA), nA <= kRegionA
  // (bucket 0 must fit)
  int bA = 0;
  {
    int l = 0, h = nbk;
    while (l < h) {
      const int mid = (l + h + 1) >> 1;
      if ((int)bs.start[mid] <= kRegionA) l = mid;
      else h = mid - 1;
    }
    bA = l;
  }
  if (bA == 0) {  // uniform: bucket 0 alone holds more than kRegionA logits
    leave();
    return;
  }
  const int nA = (int)bs.start[bA];

  // 4. which buckets to store: the top, the top_k cut, the buckets around
  // each one where the denominator is predicted to leave its binade, and
  // (with a margin) each bucket where top_p's sum of p / S or r's of p / S
  // (/ S2, about top_p when top_p < 1: the kept sum first reaches top_p) is
  // predicted to reach its threshold; the others get the binade the
  // denominator is predicted to have at their start
  const float* pc = reinterpret_cast<const float*>(bs.cur);
  for (int b = tid; b < kBk; b += kST)
    bs.flag[b] = b >= bA && b < nbk && bs.start[b + 1] > bs.start[b] &&
                 binade_of(pc[b]) != binade_of(pc[b + 1]) ? kGather : 0;
  __syncthreads();
  short egp[kBk / kST];
#pragma unroll
  for (int q = 0; q < kBk / kST; ++q) egp[q] = binade_of(pc[tid + q * kST]);
  __syncthreads();  // (cur is cleared below)
  const float Sest = bs.pm[kBk];
  const bool has_p = a.top_p == a.top_p;  // Some(top_p)
  const float S3est = Sest * (has_p ? fminf(fmaxf(a.top_p, 0x1p-20f), 1.0f) : 1.0f);
  auto reaches = [&](int b, float div, float thr) {
    return bs.pm[b] * (1.0f - kMargin) / div <= thr * (1.0f + kMargin) &&
           bs.pm[b + 1] * (1.0f + kMargin) / div >= thr * (1.0f - kMargin);
  };
  unsigned char fl[kBk / kST];
#pragma unroll
  for (int q = 0; q < kBk / kST; ++q) {
    const int b = tid + q * kST;
    bool near = false;
    for (int o = max(b - 2, 0); o <= min(b + 2, kBk - 1); ++o) near |= bs.flag[o] == kGather;
    const bool st = b < bA || b == part ||
                    (b < nbk && bs.start[b + 1] > bs.start[b] &&
                     (near || reaches(b, S3est, a.r) || (has_p && reaches(b, Sest, a.top_p))));
    fl[q] = b < bA ? kStored | kSorted : st ? kStored : 0;
    bs.eg[b] = st ? kNoBinade : egp[q];
    bs.inc[b] = 0ull;
    bs.cur[b] = 0u;
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < kBk / kST; ++q) bs.flag[tid + q * kST] = fl[q];
  __syncthreads();

  // 5. store the flagged buckets' keys (the top in LDS); the others'
  // increments for the denominator, decided from __expf where it settles
  // the rounding (quick_inc) and otherwise from the exact value (through a
  // per-wave queue in LDS, so that the exact exponentials and splits run on
  // full waves)
  uint32_t* K = a.scratch + (size_t)blockIdx.x * 2 * (size_t)V;  // keys
  uint32_t* KI = K + V;                                           // their indices
  const BucketValue p_of{aT, ymax, 1.0f, 1.0f, 0, bs.exptab};
  {
    float* qt = reinterpret_cast<float*>(bs.stage[wv]);
    int* qb = reinterpret_cast<int*>(bs.stage[wv]) + 128;
    static_assert(kWaveSortMax >= 256, "a queue of 128 (t, bucket) pairs per wave");
    int qn = 0;  // wave-uniform
    auto drain = [&](int n) {
      if (lane < n) {
        const int b = qb[lane];
        add_inc(bs, b, p_of.of_t(qt[lane]), bs.eg[b]);
      }
    };
    row_converged<VEC, 4>(x, V, [&](bool valid, int i, float v) {
      const float xp = neg ? -v : v;
      const float t = xp / aT - ymax;
      const int b = valid ? rw.bucket(t) : kBk;
      const bool play = b < nbk;
      const unsigned char fl = play ? bs.flag[b] : 0;
      if (play && (fl & kStored)) {  // the top in LDS, other stored buckets in K
        const unsigned p = bs.start[b] + atomicAdd(&bs.cur[b], 1u);
        if (b < bA) {
          bs.topk[p] = order_key(xp);
          bs.topi[p] = (uint32_t)i;
        } else {
          K[p] = order_key(xp);
          KI[p] = (uint32_t)i;
        }
      }
      const int e = play && !(fl & kStored) ? bs.eg[b] : kNoBinade;
      bool push = false;
      if (e != kNoBinade) {
        unsigned qi;
        if (!quick_inc(__expf(t), e, qi)) push = true;  // the exact value, through the queue
        else if (qi) atomicAdd(&bs.inc[b], (unsigned long long)qi);
      }
      const unsigned long long m = __ballot(push);
      if (m) {  // wave-uniform
        const int at = qn + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                           __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        if (push) {
          qt[at] = t;
          qb[at] = b;
        }
        qn += __popcll(m);
        if (qn >= 64) {
          drain(64);
          if (lane < qn - 64) {
            qt[lane] = qt[64 + lane];
            qb[lane] = qb[64 + lane];
          }
          qn -= 64;
        }
      }
    });
    drain(qn);
  }
  __syncthreads();
  // the top, sorted in LDS: each key's rank within its bucket
  {
    uint32_t* stg = &bs.stage[0][0];
    static_assert(kRegionA <= kBkSortMax, "the top is staged in one piece");
    uint32_t mk[kRegionA / kST], mx[kRegionA / kST];
#pragma unroll
    for (int q = 0; q < kRegionA / kST; ++q) {
      const int i = tid + q * kST;
      if (i < nA) {
        mk[q] = bs.topk[i];
        mx[q] = bs.topi[i];
        stg[i] = mk[q];
      }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < kRegionA / kST; ++q) {
      const int i = tid + q * kST;
      if (i >= nA) continue;
      int l = 0, h = bA - 1;  // the bucket of position i: the last with start <= i
      while (l < h) {
        const int mid = (l + h + 1) >> 1;
        if ((int)bs.start[mid] <= i) l = mid;
        else h = mid - 1;
      }
      const int st = (int)bs.start[l], en = (int)bs.start[l + 1];
      int r = 0;
      for (int j = st; j < en; ++j) {
        const uint32_t o = stg[j];
        r += o > mk[q] || (o == mk[q] && j < i);
      }
      bs.topk[st + r] = mk[q];
      bs.topi[st + r] = mx[q];
    }
    __syncthreads();
  }
  if (!sort_stored(bs, K, KI, bA, nbk) ||
      !bucket_walk(bs, K, KI, rw, nA, bA, nbk, part, len, false, 0.0f, p_of)) {
    leave();  // sum += p
    return;
  }
  const float S = bs.s;

  // predictions (mass prefixes over div) and increments of vf for a
  // threshold run, for the buckets not stored below the first one predicted
  // past thr (the walk stops before it); one more pass over the row when any
  // bucket needs them
  auto prepare = [&](float div, float thr, const BucketValue& vf) {
    int bc = nbk;
    for (int b = tid; b < nbk; b += kST)
      if (bs.pm[b] / div > thr * 1.0625f) {
        bc = b;
        break;
      }
    bc = wave_reduce32(bc, [](int p, int q) { return min(p, q); });
    if (lane == 0) bs.wi[wv] = bc;
    __syncthreads();
    for (int w = 0; w < kSW; ++w) bc = min(bc, bs.wi[w]);
    bool need = false;
    for (int b = tid; b < kBk; b += kST) {
      const bool pr = b < bc && !(bs.flag[b] & kStored) && bs.start[b + 1] > bs.start[b];
      bs.eg[b] = pr ? binade_of(bs.pm[b] / div) : kNoBinade;
      bs.inc[b] = 0ull;
      need |= pr;
    }
    need = __ballot(need) != 0ull;
    if (lane == 0) bs.wtmp[wv] = need;
    __syncthreads();
    bool any = false;
    for (int w = 0; w < kSW; ++w) any |= bs.wtmp[w] != 0u;
    if (any) {
      rw.each([&](float, float t) {
        const int b = rw.bucket(t);
        if (b >= nbk) return;
        const int e = bs.eg[b];
        if (e == kNoBinade) return;
        unsigned qi;
        if (!quick_inc(vf.approx(t), e, qi)) add_inc(bs, b, vf.of_t(t), e);
        else if (qi) atomicAdd(&bs.inc[b], (unsigned long long)qi);
      });
    }
    __syncthreads();
  };

  float S2 = 1.0f;
  if (has_p) {  // cumulative q until it reaches top_p; keep that prefix
    const BucketValue q_of{aT, ymax, S, 1.0f, 1, bs.exptab};
    prepare(S, a.top_p, q_of);
    if (!bucket_walk(bs, K, KI, rw, nA, bA, nbk, part, len, true, a.top_p, q_of)) {
      leave();
      return;
    }
    S2 = bs.s;  // the f32 sum of the kept q
    if (bs.pos >= 0) {
      len = bs.pos + 1;
      cut_at(len);
    }
  }
  const BucketValue r_of{aT, ymax, S, S2, has_p ? 2 : 1, bs.exptab};
  prepare(has_p ? S * S2 : S, a.r, r_of);
  if (!bucket_walk(bs, K, KI, rw, nA, bA, nbk, part, len, true, a.r, r_of) || bs.pos < 0) {
    leave();  // (not reached: the reference takes the last kept token)
    return;
  }
  // the token at sorted position j: the tokens of its y (all in its bucket,
  // stored and sorted by key; equal keys in any order) are in index order in
  // the reference's stable sort, so it is the (j - g0)-th smallest index of
  // that group, g0 its first position
  const int j = bs.pos;
  auto key_at = [&](int i) { return i < nA ? bs.topk[i] : K[i]; };
  auto idx_at = [&](int i) { return i < nA ? bs.topi[i] : KI[i]; };
  const float yj = key_value(key_at(j)) / aT;
  const uint32_t ky = order_key(yj);
  const int bj = rw.bucket(yj - ymax);
  const int st = (int)bs.start[bj], en = (int)bs.start[bj + 1];
  int before = 0, all = 0;
  for (int i = st + tid; i < en; i += kST) {
    const bool same = order_key(key_value(key_at(i)) / aT) == ky;
    before += same && i < j;
    all += same;
  }
  before = wsum_i32(before);
  all = wsum_i32(all);
  if (lane == 0) {
    bs.wi[wv] = before;
    bs.wtmp[wv] = (unsigned)all;
  }
  if (tid == 0) bs.tok = 0;
  __syncthreads();
  int g0 = j, g1 = 0;
  for (int w = 0; w < kSW; ++w) {
    g0 -= bs.wi[w];
    g1 += (int)bs.wtmp[w];
  }
  g1 += g0;
  const int want = j - g0;  // the rank wanted among the group's indices
  for (int i = g0 + tid; i < g1; i += kST) {
    const uint32_t xi = idx_at(i);
    int r = 0;
    for (int q = g0; q < g1; ++q) r += idx_at(q) < xi;
    if (r == want) bs.tok = (int)xi;
  }
  __syncthreads();
  if (tid == 0) {
    a.tokens[row] = bs.tok;
    a.fallback[row] = 0;
    if (a.route) a.route[row] = kRouteBuckets;
  }
}

// The exp the exact path uses, for verification: out[i] = expf_glibc(in[i]).
__global__ void expf_glibc_kernel(const float* in, float* out, long long n) {
  for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (long long)gridDim.x * blockDim.x)
    out[i] = expf_glibc(in[i]);
}

// Rows per launch of the exact path: the key scratch (8 bytes per logit)
// stays within kExactScratch bytes.
constexpr size_t kExactScratch = 512ull << 20;

template <int DT, bool VEC>
void launch_exact_rows(const ExactArgs& a, int rows, hipStream_t stream) {
  if constexpr (DT == PKV_F32) {
    // sampled rows go to the buckets first; the rows they leave (a.fallback)
    // to the runs of equal values when every logit is a bf16 value, then to
    // the sort
    if (a.fallback) {
      sample_bucket_kernel<VEC><<<rows, kST, 0, stream>>>(a);
      sample_runs_kernel<DT, VEC><<<rows, kST, 0, stream>>>(a);
    }
    sample_exact_kernel<DT, VEC><<<rows, kST, 0, stream>>>(a);
  } else {
    sample_runs_kernel<DT, VEC><<<rows, kST, 0, stream>>>(a);
  }
}

template <int DT, bool VEC>
hipError_t launch_exact_dt(const ExactArgs& a0, int batch, hipStream_t stream) {
  if (!grid_fits(batch, kST)) return hipErrorInvalidValue;
  if (!a0.temps || a0.vocab <= 1) {  // every row is argmax: no scratch
    launch_exact_rows<DT, VEC>(a0, batch, stream);
    return hipGetLastError();
  }
  // scratch per row: the runs (keys, counts, starts, values); f32 logits
  // also the two key arrays of the radix sort (the kernels run one after the
  // other), and a fallback flag per row of the call
  const size_t runs_row = (size_t)4 * kMaxRuns * sizeof(uint32_t);
  const size_t per_row =
      DT == PKV_F32 ? std::max((size_t)2 * (size_t)a0.vocab * sizeof(uint32_t), runs_row)
                    : runs_row;
  const int rows = (int)std::max<size_t>(1, std::min<size_t>(batch, kExactScratch / per_row));
  const size_t flags = DT == PKV_F32 ? (size_t)batch * sizeof(int32_t) : 0;
  void* p = nullptr;
  hipError_t e = hipMallocAsync(&p, per_row * rows + flags, stream);
  if (e != hipSuccess) return e;
  ExactArgs a = a0;
  a.scratch = static_cast<uint32_t*>(p);
  if (DT == PKV_F32)
    a.fallback = reinterpret_cast<int32_t*>(static_cast<char*>(p) + per_row * rows);
  for (int r0 = 0; r0 < batch; r0 += rows) {
    a.row0 = r0;
    launch_exact_rows<DT, VEC>(a, std::min(rows, batch - r0), stream);
  }
  e = hipGetLastError();
  const hipError_t f = hipFreeAsync(p, stream);
  return e != hipSuccess ? e : f;
}

// Workgroups per row for the split path (1: one workgroup per row).  Rows
// without temperatures are all greedy: one pass, one launch.
int split_groups(int batch, int vocab, const float* temps, int top_k, float top_p) {
  if (!temps || (top_k > 0 && top_k < vocab) || top_p < 1.0f || batch <= 0) return 1;
  int g = 256 / batch;                                 // fill the CUs
  g = std::min(g, kMaxG);
  g = std::min(g, (vocab + kSplitMinChunk - 1) / kSplitMinChunk);  // chunks worth a workgroup
  return std::max(g, 1);
}

template <int DT, bool VEC>
hipError_t launch_dt(const SampleArgs& a, int batch, hipStream_t stream) {
  if (!grid_fits(batch, kST)) return hipErrorInvalidValue;
  const int G = split_groups(batch, a.vocab, a.temps, a.top_k, a.top_p);
  if (G > 1) {
    void* p = nullptr;
    const size_t bytes = (size_t)batch * (sizeof(SplitWs) + (size_t)G * kB2 * sizeof(unsigned));
    if (hipMallocAsync(&p, bytes, stream) == hipSuccess) {
      SplitWs* ws = static_cast<SplitWs*>(p);
      const dim3 grid(G, batch);
      split_max_kernel<DT, VEC><<<grid, kST, 0, stream>>>(a, ws);
      split_mass_kernel<DT, VEC><<<grid, kST, 0, stream>>>(a, ws);
      split_digit_kernel<DT, VEC, false><<<grid, kST, 0, stream>>>(a, ws);
      split_digit_kernel<DT, VEC, true><<<grid, kST, 0, stream>>>(a, ws);
      split_finish_kernel<DT, VEC><<<batch, kST, 0, stream>>>(a, ws, G);
      const hipError_t e = hipGetLastError();
      const hipError_t f = hipFreeAsync(p, stream);
      return e != hipSuccess ? e : f;
    }
    (void)hipGetLastError();  // allocation failed: one workgroup per row
  }
  sample_kernel<DT, VEC><<<batch, kST, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_sample(const void* logits, int dtype, long long row_stride, int batch,
                         int vocab, const float* temperatures, int top_k, float top_p,
                         float r, int32_t* tokens, hipStream_t stream) {
  const long long sb = row_stride * (long long)dtype_bytes(dtype);
  SampleArgs a{static_cast<const char*>(logits), sb, vocab, temperatures, top_k, top_p, r,
               tokens};
  // 16-byte loads when every row starts on a 16-byte boundary
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (batch == 1 || sb % 16 == 0);
  if (dtype == PKV_F32) return vec ? launch_dt<PKV_F32, true>(a, batch, stream)
                                   : launch_dt<PKV_F32, false>(a, batch, stream);
  if (dtype == PKV_BF16) return vec ? launch_dt<PKV_BF16, true>(a, batch, stream)
                                    : launch_dt<PKV_BF16, false>(a, batch, stream);
  return vec ? launch_dt<PKV_F16, true>(a, batch, stream)
             : launch_dt<PKV_F16, false>(a, batch, stream);
}

hipError_t launch_sample_exact(const void* logits, int dtype, long long row_stride, int batch,
                               int vocab, const float* temperatures, int top_k, float top_p,
                               float r, int32_t* tokens, int32_t* routes, hipStream_t stream) {
  const long long sb = row_stride * (long long)dtype_bytes(dtype);
  ExactArgs a{static_cast<const char*>(logits), sb, vocab, temperatures, top_k, top_p, r,
              tokens, nullptr, 0, nullptr, routes};
  const bool vec = (reinterpret_cast<uintptr_t>(logits) & 15u) == 0 && (batch == 1 || sb % 16 == 0);
  if (dtype == PKV_F32) return vec ? launch_exact_dt<PKV_F32, true>(a, batch, stream)
                                   : launch_exact_dt<PKV_F32, false>(a, batch, stream);
  if (dtype == PKV_BF16) return vec ? launch_exact_dt<PKV_BF16, true>(a, batch, stream)
                                    : launch_exact_dt<PKV_BF16, false>(a, batch, stream);
  return vec ? launch_exact_dt<PKV_F16, true>(a, batch, stream)
             : launch_exact_dt<PKV_F16, false>(a, batch, stream);
}

hipError_t launch_expf_glibc(const float* in, float* out, long long n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const long long blocks = std::min<long long>((n + 255) / 256, 65536);
  expf_glibc_kernel<<<(unsigned)blocks, 256, 0, stream>>>(in, out, n);
  return hipGetLastError();
}

}  // namespace pkv
