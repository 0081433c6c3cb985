// pkv_kvcopy.hip -- byte-moving kernels of the paged KV pool (gfx950):
//   append/scatter (KvPool::write, attention.rs:57-83),
//   gather (KvPool::gather_seq, attention.rs:85-97),
//   block copy (copy-on-write) and in-place compaction (no reference
//   counterpart), and a counter-based N(0,1) fill for benchmarks.
//
// All of them are HBM-bound streams of 16-byte vectors: every thread moves
// whole 16-byte chunks, consecutive lanes touch consecutive chunks, and each
// thread issues all of its loads before its stores so that several requests
// are in flight per lane.  Rows are head_dim * elem_bytes >= 128 bytes, so a
// token row is always a whole number of 16-byte chunks.
#include <algorithm>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {
namespace {

constexpr int kCopyThreads = 256;

// One thread per 16-byte chunk of a token row; K and V in the same thread.
__global__ void __launch_bounds__(kCopyThreads)
    append_kernel(u32x4* __restrict__ kp, u32x4* __restrict__ vp,
                  const u32x4* __restrict__ k, const u32x4* __restrict__ v,
                  const int32_t* __restrict__ slots, int n, int row_vec,
                  long long n_slots, uint32_t* err) {
  long long i = (long long)blockIdx.x * kCopyThreads + threadIdx.x;
  if (i >= (long long)n * row_vec) return;
  int t = (int)(i / row_vec);
  int c = (int)(i - (long long)t * row_vec);
  int s = slots[t];
  if (s < 0) return;  // padding token
  if (s >= n_slots) {
    if (c == 0) atomicOr(err, PKV_EBIT_SLOT);
    return;
  }
  u32x4 a = k[i];
  u32x4 b = v[i];
  size_t o = (size_t)s * row_vec + c;
  kp[o] = a;
  vp[o] = b;
}

// out[p] = pool[blocks[p / bs] * bs + p % bs], K and V.
__global__ void __launch_bounds__(kCopyThreads)
    gather_kernel(const u32x4* __restrict__ kp, const u32x4* __restrict__ vp,
                  u32x4* __restrict__ ok, u32x4* __restrict__ ov,
                  const int32_t* __restrict__ table, int len, int row_vec,
                  int bs_log2, int num_blocks, uint32_t* err) {
  long long i = (long long)blockIdx.x * kCopyThreads + threadIdx.x;
  if (i >= (long long)len * row_vec) return;
  int p = (int)(i / row_vec);
  int c = (int)(i - (long long)p * row_vec);
  int blk = table[p >> bs_log2];
  if (blk < 0 || blk >= num_blocks) {
    if (c == 0) atomicOr(err, PKV_EBIT_BLOCK);
    ok[i] = u32x4{0, 0, 0, 0};
    ov[i] = u32x4{0, 0, 0, 0};
    return;
  }
  size_t s = ((size_t)blk << bs_log2) + (p & ((1 << bs_log2) - 1));
  size_t o = s * row_vec + c;
  u32x4 a = kp[o];
  u32x4 b = vp[o];
  ok[i] = a;
  ov[i] = b;
}

// Gather of several sequences: thread per 16-byte chunk of an output row;
// the row's sequence is found by a binary search of cu_lens held in LDS
// (batch <= kVarlenMaxBatch).  Sequence b's row r is its position r.
constexpr int kVarlenMaxBatch = 4096;
__global__ void __launch_bounds__(kCopyThreads)
    gather_varlen_kernel(const u32x4* __restrict__ kp, const u32x4* __restrict__ vp,
                         u32x4* __restrict__ ok, u32x4* __restrict__ ov,
                         const int32_t* __restrict__ tables, int mbps,
                         const int32_t* __restrict__ cu_lens, int batch, int total_rows,
                         int row_vec, int bs_log2, int num_blocks, uint32_t* err) {
  __shared__ int cu[kVarlenMaxBatch + 1];
  for (int i = threadIdx.x; i <= batch; i += kCopyThreads) cu[i] = cu_lens[i];
  __syncthreads();
  const long long i = (long long)blockIdx.x * kCopyThreads + threadIdx.x;
  if (i >= (long long)total_rows * row_vec) return;
  const int row = (int)(i / row_vec);
  const int c = (int)(i - (long long)row * row_vec);
  // last b with cu[b] <= row
  int lo = 0, hi = batch - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  const int p = row - cu[lo];
  const int tb = p >> bs_log2;
  const int blk = tb < mbps && p >= 0 ? tables[(size_t)lo * mbps + tb] : -1;
  if (blk < 0 || blk >= num_blocks) {
    if (c == 0) atomicOr(err, PKV_EBIT_BLOCK);
    ok[i] = u32x4{0, 0, 0, 0};
    ov[i] = u32x4{0, 0, 0, 0};
    return;
  }
  const size_t o = (((size_t)blk << bs_log2) + (p & ((1 << bs_log2) - 1))) * row_vec + c;
  const u32x4 a = kp[o];
  const u32x4 b = vp[o];
  ok[i] = a;
  ov[i] = b;
}

// Copy-on-write: items (pair, K/V slab of a layer, chunk of a block), chunk
// fastest; each workgroup moves items blockIdx.x, + gridDim.x, ... and each
// thread kVecPerThread 16-byte vectors of an item, all loads before the
// stores.  A grid of long-lived workgroups (a few per CU) moves the 2 GiB of
// cfg5's 512 copies 1.45x faster than one short workgroup per item.
constexpr int kVecPerThread = 8;
constexpr int kCopyGrid = 4096;       // workgroups of the copy: 16 per CU
constexpr int kCompactGrid = 16384;   // of the compaction (its items are shorter)

__global__ void __launch_bounds__(kCopyThreads)
    copy_blocks_kernel(char* __restrict__ base, size_t layer_bytes, int block_vec,
                       const int32_t* __restrict__ src, const int32_t* __restrict__ dst,
                       int num_blocks, uint32_t* err, int n, int n_slabs, int chunks) {
  const long long items = (long long)n * n_slabs * chunks;
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int chunk = (int)(it % chunks);
    const long long ps = it / chunks;
    const int slab_i = (int)(ps % n_slabs);
    const int pair = (int)(ps / n_slabs);
    const int s = src[pair], d = dst[pair];
    if (s < 0 || d < 0 || s >= num_blocks || d >= num_blocks) {
      if (threadIdx.x == 0 && slab_i == 0 && chunk == 0) atomicOr(err, PKV_EBIT_BLOCK);
      continue;
    }
    char* slab = base + (size_t)slab_i * layer_bytes;
    const u32x4* from = reinterpret_cast<const u32x4*>(slab) + (size_t)s * block_vec;
    u32x4* to = reinterpret_cast<u32x4*>(slab) + (size_t)d * block_vec;
    const int v0 = chunk * (kCopyThreads * kVecPerThread) + threadIdx.x;
    u32x4 r[kVecPerThread];
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int v = v0 + j * kCopyThreads;
      if (v < block_vec) r[j] = __builtin_nontemporal_load(from + v);
    }
#pragma unroll
    for (int j = 0; j < kVecPerThread; ++j) {
      const int v = v0 + j * kCopyThreads;
      if (v < block_vec) __builtin_nontemporal_store(r[j], to + v);
    }
  }
}

// In-place compaction.  Items (chain, K/V slab of a layer, chunk of a
// block), chunk fastest; each workgroup takes items blockIdx.x, + gridDim.x,
// ...  (cfg5's chains average under two moves, so one workgroup per item
// would be short-lived: long-lived workgroups took its compaction from 24.2
// to 20.5-21.2 ms).  Each thread owns the same byte range of every block in
// its chain and performs the chain's moves in order, so a block's old bytes
// are read (by the same thread, same address) before they are overwritten;
// no cross-thread ordering is needed.  A cycle's first move parks one block
// in registers (dst == -1) and its last move writes it back (src == -1).
// The next move's source is loaded before this move's stores: the blocks of
// a chain are distinct and each is read before it is written, so that read
// never sees a byte this move writes (25.1 -> 24.2 ms).
__global__ void __launch_bounds__(kCopyThreads)
    compact_kernel(char* __restrict__ base, size_t layer_bytes, int block_vec,
                   const int32_t* __restrict__ ops, const int32_t* __restrict__ chain_start,
                   int n_chains, int n_slabs, int chunks) {
  const long long items = (long long)n_chains * n_slabs * chunks;
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int chunk = (int)(it % chunks);
    const long long cs = it / chunks;
    const int slab_i = (int)(cs % n_slabs);
    const int c = (int)(cs / n_slabs);
    const int o0 = chain_start[c], o1 = chain_start[c + 1];
    u32x4* pool = reinterpret_cast<u32x4*>(base + (size_t)slab_i * layer_bytes);
    const int v0 = chunk * (kCopyThreads * kVecPerThread) + threadIdx.x;
    u32x4 held[kVecPerThread];
    u32x4 ra[kVecPerThread], rb[kVecPerThread];
    auto load_src = [&](int o, u32x4 (&r)[kVecPerThread]) __attribute__((always_inline)) {
      const int s = ops[2 * o];
      if (s < 0) return;  // the write-back of a cycle comes from `held`
#pragma unroll
      for (int j = 0; j < kVecPerThread; ++j) {
        const int v = v0 + j * kCopyThreads;
        if (v < block_vec) r[j] = __builtin_nontemporal_load(pool + (size_t)s * block_vec + v);
      }
    };
    if (o0 < o1) load_src(o0, ra);
    for (int o = o0; o < o1; ++o) {
      const int s = ops[2 * o], d = ops[2 * o + 1];
      if (o + 1 < o1) load_src(o + 1, rb);  // next source: never a block this move writes
#pragma unroll
      for (int j = 0; j < kVecPerThread; ++j) {
        const int v = v0 + j * kCopyThreads;
        if (v < block_vec) {
          const u32x4 x = s >= 0 ? ra[j] : held[j];
          if (d >= 0)
            __builtin_nontemporal_store(x, pool + (size_t)d * block_vec + v);
          else
            held[j] = x;
        }
      }
#pragma unroll
      for (int j = 0; j < kVecPerThread; ++j) ra[j] = rb[j];
    }
  }
}

// SplitMix64 finaliser (Steele, Lea, Flood 2014) as a counter-based hash.
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// N(0,1) by Box-Muller from two 32-bit uniforms of one hash.  No fused
// multiply-adds, so the value does not depend on the code around a call.
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t idx) {
#pragma clang fp contract(off)
  uint64_t h = mix64(seed + 0x9e3779b97f4a7c15ull * (idx + 1));
  float u1 = ((uint32_t)(h >> 40) + 1) * (1.0f / 16777217.0f);  // (0,1]
  float u2 = (uint32_t)(h & 0xffffffu) * (1.0f / 16777216.0f);
  return sqrtf(-2.0f * __logf(u1)) * __cosf(6.28318530718f * u2);
}

// The 16-byte chunk `chunk` of a slab filled with seed (4 or 8 elements of
// normal_at, rounded to DT).  One out-of-line body serves the fill and its
// verification, so both produce the same bits.
template <int DT>
__device__ __noinline__ u32x4 normal_chunk(uint64_t seed, size_t chunk) {
  u32x4 w;
  if constexpr (DT == PKV_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(normal_at(seed, chunk * 4 + i));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = normal_at(seed, chunk * 8 + 2 * i);
      float b = normal_at(seed, chunk * 8 + 2 * i + 1);
      uint32_t lo = DT == PKV_BF16 ? f32_to_bf16_bits(a) : f32_to_f16_bits(a);
      uint32_t hi = DT == PKV_BF16 ? f32_to_bf16_bits(b) : f32_to_f16_bits(b);
      w[i] = lo | (hi << 16);
    }
  }
  return w;
}

template <int DT>
__global__ void __launch_bounds__(kCopyThreads)
    fill_normal_kernel(char* __restrict__ base, size_t n_elems, uint64_t seed) {
  // Each thread writes one 16-byte chunk (4 or 8 elements).
  constexpr int EPL = DT == PKV_F32 ? 4 : 8;
  size_t chunk = (size_t)blockIdx.x * kCopyThreads + threadIdx.x;
  size_t stride = (size_t)gridDim.x * kCopyThreads;
  for (; chunk * EPL < n_elems; chunk += stride)
    reinterpret_cast<u32x4*>(base)[chunk] = normal_chunk<DT>(seed, chunk);
}

// Verification of a filled pool after blocks moved: entry i says that block
// blocks[i] should hold, in every layer's K and V, the bytes the fill wrote
// into block origin[i].  Items (entry, K/V slab of a layer) are spread over
// a grid of long-lived workgroups; each counts the 16-byte chunks that
// differ and adds its count to *count once.  An id out of range sets the
// block error bit and counts the item's chunks as mismatches.
template <int DT>
__global__ void __launch_bounds__(kCopyThreads)
    verify_normal_kernel(const char* __restrict__ base, size_t layer_bytes, int block_vec,
                         int num_blocks, const int32_t* __restrict__ blocks,
                         const int32_t* __restrict__ origin, int n, int n_slabs, uint64_t seed,
                         unsigned long long* count, uint32_t* err) {
  __shared__ unsigned long long wg_count;
  if (threadIdx.x == 0) wg_count = 0;
  __syncthreads();
  unsigned long long bad = 0;
  const long long items = (long long)n * n_slabs;
  for (long long it = blockIdx.x; it < items; it += gridDim.x) {
    const int i = (int)(it / n_slabs);
    const int slab = (int)(it % n_slabs);
    const int b = blocks[i], o = origin[i];
    if (b < 0 || o < 0 || b >= num_blocks || o >= num_blocks) {
      if (threadIdx.x == 0) {
        atomicOr(err, PKV_EBIT_BLOCK);
        bad += block_vec;
      }
      continue;
    }
    const u32x4* got =
        reinterpret_cast<const u32x4*>(base + (size_t)slab * layer_bytes) + (size_t)b * block_vec;
    // chunk index of the origin block's bytes in the whole slab
    const size_t c0 = ((size_t)slab * num_blocks + o) * block_vec;
    for (int v = threadIdx.x; v < block_vec; v += kCopyThreads) {
      const u32x4 x = __builtin_nontemporal_load(got + v);
      const u32x4 w = normal_chunk<DT>(seed, c0 + v);
      bad += (x[0] != w[0]) | (x[1] != w[1]) | (x[2] != w[2]) | (x[3] != w[3]);
    }
  }
  if (bad) atomicAdd(&wg_count, bad);
  __syncthreads();
  if (threadIdx.x == 0 && wg_count) atomicAdd(count, wg_count);
}

// Read-only stream over blocks[i] in every layer's K and V: items (entry,
// K/V slab of a layer, 2048-vector chunk of a block), one item per wave and
// step over a grid of long-lived workgroups.  Each lane issues its 32
// sixteen-byte non-temporal loads before it adds any of them up, so a wave
// keeps a whole 32 KiB block slab in flight (three waves per SIMD, 384 KiB
// per CU).  The 32-bit words are summed (mod 2^64) into *sum,
// one atomic per workgroup: the loads cannot be dropped, and the sum checks the
// bytes.  An id out of range sets the block error bit and is skipped.
constexpr int kReadVec = 32;                    // loads per lane per item
constexpr int kReadChunk = kWave * kReadVec;    // 16-byte vectors per item
__global__ void __launch_bounds__(kCopyThreads)
    read_blocks_kernel(const char* __restrict__ base, size_t layer_bytes, int block_vec,
                       int num_blocks, const int32_t* __restrict__ blocks, int n, int n_slabs,
                       int chunks, unsigned long long* sum, uint32_t* err) {
  const int lane = threadIdx.x & (kWave - 1);
  const long long waves = (long long)gridDim.x * (kCopyThreads / kWave);
  const long long w0 = (long long)blockIdx.x * (kCopyThreads / kWave) + (threadIdx.x >> 6);
  unsigned long long acc = 0;
  const long long items = (long long)n * n_slabs * chunks;
  for (long long it = w0; it < items; it += waves) {
    const int chunk = (int)(it % chunks);
    const long long es = it / chunks;
    const int slab = (int)(es % n_slabs);
    const int b = blocks[es / n_slabs];
    if (b < 0 || b >= num_blocks) {
      if (lane == 0 && slab == 0 && chunk == 0) atomicOr(err, PKV_EBIT_BLOCK);
      continue;
    }
    const u32x4* from = reinterpret_cast<const u32x4*>(base + (size_t)slab * layer_bytes) +
                        (size_t)b * block_vec + chunk * kReadChunk + lane;
    const int left = block_vec - chunk * kReadChunk;  // vectors of this chunk
    if (left >= kReadChunk) {
      u32x4 r[kReadVec];
#pragma unroll
      for (int j = 0; j < kReadVec; ++j) r[j] = __builtin_nontemporal_load(from + j * kWave);
#pragma unroll
      for (int j = 0; j < kReadVec; ++j) {
        const unsigned long long lo = (unsigned long long)r[j][0] + r[j][1];
        const unsigned long long hi = (unsigned long long)r[j][2] + r[j][3];
        acc += lo + hi;
      }
    } else {  // a block's last, partial chunk (or a block under 32 KiB)
      for (int j = 0; j * kWave < left; ++j) {
        if (j * kWave + lane >= left) break;
        const u32x4 x = __builtin_nontemporal_load(from + j * kWave);
        acc += (unsigned long long)x[0] + x[1] + x[2] + x[3];
      }
    }
  }
  __shared__ unsigned long long wg_sum;
  if (threadIdx.x == 0) wg_sum = 0;
  __syncthreads();
  if (acc) atomicAdd(&wg_sum, acc);
  __syncthreads();
  if (threadIdx.x == 0 && wg_sum) atomicAdd(sum, wg_sum);
}

int ilog2(int x) {
  int r = 0;
  while ((1 << r) < x) ++r;
  return r;
}

}  // namespace

hipError_t launch_append(const pkv_pool* p, int layer, const void* k,
                         const void* v, const int32_t* slots, int n,
                         hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  int row_vec = (int)(p->row_bytes * p->n_kv_head / 16);
  long long total = (long long)n * row_vec;
  if (!grid_fits((total + kCopyThreads - 1) / kCopyThreads, kCopyThreads))
    return hipErrorInvalidValue;
  unsigned grid = (unsigned)((total + kCopyThreads - 1) / kCopyThreads);
  append_kernel<<<grid, kCopyThreads, 0, stream>>>(
      reinterpret_cast<u32x4*>(p->layer_k(layer)),
      reinterpret_cast<u32x4*>(p->layer_v(layer)),
      reinterpret_cast<const u32x4*>(k), reinterpret_cast<const u32x4*>(v),
      slots, n, row_vec, (long long)p->num_blocks * p->block_size, p->err);
  return hipGetLastError();
}

hipError_t launch_gather(const pkv_pool* p, int layer, const int32_t* table,
                         int len, void* out_k, void* out_v,
                         hipStream_t stream) {
  if (len <= 0) return hipSuccess;
  int row_vec = (int)(p->row_bytes * p->n_kv_head / 16);
  long long total = (long long)len * row_vec;
  if (!grid_fits((total + kCopyThreads - 1) / kCopyThreads, kCopyThreads))
    return hipErrorInvalidValue;
  unsigned grid = (unsigned)((total + kCopyThreads - 1) / kCopyThreads);
  gather_kernel<<<grid, kCopyThreads, 0, stream>>>(
      reinterpret_cast<const u32x4*>(p->layer_k(layer)),
      reinterpret_cast<const u32x4*>(p->layer_v(layer)),
      reinterpret_cast<u32x4*>(out_k), reinterpret_cast<u32x4*>(out_v), table,
      len, row_vec, ilog2(p->block_size), p->num_blocks, p->err);
  return hipGetLastError();
}

hipError_t launch_gather_varlen(const pkv_pool* p, int layer, const int32_t* tables, int mbps,
                                const int32_t* cu_lens, int batch, int total_rows, void* out_k,
                                void* out_v, hipStream_t stream) {
  if (total_rows <= 0 || batch <= 0) return hipSuccess;
  if (batch > kVarlenMaxBatch) return hipErrorInvalidValue;
  const int row_vec = (int)(p->row_bytes * p->n_kv_head / 16);
  const long long total = (long long)total_rows * row_vec;
  if (!grid_fits((total + kCopyThreads - 1) / kCopyThreads, kCopyThreads))
    return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((total + kCopyThreads - 1) / kCopyThreads);
  gather_varlen_kernel<<<grid, kCopyThreads, 0, stream>>>(
      reinterpret_cast<const u32x4*>(p->layer_k(layer)),
      reinterpret_cast<const u32x4*>(p->layer_v(layer)), reinterpret_cast<u32x4*>(out_k),
      reinterpret_cast<u32x4*>(out_v), tables, mbps, cu_lens, batch, total_rows, row_vec,
      ilog2(p->block_size), p->num_blocks, p->err);
  return hipGetLastError();
}

hipError_t launch_copy_blocks(const pkv_pool* p, const int32_t* src,
                              const int32_t* dst, int n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int block_vec = (int)(p->block_bytes / 16);
  const int per_block = kCopyThreads * kVecPerThread;
  const int chunks = (block_vec + per_block - 1) / per_block;
  const long long items = (long long)n * 2 * p->n_layers * chunks;
  const unsigned grid = (unsigned)(items < kCopyGrid ? items : kCopyGrid);
  copy_blocks_kernel<<<grid, kCopyThreads, 0, stream>>>(p->base, p->layer_bytes, block_vec, src,
                                                        dst, p->num_blocks, p->err, n,
                                                        2 * p->n_layers, chunks);
  return hipGetLastError();
}

hipError_t launch_compact(const pkv_pool* p, const int32_t* ops,
                          const int32_t* chain_start, int n_chains,
                          hipStream_t stream) {
  if (n_chains <= 0) return hipSuccess;
  int block_vec = (int)(p->block_bytes / 16);
  int per_block = kCopyThreads * kVecPerThread;
  const int chunks = (block_vec + per_block - 1) / per_block;
  const long long items = (long long)n_chains * 2 * p->n_layers * chunks;
  const unsigned grid = (unsigned)(items < kCompactGrid ? items : kCompactGrid);
  compact_kernel<<<grid, kCopyThreads, 0, stream>>>(
      p->base, p->layer_bytes, block_vec, ops, chain_start, n_chains, 2 * p->n_layers, chunks);
  return hipGetLastError();
}

hipError_t launch_fill_normal(const pkv_pool* p, uint64_t seed,
                              hipStream_t stream) {
  size_t total_bytes = p->layer_bytes * 2 * (size_t)p->n_layers;
  size_t n_elems = total_bytes / p->elem_bytes;
  unsigned grid = 8192;
  switch (p->dtype) {
    case PKV_F32:
      fill_normal_kernel<PKV_F32><<<grid, kCopyThreads, 0, stream>>>(p->base, n_elems, seed);
      break;
    case PKV_F16:
      fill_normal_kernel<PKV_F16><<<grid, kCopyThreads, 0, stream>>>(p->base, n_elems, seed);
      break;
    default:
      fill_normal_kernel<PKV_BF16><<<grid, kCopyThreads, 0, stream>>>(p->base, n_elems, seed);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_verify_normal(const pkv_pool* p, uint64_t seed, const int32_t* blocks,
                                const int32_t* origin, int n, unsigned long long* count,
                                hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int block_vec = (int)(p->block_bytes / 16);
  const int n_slabs = 2 * p->n_layers;
  const long long items = (long long)n * n_slabs;
  const unsigned grid = (unsigned)std::min<long long>(items, kCompactGrid);
  switch (p->dtype) {
    case PKV_F32:
      verify_normal_kernel<PKV_F32><<<grid, kCopyThreads, 0, stream>>>(
          p->base, p->layer_bytes, block_vec, p->num_blocks, blocks, origin, n, n_slabs, seed,
          count, p->err);
      break;
    case PKV_F16:
      verify_normal_kernel<PKV_F16><<<grid, kCopyThreads, 0, stream>>>(
          p->base, p->layer_bytes, block_vec, p->num_blocks, blocks, origin, n, n_slabs, seed,
          count, p->err);
      break;
    default:
      verify_normal_kernel<PKV_BF16><<<grid, kCopyThreads, 0, stream>>>(
          p->base, p->layer_bytes, block_vec, p->num_blocks, blocks, origin, n, n_slabs, seed,
          count, p->err);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_read_blocks(const pkv_pool* p, const int32_t* blocks, int n,
                              unsigned long long* sum, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int block_vec = (int)(p->block_bytes / 16);
  const int chunks = (block_vec + kReadChunk - 1) / kReadChunk;
  const long long items = (long long)n * 2 * p->n_layers * chunks;
  // three workgroups (12 waves, 384 KiB of loads) per CU: what the
  // registers hold (158 per lane, three waves per SIMD)
  const long long waves_per_wg = kCopyThreads / kWave;
  const long long cap = p->n_cu > 0 ? 3LL * p->n_cu : kCopyGrid;
  const unsigned grid =
      (unsigned)std::min<long long>((items + waves_per_wg - 1) / waves_per_wg, cap);
  read_blocks_kernel<<<grid, kCopyThreads, 0, stream>>>(p->base, p->layer_bytes, block_vec,
                                                        p->num_blocks, blocks, n, 2 * p->n_layers,
                                                        chunks, sum, p->err);
  return hipGetLastError();
}

}  // namespace pkv
