// pkv_rope.hip -- rotary position embedding of the decode/prefill rows
// (crates/ai-engine-candle/src/paged/rope.rs; applied per row in the decode
// step, transformer.rs:252-269, and to the prompt in prefill_seq, :160-167).
//
// Tables: Rope::new (rope.rs:14-23) computes theta_i = 1 / base^(2i / dim)
// in f32, angle = (float)p * theta_i (a K = 1 matmul: one rounded product)
// and cos/sin in f32.  They are computed here on the host with the same f32
// operations (libm powf/cosf/sinf) and uploaded once; they are position
// tables, not part of the per-step work.
//
// Rotation: candle's rotate-half rope (rope.rs:38-42): for the halves
// x1 = x[i], x2 = x[i + d/2] of each head row, out[i] = x1 cos - x2 sin and
// out[i + d/2] = x1 sin + x2 cos, each product rounded in f32 (contraction
// off, as the reference's scalar loop computes it), then rounded to the
// output dtype.
#include <cmath>

#include "pkv_device.h"
#include "pkv_internal.h"

namespace pkv {

void rope_tables_host(int rope_dim, float freq_base, int max_seq, float* cos_t,
                      float* sin_t) {
  const int half = rope_dim / 2;
  for (int i = 0; i < half; ++i) {
    const float theta = 1.0f / powf(freq_base, 2.0f * (float)i / (float)rope_dim);
    for (int p = 0; p < max_seq; ++p) {
      const float f = (float)p * theta;
      cos_t[(size_t)p * half + i] = cosf(f);
      sin_t[(size_t)p * half + i] = sinf(f);
    }
  }
}

namespace {

constexpr int kRopeThreads = 256;

// Four consecutive elements of a row as floats / back to the row's dtype.
__device__ __forceinline__ f32x4 load4(const char* row, int elem, int dt) {
  if (dt == PKV_F32) return *reinterpret_cast<const f32x4*>(row + (size_t)elem * 4);
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 w = *reinterpret_cast<const u32x2*>(row + (size_t)elem * 2);
  if (dt == PKV_BF16) return f32x4{bf16lo(w[0]), bf16hi(w[0]), bf16lo(w[1]), bf16hi(w[1])};
  return f32x4{f16lo(w[0]), f16hi(w[0]), f16lo(w[1]), f16hi(w[1])};
}
__device__ __forceinline__ void store4(char* row, int elem, int dt, const f32x4& x) {
  if (dt == PKV_F32) {
    *reinterpret_cast<f32x4*>(row + (size_t)elem * 4) = x;
    return;
  }
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  uint32_t h[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) h[i] = dt == PKV_BF16 ? f32_to_bf16_bits(x[i]) : f32_to_f16_bits(x[i]);
  *reinterpret_cast<u32x2*>(row + (size_t)elem * 2) = u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
}

// One thread per (token, head, 4 element pairs).
__global__ void __launch_bounds__(kRopeThreads)
    rope_apply_kernel(const char* __restrict__ x, int in_dt, char* out, int out_dt,
                      const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                      const int32_t* __restrict__ positions, int n_tokens, int n_head,
                      int d, int max_seq, uint32_t* err) {
  const int half = d / 2;
  const int groups = half / 4;
  const long long i = (long long)blockIdx.x * kRopeThreads + threadIdx.x;
  if (i >= (long long)n_tokens * n_head * groups) return;
  const int gi = (int)(i % groups);
  const long long row = i / groups;  // token * n_head + head
  const int t = (int)(row / n_head);
  const int pos = positions[t];
  if (pos < 0 || pos >= max_seq) {
    if (gi == 0) atomicOr(err, PKV_EBIT_POSITION);
    return;
  }
  const int e = 4 * gi;
  const size_t ib = in_dt == PKV_F32 ? 4 : 2, ob = out_dt == PKV_F32 ? 4 : 2;
  const char* xr = x + (size_t)row * d * ib;
  char* orow = out + (size_t)row * d * ob;
  const f32x4 x1 = load4(xr, e, in_dt);
  const f32x4 x2 = load4(xr, e + half, in_dt);
  const f32x4 c = *reinterpret_cast<const f32x4*>(cos_t + (size_t)pos * half + e);
  const f32x4 s = *reinterpret_cast<const f32x4*>(sin_t + (size_t)pos * half + e);
  f32x4 o1, o2;
  {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      o1[j] = x1[j] * c[j] - x2[j] * s[j];
      o2[j] = x1[j] * s[j] + x2[j] * c[j];
    }
  }
  store4(orow, e, out_dt, o1);
  store4(orow, e + half, out_dt, o2);
}

// Prefill glue in one pass (prefill_seq, transformer.rs:160-174): rows of
// token t are its n_kv k rows (rotated, stored at pool slot slots[t]), its
// n_kv v rows (stored as they are) and, when q is given, its n_head q rows
// (rotated, stored to q_out); all converted from in_dt to the pool dtype.
// One thread per (token, row, 4 element pairs).  slots[t] < 0 is a padding
// token: its k/v rows are skipped, its q rows still rotated.
__global__ void __launch_bounds__(kRopeThreads)
    append_rope_kernel(const char* __restrict__ k, const char* __restrict__ v,
                       const char* q, char* q_out, int in_dt, char* __restrict__ kp,
                       char* __restrict__ vp, int pool_dt, const int32_t* __restrict__ slots,
                       long long n_slots, const float* __restrict__ cos_t,
                       const float* __restrict__ sin_t, const int32_t* __restrict__ positions,
                       int n_tokens, int n_kv, int n_q, int d, int max_seq, uint32_t* err) {
  const int half = d / 2;
  const int groups = half / 4;
  const int rows = 2 * n_kv + n_q;
  const long long i = (long long)blockIdx.x * kRopeThreads + threadIdx.x;
  if (i >= (long long)n_tokens * rows * groups) return;
  const int gi = (int)(i % groups);
  const long long tr = i / groups;
  const int t = (int)(tr / rows);
  const int r = (int)(tr - (long long)t * rows);
  const int e = 4 * gi;
  const size_t ib = in_dt == PKV_F32 ? 4 : 2, pb = pool_dt == PKV_F32 ? 4 : 2;
  const char* src;
  char* dst;
  bool rotate = true;
  if (r < 2 * n_kv) {
    const int s = slots[t];
    if (s < 0) return;
    if (s >= n_slots) {
      if (gi == 0) atomicOr(err, PKV_EBIT_SLOT);
      return;
    }
    const int h = r < n_kv ? r : r - n_kv;
    const size_t in_row = (size_t)t * n_kv + h;
    const size_t pool_row = (size_t)s * n_kv + h;
    if (r < n_kv) {
      src = k + in_row * d * ib;
      dst = kp + pool_row * d * pb;
    } else {
      src = v + in_row * d * ib;
      dst = vp + pool_row * d * pb;
      rotate = false;
    }
  } else {
    const size_t row = (size_t)t * n_q + (r - 2 * n_kv);
    src = q + row * d * ib;
    dst = q_out + row * d * pb;
  }
  f32x4 x1 = load4(src, e, in_dt);
  f32x4 x2 = load4(src, e + half, in_dt);
  if (rotate) {
    const int pos = positions[t];
    if (pos < 0 || pos >= max_seq) {
      if (gi == 0) atomicOr(err, PKV_EBIT_POSITION);
      return;
    }
    const f32x4 c = *reinterpret_cast<const f32x4*>(cos_t + (size_t)pos * half + e);
    const f32x4 s = *reinterpret_cast<const f32x4*>(sin_t + (size_t)pos * half + e);
    f32x4 o1, o2;
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        o1[j] = x1[j] * c[j] - x2[j] * s[j];
        o2[j] = x1[j] * s[j] + x2[j] * c[j];
      }
    }
    x1 = o1;
    x2 = o2;
  }
  store4(dst, e, pool_dt, x1);
  store4(dst, e + half, pool_dt, x2);
}

}  // namespace

hipError_t launch_append_rope(const pkv_pool* p, int layer, const pkv_rope* r,
                              const int32_t* positions, int in_dtype, const void* k,
                              const void* v, const int32_t* slots, int n_tokens, const void* q,
                              void* q_out, int n_head, hipStream_t stream) {
  const int n_q = q ? n_head : 0;
  const long long threads =
      (long long)n_tokens * (2 * p->n_kv_head + n_q) * (p->head_dim / 8);
  if (threads <= 0) return hipSuccess;
  if (!grid_fits((threads + kRopeThreads - 1) / kRopeThreads, kRopeThreads))
    return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((threads + kRopeThreads - 1) / kRopeThreads);
  append_rope_kernel<<<grid, kRopeThreads, 0, stream>>>(
      static_cast<const char*>(k), static_cast<const char*>(v), static_cast<const char*>(q),
      static_cast<char*>(q_out), in_dtype, p->layer_k(layer), p->layer_v(layer), p->dtype, slots,
      (long long)p->num_blocks * p->block_size, r->cos, r->sin, positions, n_tokens,
      p->n_kv_head, n_q, p->head_dim, r->max_seq, p->err);
  return hipGetLastError();
}

hipError_t launch_rope_apply(const pkv_rope* r, const void* x, int in_dtype, void* out,
                             int out_dtype, const int32_t* positions, int n_tokens, int n_head,
                             hipStream_t stream) {
  const long long threads = (long long)n_tokens * n_head * (r->rope_dim / 8);
  if (threads <= 0) return hipSuccess;
  if (!grid_fits((threads + kRopeThreads - 1) / kRopeThreads, kRopeThreads))
    return hipErrorInvalidValue;
  const unsigned grid = (unsigned)((threads + kRopeThreads - 1) / kRopeThreads);
  rope_apply_kernel<<<grid, kRopeThreads, 0, stream>>>(
      static_cast<const char*>(x), in_dtype, static_cast<char*>(out), out_dtype, r->cos, r->sin,
      positions, n_tokens, n_head, r->rope_dim, r->max_seq, r->err);
  return hipGetLastError();
}

}  // namespace pkv
