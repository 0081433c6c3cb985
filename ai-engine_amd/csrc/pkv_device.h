// pkv_device.h -- device-side helpers for the gfx950 kernels: vector types,
// element conversions, wave64 reductions on DPP and the MFMA wrappers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../include/pagedkv.h"

namespace pkv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// ---- element conversions (exact widening; RNE narrowing) ----------------
__device__ __forceinline__ float bf16lo(uint32_t w) {
  return __uint_as_float(w << 16);
}
__device__ __forceinline__ float bf16hi(uint32_t w) {
  return __uint_as_float(w & 0xffff0000u);
}
__device__ __forceinline__ float f16lo(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
__device__ __forceinline__ float f16hi(uint32_t w) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (u >> 16) | 0x40u;  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// Widen the 16-byte chunk `c` (EPL elements of storage type DT) to floats.
template <int DT, int EPL>
__device__ __forceinline__ void widen16(const u32x4& c, float (&x)[EPL]) {
  if constexpr (DT == PKV_F32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(c[i]);
  } else if constexpr (DT == PKV_BF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = bf16lo(c[i]);
      x[2 * i + 1] = bf16hi(c[i]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = f16lo(c[i]);
      x[2 * i + 1] = f16hi(c[i]);
    }
  }
}

// ---- DPP row (16-lane) all-reductions -----------------------------------
// row_ror:n rotates within each row of 16 lanes; combining with rotations
// by 8, 4, 2, 1 leaves the row's full reduction in every lane of the row.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(
      0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}
__device__ __forceinline__ float row_max16(float x) {
  x = fmaxf(x, dpp_f<0x128>(x));
  x = fmaxf(x, dpp_f<0x124>(x));
  x = fmaxf(x, dpp_f<0x122>(x));
  x = fmaxf(x, dpp_f<0x121>(x));
  return x;
}
__device__ __forceinline__ float row_sum16(float x) {
  x += dpp_f<0x128>(x);
  x += dpp_f<0x124>(x);
  x += dpp_f<0x122>(x);
  x += dpp_f<0x121>(x);
  return x;
}

// Sums across rows of 16 lanes with the gfx950 permlane swaps (VALU, no
// LDS round trip): given the same register twice, the two results hold each
// lane's own value and its partner's (lane ^ 16, resp. lane ^ 32).
__device__ __forceinline__ float swap16_sum(float x) {
  auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float swap32_sum(float x) {
  auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x),
                                            false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum of x over the lanes l' with l' % CH == l % CH (CH a power of two in
// [4, 64]); every lane receives the sum.
template <int CH>
__device__ __forceinline__ float group_sum(float x) {
  if constexpr (CH <= 4) x += dpp_f<0x124>(x);  // row_ror:4
  if constexpr (CH <= 8) x += dpp_f<0x128>(x);  // row_ror:8
  if constexpr (CH <= 16) x = swap16_sum(x);
  if constexpr (CH <= 32) x = swap32_sum(x);
  return x;
}

__device__ __forceinline__ float readlane_f(float x, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), lane));
}
__device__ __forceinline__ int readlane_i(int x, int lane) {
  return __builtin_amdgcn_readlane(x, lane);
}
__device__ __forceinline__ float shfl_xor_f(float x, int mask) {
  int lane = __lane_id();
  return __int_as_float(
      __builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(x)));
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

// ---- MFMA 16x16 tiles -----------------------------------------------------
// D[m][n] += sum_k A[m][k] B[k][n]; lane l supplies row m = l % 16 of A and
// column n = l % 16 of B for the k-slice owned by lane group l / 16, and
// receives D[4 * (l / 16) + j][l % 16] in register j.
// One 16-byte fragment per lane covers 32 (16-bit types) or, via four
// instructions, 16 (f32) values of k.
template <int DT>
__device__ __forceinline__ void mfma_frag(const u32x4& a, const u32x4& b,
                                          f32x4& acc) {
  if constexpr (DT == PKV_BF16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), acc, 0,
        0, 0);
  } else if constexpr (DT == PKV_F16) {
    acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), acc, 0, 0,
        0);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(
          __uint_as_float(a[i]), __uint_as_float(b[i]), acc, 0, 0, 0);
  }
}

__device__ __forceinline__ u32x4 ld16(const void* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
// Non-temporal 16-byte load for data read once per launch (the K/V
// stream): the L2 evicts such lines first, which keeps the small partial
// results a kernel writes resident instead of sending them to HBM in the
// middle of the read stream.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(void* p, const u32x4& v) {
  *reinterpret_cast<u32x4*>(p) = v;
}

}  // namespace pkv
