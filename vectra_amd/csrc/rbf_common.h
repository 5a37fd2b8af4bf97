// Device-side helpers shared by the RBF-attention kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "vectra_rbf.h"

namespace vectra {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kWave = 64;

// Everything a kernel needs, passed by value as the kernel argument.
// Strides are in elements; sizes are 64-bit so any tensor the caller can
// address is indexed without overflow.
struct Problem {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  const void* scale;
  const void* bias;
  int32_t scale_dtype;
  int32_t bias_dtype;
  int64_t B, H, Nq, Nk, D, Dv;
  int64_t sq[4], sk[4], sv[4], so[4];
  int64_t ssb, ssh;
  int64_t sbb, sbh, sbn;
  int64_t total_rows;  // B * H * Nq
};

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// Loads element i of a buffer whose dtype is only known at run time
// (scale and key_bias accept any floating dtype) and converts it to fp32.
__device__ __forceinline__ float load_any(const void* p, int64_t i, int32_t dtype) {
  switch (dtype) {
    case VECTRA_F32:
      return static_cast<const float*>(p)[i];
    case VECTRA_F16:
      return static_cast<float>(static_cast<const _Float16*>(p)[i]);
    case VECTRA_BF16:
      return bf16_bits_to_float(static_cast<const uint16_t*>(p)[i]);
    default:
      return static_cast<float>(static_cast<const double*>(p)[i]);
  }
}

template <typename T>
__device__ __forceinline__ float to_float(T x);
template <>
__device__ __forceinline__ float to_float<float>(float x) { return x; }
template <>
__device__ __forceinline__ float to_float<_Float16>(_Float16 x) { return static_cast<float>(x); }
template <>
__device__ __forceinline__ float to_float<__bf16>(__bf16 x) { return static_cast<float>(x); }

// fp32 -> T with round-to-nearest-even (the conversion torch's .to() uses).
template <typename T>
__device__ __forceinline__ T from_float(float x) { return static_cast<T>(x); }

// ---------------------------------------------------------- 16-byte chunks

// Number of elements of T in one 128-bit load.
template <typename T>
struct Vec {
  static constexpr int kN = 16 / sizeof(T);
};

// Converts one 128-bit chunk of T into fp32 values.
template <typename T>
__device__ __forceinline__ void unpack(const uint4& r, float* f);

template <>
__device__ __forceinline__ void unpack<float>(const uint4& r, float* f) {
  f[0] = __uint_as_float(r.x);
  f[1] = __uint_as_float(r.y);
  f[2] = __uint_as_float(r.z);
  f[3] = __uint_as_float(r.w);
}

template <>
__device__ __forceinline__ void unpack<__bf16>(const uint4& r, float* f) {
  const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

template <>
__device__ __forceinline__ void unpack<_Float16>(const uint4& r, float* f) {
  typedef _Float16 h8 __attribute__((ext_vector_type(8)));
  const h8 h = __builtin_bit_cast(h8, r);
#pragma unroll
  for (int i = 0; i < 8; ++i) f[i] = static_cast<float>(h[i]);
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *static_cast<const uint4*>(p);
}

// Writes N fp32 values as OutT to a 16-byte-aligned address.
template <typename OutT, int N>
__device__ __forceinline__ void store_chunk(OutT* dst, const float* f) {
  OutT tmp[N];
#pragma unroll
  for (int i = 0; i < N; ++i) tmp[i] = from_float<OutT>(f[i]);
  constexpr int kBytes = N * static_cast<int>(sizeof(OutT));
  static_assert(kBytes % 8 == 0, "chunk must be a multiple of 8 bytes");
  if constexpr (kBytes % 16 == 0) {
#pragma unroll
    for (int i = 0; i < kBytes / 16; ++i)
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(tmp)[i];
  } else {
#pragma unroll
    for (int i = 0; i < kBytes / 8; ++i)
      reinterpret_cast<uint2*>(dst)[i] = reinterpret_cast<const uint2*>(tmp)[i];
  }
}

// ------------------------------------------------------- cross-lane moves
//
// DPP controls (GFX9): quad_perm [1,0,3,2] = 0xB1 (lane ^ 1),
// quad_perm [2,3,0,1] = 0x4E (lane ^ 2), row_ror:4 = 0x124, row_ror:8 =
// 0x128 (lane ^ 8 within a 16-lane row), row_half_mirror = 0x141,
// row_mirror = 0x140.

template <int kCtrl>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(
      __builtin_amdgcn_mov_dpp(__float_as_int(x), kCtrl, 0xf, 0xf, true));
}

__device__ __forceinline__ float xor_lanes(float x, int mask) {
  return __shfl_xor(x, mask, kWave);
}

struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// All-reduce over the low lane bits 1 .. kGroup/2 (groups of kGroup adjacent
// lanes; kGroup a power of two <= 16).  Mirrors are valid because the lower
// bits are already reduced when they run.
template <int kGroup, typename Op>
__device__ __forceinline__ float reduce_low(float x, Op op) {
  if constexpr (kGroup >= 2) x = op(x, dpp<0xB1>(x));
  if constexpr (kGroup >= 4) x = op(x, dpp<0x4E>(x));
  if constexpr (kGroup >= 8) x = op(x, dpp<0x141>(x));
  if constexpr (kGroup >= 16) x = op(x, dpp<0x140>(x));
  return x;
}

// All-reduce over lane bits kFrom .. 32 (kFrom a power of two), leaving
// values that differ in the bits below kFrom apart.
template <int kFrom, typename Op>
__device__ __forceinline__ float reduce_high(float x, Op op) {
  if constexpr (kFrom <= 1) x = op(x, dpp<0xB1>(x));
  if constexpr (kFrom <= 2) x = op(x, dpp<0x4E>(x));
  if constexpr (kFrom <= 4) {
    // Bits 4 and 8 together: rotate by 4 then by 8 within each row.
    x = op(x, dpp<0x124>(x));
    x = op(x, dpp<0x128>(x));
  } else if constexpr (kFrom == 8) {
    x = op(x, dpp<0x128>(x));
  }
  if constexpr (kFrom <= 16) x = op(x, xor_lanes(x, 16));
  x = op(x, xor_lanes(x, 32));
  return x;
}

template <typename Op>
__device__ __forceinline__ float reduce_wave(float x, Op op) {
  return reduce_high<1>(x, op);
}

}  // namespace vectra
