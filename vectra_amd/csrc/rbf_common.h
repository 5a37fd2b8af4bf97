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
  int32_t grid_waves;  // waves launched by persistent kernels (<= total_rows)
  int32_t compute_units;  // of the device the launch runs on
  int32_t flags;          // VECTRA_FLAG_* bits
  uint32_t nq_mul, nq_shift;  // FastDiv of Nq (see fast_div)
  uint32_t h_mul, h_shift;    // FastDiv of H
};

// Loads the given kernel arguments into scalar registers at this point: the
// compiler then issues all of their scalar loads as one batch with one wait.
// Left to itself it loads each argument where it is first used, which in a
// prologue with branches becomes several dependent rounds of scalar-cache
// latency before a wave can issue its first vector load.
template <typename T>
__device__ __forceinline__ void arg_in_sgprs(const T& a) {
  asm volatile("" ::"s"(a));
}
template <typename... A>
__device__ __forceinline__ void args_in_sgprs(const A&... a) {
  (arg_in_sgprs(a), ...);
}

// floor(n / d) for 0 <= n < 2^31 from a multiplier and shift made on the host
// (make_fast_div): mul == 0 means d is a power of two, else
// mul = ceil(2^(31+l) / d) with l = ceil(log2 d) and shift = l - 1.  Then
// n * mul / 2^(31+l) = n/d + err with 0 <= err < n / 2^(31+l) < 1/d, so the
// floor is exact; mul < 2^32 because d > 2^(l-1).
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint32_t mul, uint32_t shift) {
  return mul ? (__umulhi(n, mul) >> shift) : (n >> shift);
}

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// max(d, 0) for an expanded squared distance, keeping NaN (one
// v_maximum3_f32): a NaN in q or k must reach the softmax, where it makes the
// row NaN as the eager chain's (q - k)^2 does, even for a masked key.
// fmaxf(NaN, 0) would return 0.
__device__ __forceinline__ float clamp_distance(float d) {
  return __builtin_elementwise_maximum(d, 0.f);
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
// The fp32 value is made opaque first: otherwise the compiler fuses the
// product that produced it with the conversion (v_fma_mixlo_f16, one
// rounding), and a 16-bit output would no longer be exactly the fp32 result
// rounded once more, as the operator's output is defined.
template <typename T>
__device__ __forceinline__ T from_float(float x) {
  if constexpr (sizeof(T) < sizeof(float)) asm volatile("" : "+v"(x));
  return static_cast<T>(x);
}

// A 2- or 4-byte float element fetched as the aligned 32-bit word that holds
// it.  The load has no dtype-dependent control flow, so it can be issued
// with the tile's other loads and decoded at first use without an early
// wait.  The aligned word never leaves the element's page.
struct RawScalar {
  uint32_t word;
  uint32_t shift;  // 0 or 16: position of a 2-byte element in the word
};

__device__ __forceinline__ RawScalar load_raw_scalar(const void* base, int64_t index,
                                                     int32_t dtype) {
  // Offsets are formed from `base` itself (not an integer address) so the
  // access stays a global load rather than a flat one.
  const int64_t misalign = static_cast<int64_t>(reinterpret_cast<uintptr_t>(base) & 3);
  const int64_t bytes = index * (dtype == VECTRA_F32 ? 4 : 2) + misalign;
  RawScalar r;
  r.word = *reinterpret_cast<const uint32_t*>(static_cast<const char*>(base) + (bytes & ~int64_t{3}) -
                                              misalign);
  r.shift = static_cast<uint32_t>(bytes & 2) * 8;
  return r;
}

// Same, for an element at a 32-bit element offset from a wave-uniform base
// that is only 2-byte aligned (a (b, h) plane of a 2-byte bias starts
// wherever the batch and head strides put it).  The word read is the aligned
// 32-bit word holding the element, never the bytes after it; the address is
// aligned base + 32-bit lane offset, which global_load encodes directly.
// `misalign` must be base_misalign(base); decodes recompute the shift from it.
__device__ __forceinline__ uint32_t base_misalign(const char* base) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(base) & 3);
}

__device__ __forceinline__ RawScalar load_raw_scalar32(const char* base, uint32_t misalign,
                                                       uint32_t elem_offset, int32_t dtype) {
  const uint32_t bytes = elem_offset * (dtype == VECTRA_F32 ? 4u : 2u) + misalign;
  RawScalar r;
  r.word = *reinterpret_cast<const uint32_t*>(base - misalign + (bytes & ~3u));
  r.shift = (bytes & 2u) * 8u;
  return r;
}

// dtype is F32, F16 or BF16 (F64 operands never reach the stream kernels).
__device__ __forceinline__ float decode_raw_scalar(RawScalar r, int32_t dtype) {
  const uint32_t half_bits = (r.word >> r.shift) & 0xffffu;
  const float as_bf16 = __uint_as_float(half_bits << 16);
  const float as_f16 = static_cast<float>(
      __builtin_bit_cast(_Float16, static_cast<uint16_t>(half_bits)));
  const float as_f32 = __uint_as_float(r.word);
  return dtype == VECTRA_F32 ? as_f32 : (dtype == VECTRA_BF16 ? as_bf16 : as_f16);
}

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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// A buffer resource over `bytes` bytes from `base`: loads past the end read
// as zeros.  Word 3 is the gfx9 data-format field of a raw buffer.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t plane_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// Cache policy of the streaming loads: non-temporal.
constexpr int kNt = 2;
__device__ __forceinline__ uint4 load16_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kNt);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ __forceinline__ uint4 load16(const void* p) {
  return *static_cast<const uint4*>(p);
}

// 128-bit load marked non-temporal: K and V are each read once, so they
// should not displace reused lines (q, bias) in the caches.  Measured on
// MI355X, a plain 64 MB read at the serving layout runs 11% faster this way.
__device__ __forceinline__ uint4 load16_stream(const void* p) {
  const u32x4 r = __builtin_nontemporal_load(static_cast<const u32x4*>(p));
  return make_uint4(r.x, r.y, r.z, r.w);
}

// Dot product of two 128-bit chunks in fp32: v_dot2 on packed bf16 / fp16
// pairs (products of 16-bit floats are exact in fp32), FMAs for fp32.
template <typename T>
__device__ __forceinline__ float dot_chunk(const uint4& a, const uint4& b, float acc);

template <>
__device__ __forceinline__ float dot_chunk<__bf16>(const uint4& a, const uint4& b, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  const uint32_t x[4] = {a.x, a.y, a.z, a.w};
  const uint32_t y[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x[i]),
                                          __builtin_bit_cast(bf16x2, y[i]), acc, false);
  return acc;
}

template <>
__device__ __forceinline__ float dot_chunk<_Float16>(const uint4& a, const uint4& b, float acc) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  const uint32_t x[4] = {a.x, a.y, a.z, a.w};
  const uint32_t y[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
  for (int i = 0; i < 4; ++i)
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, x[i]), __builtin_bit_cast(f16x2, y[i]),
                                 acc, false);
  return acc;
}

template <>
__device__ __forceinline__ float dot_chunk<float>(const uint4& a, const uint4& b, float acc) {
  acc = fmaf(__uint_as_float(a.x), __uint_as_float(b.x), acc);
  acc = fmaf(__uint_as_float(a.y), __uint_as_float(b.y), acc);
  acc = fmaf(__uint_as_float(a.z), __uint_as_float(b.z), acc);
  return fmaf(__uint_as_float(a.w), __uint_as_float(b.w), acc);
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

// Writes N (1 or 2) fp32 values as OutT (N * sizeof(OutT)-aligned address).
template <typename OutT, int N>
__device__ __forceinline__ void store_small(OutT* dst, const float* f) {
  if constexpr (N == 1) {
    dst[0] = from_float<OutT>(f[0]);
  } else {
    static_assert(N == 2, "one or two values");
    if constexpr (sizeof(OutT) == 4) {
      *reinterpret_cast<float2*>(dst) = make_float2(f[0], f[1]);
    } else {
      OutT pair[2] = {from_float<OutT>(f[0]), from_float<OutT>(f[1])};
      *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(pair);
    }
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

// gfx950 lane swaps (VALU, no LDS traffic).  With both operands equal to x,
// permlane16_swap returns {rows 0,0,2,2 of x; rows 1,1,3,3 of x} (a row is 16
// lanes) and permlane32_swap returns {lanes 0-31 twice; lanes 32-63 twice}, so
// op(r[0], r[1]) is the all-reduce over lane bit 16 or bit 32.  The layout
// was checked on the device.
template <typename Op>
__device__ __forceinline__ float allreduce_bit16(float x, Op op) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

template <typename Op>
__device__ __forceinline__ float allreduce_bit32(float x, Op op) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return op(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};
struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// All-reduce over the low lane bits 1 .. kGroup/2 (groups of kGroup adjacent
// lanes; kGroup a power of two <= 64).  Mirrors are valid because the lower
// bits are already reduced when they run.
template <int kGroup, typename Op>
__device__ __forceinline__ float reduce_low(float x, Op op) {
  if constexpr (kGroup >= 2) x = op(x, dpp<0xB1>(x));
  if constexpr (kGroup >= 4) x = op(x, dpp<0x4E>(x));
  if constexpr (kGroup >= 8) x = op(x, dpp<0x141>(x));
  if constexpr (kGroup >= 16) x = op(x, dpp<0x140>(x));
  if constexpr (kGroup >= 32) x = allreduce_bit16(x, op);
  if constexpr (kGroup >= 64) x = allreduce_bit32(x, op);
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
  if constexpr (kFrom <= 16) x = allreduce_bit16(x, op);
  return allreduce_bit32(x, op);
}

template <typename Op>
__device__ __forceinline__ float reduce_wave(float x, Op op) {
  return reduce_high<1>(x, op);
}

}  // namespace vectra
