// gfx950 matrix-core operations shared by the query-tile kernels
// (rbf_mfma_impl.h, rbf_plane_impl.h).
//
// Lane layouts of the instructions used (wave64, l = lane, g = l / 16):
//   16x16x32 bf16/f16  A: row l % 16, deep 8g .. 8g+7;  B: column l % 16, same
//   16x16x16 bf16/f16  A: row l % 16, deep 4g .. 4g+3;  B: column l % 16, same
//   16x16x4  f32       A: row l % 16, deep g;           B: column l % 16, deep g
//   result C (16 x 16 fp32): column l % 16, rows 4g .. 4g+3.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vectra {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

// The products for one input type.  `Qk` is a 16-byte (8-element) operand
// of the 32-deep instruction, `Pv` a 4-element operand of the 16-deep one.
template <typename T>
struct MfmaOps;

template <>
struct MfmaOps<__bf16> {
  typedef __bf16 Qk __attribute__((ext_vector_type(8)));
  typedef short Pv __attribute__((ext_vector_type(4)));  // four bf16 bit patterns
  static constexpr uint32_t kOnePair = 0x3f803f80u;     // two bf16 1.0
  static __device__ __forceinline__ f32x4 qk(Qk a, Qk b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(Pv a, Pv b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
  // Two weights as packed bf16 hi (round to nearest, v_cvt_pk_bf16_f32) and
  // lo = bf16(w - hi): hi + lo = w to ~2^-17.  w - hi is exact in fp32 and
  // comes from one v_dot2 per weight (hi . (-1, 0) + w), which reads the
  // packed hi directly.  The (-1, 0) and (0, -1) pairs come from scalar
  // registers (v_dot2c takes one as its first source, so they cost no VGPR):
  // as an inline constant, the compiler encodes the bf16 pair (-1, 0) as the
  // 32-bit constant -1.0, which the hardware reads as (0, -1).
  static __device__ __forceinline__ void split2(float w0, float w1, uint32_t& hi, uint32_t& lo) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{w0, w1}, b2));
    const b2 h = __builtin_bit_cast(b2, hi);
    uint32_t neg_lo, neg_hi;  // bf16 pairs (-1, 0), (0, -1), in scalar registers
    asm("s_mov_b32 %0, 0xbf80" : "=s"(neg_lo));
    asm("s_mov_b32 %0, 0xbf800000" : "=s"(neg_hi));
    const float d0 = __builtin_amdgcn_fdot2_f32_bf16(h, __builtin_bit_cast(b2, neg_lo), w0, false);
    const float d1 = __builtin_amdgcn_fdot2_f32_bf16(h, __builtin_bit_cast(b2, neg_hi), w1, false);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{d0, d1}, b2));
  }
  // The same split with hi widened by shifts and w - hi by subtractions (two
  // more instructions per pair).  The tile kernel keeps this form: with the
  // v_dot2 form it measured 3% slower (1.81 against 1.75 ms at 4096 keys).
  static __device__ __forceinline__ void split2_sub(float w0, float w1, uint32_t& hi, uint32_t& lo) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    hi = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{w0, w1}, b2));
    const float h0 = __uint_as_float(hi << 16), h1 = __uint_as_float(hi & 0xffff0000u);
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{w0 - h0, w1 - h1}, b2));
  }
};

template <>
struct MfmaOps<_Float16> {
  typedef _Float16 Qk __attribute__((ext_vector_type(8)));
  typedef _Float16 Pv __attribute__((ext_vector_type(4)));
  static constexpr uint32_t kOnePair = 0x3c003c00u;  // two fp16 1.0
  static __device__ __forceinline__ f32x4 qk(Qk a, Qk b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ f32x4 pv(Pv a, Pv b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
  }
  // Two weights as packed fp16 hi (round toward zero, v_cvt_pkrtz_f16_f32)
  // and lo = fp16(w - hi), w - hi being exact in fp32: hi + lo = w to ~2^-20.
  // w - hi comes from one v_dot2 per weight, as for bf16 (fp16 denormals are
  // kept: the kernels run in the default IEEE mode).
  static __device__ __forceinline__ void split2(float w0, float w1, uint32_t& hi, uint32_t& lo) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    const h2 h = __builtin_bit_cast(h2, __builtin_amdgcn_cvt_pkrtz(w0, w1));
    hi = __builtin_bit_cast(uint32_t, h);
    const float d0 = __builtin_amdgcn_fdot2(h, h2{static_cast<_Float16>(-1.f), static_cast<_Float16>(0.f)}, w0, false);
    const float d1 = __builtin_amdgcn_fdot2(h, h2{static_cast<_Float16>(0.f), static_cast<_Float16>(-1.f)}, w1, false);
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(d0, d1));
  }
  static __device__ __forceinline__ void split2_sub(float w0, float w1, uint32_t& hi, uint32_t& lo) {
    split2(w0, w1, hi, lo);  // fp16: the v_dot2 form everywhere
  }
};

// gfx950's transposing LDS read (ds_read_b64_tr_b16) of 16-bit elements.
// Within each group of 16 lanes, lane i receives element i % 4 of the 8-byte
// pieces addressed by lanes i / 4, 4 + i / 4, 8 + i / 4 and 12 + i / 4: with
// lane i addressing row r0 + i / 4, elements 4 (i % 4) .. +3 of row-major
// data, lane i gets element i of rows r0 .. r0 + 3 (the A operand of a
// 16-deep product read from a row-major B).  The mapping was checked on the
// device.
typedef short lds_v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
  // A C-style cast converts the generic pointer to the LDS address space.
  const lds_v4s r =
      __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) lds_v4s*)(const_cast<void*>(p)));
  return __builtin_bit_cast(uint2, r);
}

// Two fp32 values as one 32-bit word of two OutT (round to nearest even,
// each value first materialised in fp32: see from_float).
template <typename OutT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  asm volatile("" : "+v"(a), "+v"(b));
  typedef OutT o2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{a, b}, o2));
}

template <>
struct MfmaOps<float> {
  static __device__ __forceinline__ f32x4 mma(float a, float b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
  }
};

}  // namespace vectra
