// MFMA kernel dispatch: which problems it takes and which instantiation runs.
// The kernel itself is in rbf_mfma_impl.h.

#include "rbf_mfma_impl.h"

namespace vectra {

namespace {

// Largest byte offset, inside one (b, h) plane, of a row-major operand with
// `rows` rows of `cols` elements at row stride `stride` (elements).
int64_t plane_extent(int64_t rows, int64_t stride, int64_t cols, int64_t esize) {
  return ((rows - 1) * stride + cols) * esize;
}

}  // namespace

bool mfma_supports(const Problem& p, int in_dtype, int out_dtype) {
  if (in_dtype != VECTRA_BF16 && in_dtype != VECTRA_F16 && in_dtype != VECTRA_F32) return false;
  // Outputs in the input dtype or fp32.
  if (out_dtype != in_dtype && out_dtype != VECTRA_F32) return false;
  // Coefficient and bias are decoded from 2- or 4-byte elements.
  if (p.scale_dtype == VECTRA_F64 || (p.bias != nullptr && p.bias_dtype == VECTRA_F64)) return false;
  if (p.D != p.Dv || (p.D != 16 && p.D != 32 && p.D != 64 && p.D != 128)) return false;
  if (p.Nk < 1 || p.Nq < 1) return false;
  // 16-byte rows of q, k and v with unit element stride.
  const int64_t esize = in_dtype == VECTRA_F32 ? 4 : 2;
  const int64_t vec = 16 / esize;
  if (p.sq[3] != 1 || p.sk[3] != 1 || p.sv[3] != 1) return false;
  for (int d = 0; d < 3; ++d)
    if (p.sq[d] % vec != 0 || p.sk[d] % vec != 0 || p.sv[d] % vec != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
       reinterpret_cast<uintptr_t>(p.v)) & 15u)
    return false;
  // Offsets inside a (b, h) plane are 32-bit (row strides and the bias
  // stride non-negative).
  constexpr int64_t kMax32 = 0xffffffffLL;
  if (p.sq[2] < 0 || p.sk[2] < 0 || p.sv[2] < 0 || p.sbn < 0) return false;
  if (plane_extent(p.Nq, p.sq[2], p.D, esize) > kMax32 || plane_extent(p.Nk, p.sk[2], p.D, esize) > kMax32 ||
      plane_extent(p.Nk, p.sv[2], p.Dv, esize) > kMax32)
    return false;
  if (p.bias != nullptr && plane_extent(p.Nk, p.sbn, 1, p.bias_dtype == VECTRA_F32 ? 4 : 2) > kMax32)
    return false;
  // Work items (planes x query blocks) and item + grid size are 32-bit.
  return p.B * p.H * ((p.Nq + 15) / 16) < (int64_t{1} << 30);
}

hipError_t launch_mfma(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  if (in_dt == VECTRA_F32) return launch_mfma_f32_f32(p, s);
  if (in_dt == VECTRA_BF16)
    return out_dt == VECTRA_F32 ? launch_mfma_bf16_f32(p, s) : launch_mfma_bf16_bf16(p, s);
  return out_dt == VECTRA_F32 ? launch_mfma_f16_f32(p, s) : launch_mfma_f16_f16(p, s);
}

}  // namespace vectra
