// MFMA kernel dispatch: which problems it takes and which instantiation runs.
// The kernel itself is in rbf_mfma_impl.h.

#include "rbf_mfma_impl.h"

namespace vectra {

bool mfma_supports(const Problem& p, int in_dtype, int out_dtype) {
  if (in_dtype != VECTRA_BF16 && in_dtype != VECTRA_F16) return false;
  // Coefficient and bias are decoded from 2- or 4-byte elements.
  if (p.scale_dtype == VECTRA_F64 || (p.bias != nullptr && p.bias_dtype == VECTRA_F64)) return false;
  if (out_dtype != in_dtype && out_dtype != VECTRA_F32) return false;
  if (p.D != p.Dv || (p.D != 16 && p.D != 32 && p.D != 64 && p.D != 128)) return false;
  if (p.Nk < 1 || p.Nq < 1) return false;
  // 16-byte rows of q, k and v with unit element stride.
  if (p.sq[3] != 1 || p.sk[3] != 1 || p.sv[3] != 1) return false;
  for (int d = 0; d < 3; ++d)
    if (p.sq[d] % 8 != 0 || p.sk[d] % 8 != 0 || p.sv[d] % 8 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
       reinterpret_cast<uintptr_t>(p.v)) & 15u)
    return false;
  // Work items (planes x query blocks) and item + grid size are 32-bit.
  return p.B * p.H * ((p.Nq + 15) / 16) < (int64_t{1} << 30);
}

hipError_t launch_mfma(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  if (in_dt == VECTRA_BF16)
    return out_dt == VECTRA_F32 ? launch_mfma_bf16_f32(p, s) : launch_mfma_bf16_bf16(p, s);
  return out_dt == VECTRA_F32 ? launch_mfma_f16_f32(p, s) : launch_mfma_f16_f16(p, s);
}

}  // namespace vectra
