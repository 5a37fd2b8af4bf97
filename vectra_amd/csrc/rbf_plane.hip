// Plane kernel dispatch: which problems it takes and which instantiation
// runs.  The kernels are in rbf_plane_impl.h (16-bit inputs) and
// rbf_plane32_impl.h (fp32 inputs).

#include "rbf_plane32_impl.h"
#include "rbf_plane_impl.h"

namespace vectra {

bool plane_supports(const Problem& p, int in_dtype, int out_dtype) {
  if (in_dtype != VECTRA_BF16 && in_dtype != VECTRA_F16 && in_dtype != VECTRA_F32) return false;
  if (out_dtype != in_dtype && out_dtype != VECTRA_F32) return false;
  const int64_t esize = in_dtype == VECTRA_F32 ? 4 : 2;
  // Coefficient and bias are decoded from 2- or 4-byte elements.
  if (p.scale_dtype == VECTRA_F64 || (p.bias != nullptr && p.bias_dtype == VECTRA_F64)) return false;
  if (p.D != p.Dv || (p.D != 16 && p.D != 32)) return false;
  if (p.Nk < 1 || p.Nq < 1) return false;
  // Both axes fit one tile: 80 rows, or 128 for 16-dim heads.
  const int64_t rows = p.Nq > p.Nk ? p.Nq : p.Nk;
  if (rows > (p.D == 16 ? 128 : 80)) return false;
  // 16-byte-aligned rows of q, k and v with unit element stride (the kernel
  // loads 8- or 16-byte pieces of them).
  if (p.sq[3] != 1 || p.sk[3] != 1 || p.sv[3] != 1) return false;
  const int64_t per16 = 16 / esize;  // elements per 16 bytes
  for (int d = 0; d < 3; ++d)
    if (p.sq[d] % per16 != 0 || p.sk[d] % per16 != 0 || p.sv[d] % per16 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
       reinterpret_cast<uintptr_t>(p.v)) & 15u)
    return false;
  // Offsets inside a (b, h) plane are 32-bit (non-negative row strides).
  if (p.sq[2] < 0 || p.sk[2] < 0 || p.sv[2] < 0 || p.sbn < 0) return false;
  constexpr int64_t kMax32 = 0xffffffffLL;
  if (((p.Nq - 1) * p.sq[2] + p.D) * esize > kMax32 || ((p.Nk - 1) * p.sk[2] + p.D) * esize > kMax32 ||
      ((p.Nk - 1) * p.sv[2] + p.Dv) * esize > kMax32)
    return false;
  if (p.bias != nullptr && (p.Nk - 1) * p.sbn * (p.bias_dtype == VECTRA_F32 ? 4 : 2) + 4 > kMax32) return false;
  // The kernel reads through buffer resources that end at a plane's last
  // row, so rows past Nk read as zeros only if K and V rows do not overlap;
  // the offsets it forms span up to 144 rows (a tile plus a query block).
  if (p.sk[2] < p.D || p.sv[2] < p.Dv) return false;
  constexpr int64_t kRows = 144;
  if (kRows * p.sq[2] * esize > kMax32 || kRows * p.sk[2] * esize > kMax32 || kRows * p.sv[2] * esize > kMax32)
    return false;
  if (p.bias != nullptr && kRows * p.sbn * (p.bias_dtype == VECTRA_F32 ? 4 : 2) > kMax32) return false;
  // Output offsets inside a plane are 32-bit byte counts: the last element of
  // the plane's output view must lie within 4 GiB of the plane's first.
  const int64_t out_size = out_dtype == VECTRA_F32 ? 4 : 2;
  if (p.so[2] < 0 || p.so[3] < 0 ||
      ((p.Nq - 1) * p.so[2] + (p.Dv - 1) * p.so[3]) * out_size + out_size - 1 > kMax32)
    return false;
  // Plane indices (and plane + grid size) are 32-bit.
  return p.B * p.H < (int64_t{1} << 30);
}

hipError_t launch_plane(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  if (in_dt == VECTRA_F32) return launch_plane_f32_f32(p, s);
  if (in_dt == VECTRA_BF16)
    return out_dt == VECTRA_F32 ? launch_plane_bf16_f32(p, s) : launch_plane_bf16_bf16(p, s);
  return out_dt == VECTRA_F32 ? launch_plane_f16_f32(p, s) : launch_plane_f16_f16(p, s);
}

}  // namespace vectra
