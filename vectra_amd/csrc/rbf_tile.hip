// Tile kernel dispatch: which problems it takes and which instantiation
// runs.  The kernel itself is in rbf_tile_impl.h.

#include "rbf_tile_impl.h"

namespace vectra {

bool tile_supports(const Problem& p, int in_dtype, int out_dtype) {
  if (in_dtype != VECTRA_BF16 && in_dtype != VECTRA_F16) return false;
  if (out_dtype != in_dtype && out_dtype != VECTRA_F32) return false;
  // Coefficient and bias are decoded from 2- or 4-byte elements.
  if (p.scale_dtype == VECTRA_F64 || (p.bias != nullptr && p.bias_dtype == VECTRA_F64)) return false;
  if (p.D != p.Dv || (p.D != 32 && p.D != 64 && p.D != 128)) return false;
  if (p.Nk < 1 || p.Nq < 1) return false;
  // 16-byte-aligned rows of q, k and v with unit element stride.
  if (p.sq[3] != 1 || p.sk[3] != 1 || p.sv[3] != 1) return false;
  for (int d = 0; d < 3; ++d)
    if (p.sq[d] % 8 != 0 || p.sk[d] % 8 != 0 || p.sv[d] % 8 != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k) |
       reinterpret_cast<uintptr_t>(p.v)) & 15u)
    return false;
  // Offsets inside a (b, h) plane are 32-bit (non-negative row strides).
  if (p.sq[2] < 0 || p.sk[2] < 0 || p.sv[2] < 0 || p.sbn < 0) return false;
  constexpr int64_t kMax32 = 0xffffffffLL;
  if (((p.Nq - 1) * p.sq[2] + p.D) * 2 > kMax32 || ((p.Nk - 1) * p.sk[2] + p.D) * 2 > kMax32 ||
      ((p.Nk - 1) * p.sv[2] + p.Dv) * 2 > kMax32)
    return false;
  if (p.bias != nullptr && (p.Nk - 1) * p.sbn * (p.bias_dtype == VECTRA_F32 ? 4 : 2) + 4 > kMax32) return false;
  // K and V tiles are loaded whole: the offsets of rows up to the last
  // tile's end (64 keys, 32 for 128-dim heads) stay 32-bit.
  const int64_t keys_padded = (p.Nk + 63) / 64 * 64;
  if (((keys_padded - 1) * p.sk[2] + p.D) * 2 > kMax32 || ((keys_padded - 1) * p.sv[2] + p.Dv) * 2 > kMax32)
    return false;
  // Output offsets inside a plane are 32-bit byte counts: the last element of
  // the plane's output view must lie within 4 GiB of the plane's first.
  const int64_t out_size = out_dtype == VECTRA_F32 ? 4 : 2;
  if (p.so[2] < 0 || p.so[3] < 0 ||
      ((p.Nq - 1) * p.so[2] + (p.Dv - 1) * p.so[3]) * out_size + out_size - 1 > kMax32)
    return false;
  // Work items (planes x blocks of at least 128 query rows) and item + grid size are 32-bit.
  return p.B * p.H * ((p.Nq + 127) / 128) < (int64_t{1} << 30);
}

hipError_t launch_tile(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  if (in_dt == VECTRA_BF16)
    return out_dt == VECTRA_F32 ? launch_tile_bf16_f32(p, s) : launch_tile_bf16_bf16(p, s);
  return out_dt == VECTRA_F32 ? launch_tile_f16_f32(p, s) : launch_tile_f16_f16(p, s);
}

}  // namespace vectra
