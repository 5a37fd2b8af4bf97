// Query-tile RBF attention on gfx950 matrix cores (bf16 / fp16 inputs).
//
// For query tiles (Nq >= 16: self-attention over a comparable set, long key
// axes) both products run on v_mfma_f32_16x16x32_{bf16,f16}:
//
//   S^T = K . Q^T     (16 keys x 16 queries per MFMA, 32 head dims deep)
//   O^T = V^T . P^T   (16 value dims x 16 queries, 32 keys deep)
//
// Lane layouts (checked on the device): for A (16 x 32) lane l holds row
// l % 16, elements 8 (l / 16) .. +7 of the deep dimension; for B (32 x 16)
// column l % 16, the same 8 deep elements; the fp32 result C (16 x 16) gives
// lane l column l % 16, rows 4 (l / 16) + r, r = 0..3.
//
// Computing S transposed puts, in each lane, the scores of ONE query (column
// l % 16) against keys 4 (l / 16) + r of each 16-key block.  Those eight
// values for two adjacent blocks are exactly the B operand of the second
// product once the 32-key deep dimension is read in the permuted order
// {4g..4g+3, 16+4g..16+4g+3} for lane group g = l / 16 -- and V^T is read in
// the same order from LDS.  So P never moves between lanes, and the online
// softmax state (running max, sum, rescale) of a query lives in its four
// lanes l, l+16, l+32, l+48, reduced with gfx950 permlane swaps.
//
// P is fed to the second product as a bf16 (or fp16) hi + lo pair (two
// MFMAs), so the weights keep ~16 more bits than one rounding would: rounding
// P once (as the reference's Triton kernel does) misses the rtol 1e-3 gate at
// a few tens of keys.
//
// Semantics are those of rbf_stream_kernel: clamp of the distance at 0,
// -scale * d + bias, keys >= Nk masked, a running max replaced by 0 while it
// is -inf (fully masked rows end as 0/0 = NaN), fp32 accumulation.

#include "rbf_common.h"
#include "rbf_kernels.h"

namespace vectra {

typedef float f32x4 __attribute__((ext_vector_type(4)));

template <typename T>
struct Mfma;

template <>
struct Mfma<__bf16> {
  typedef __bf16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Mfma<_Float16> {
  typedef _Float16 vec8 __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x4 run(vec8 a, vec8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

// LDS tile geometry.  Row pads make the 16 rows one operand read touches
// start in distinct banks.
template <typename T, int kD, int kDv, int kKeys>
struct MfmaTile {
  static constexpr int kKSteps = (kD + 31) / 32;   // deep steps of S^T = K . Q^T
  static constexpr int kDpad = kKSteps * 32;       // head dim padded with zeros
  static constexpr int kKStride = kDpad + 8;       // K row stride (elements)
  static constexpr int kVStride = kKeys + 4;       // V^T row stride (elements)
  static constexpr int kKBytes = kKeys * kKStride * sizeof(T);
  static constexpr int kVBytes = kDv * kVStride * sizeof(T);
  static constexpr int kBytes = kKBytes + kVBytes + 2 * kKeys * sizeof(float);
};

template <typename T, typename OutT, int kD, int kDv, int kKeys>
__global__ __launch_bounds__(512) void rbf_mfma_kernel(Problem p, int32_t q_blocks) {
  using Geo = MfmaTile<T, kD, kDv, kKeys>;
  using Vec8 = typename Mfma<T>::vec8;
  constexpr int kNTiles = kKeys / 16;   // 16-key blocks per tile
  constexpr int kPSteps = kKeys / 32;   // deep steps of O^T = V^T . P^T
  constexpr int kDvTiles = kDv / 16;
  constexpr int kDChunks = kD / 8;      // 16-byte chunks per K row
  constexpr int kDvChunks = kDv / 8;
  static_assert(kD % 8 == 0 && kDv % 16 == 0 && kKeys % 32 == 0 && kKeys <= 128, "tile shape");

  extern __shared__ __align__(16) unsigned char lds[];
  T* k_lds = reinterpret_cast<T*>(lds);
  T* vt_lds = reinterpret_cast<T*>(lds + Geo::kKBytes);
  float* kn_lds = reinterpret_cast<float*>(lds + Geo::kKBytes + Geo::kVBytes);
  float* bias_lds = kn_lds + kKeys;

  const int tid = threadIdx.x;
  const int n_threads = blockDim.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = n_threads >> 6;
  const int col = lane & 15;  // query within the wave's 16
  const int grp = lane >> 4;  // lane group g

  const int32_t block = static_cast<int32_t>(blockIdx.x);
  const int32_t bh = static_cast<int32_t>(fast_div(block, p.nq_mul, p.nq_shift));  // nq_* hold q_blocks here
  const int32_t qb = block - bh * q_blocks;
  const int32_t b = static_cast<int32_t>(fast_div(bh, p.h_mul, p.h_shift));
  const int32_t h = bh - b * static_cast<int32_t>(p.H);
  const int32_t n_q = static_cast<int32_t>(p.Nq);
  const int32_t n_k = static_cast<int32_t>(p.Nk);
  const int32_t q_row = (qb * waves + wave) * 16 + col;
  const bool q_live = q_row < n_q;

  const T* q_plane = static_cast<const T*>(p.q) + b * p.sq[0] + h * p.sq[1];
  const T* k_plane = static_cast<const T*>(p.k) + b * p.sk[0] + h * p.sk[1];
  const T* v_plane = static_cast<const T*>(p.v) + b * p.sv[0] + h * p.sv[1];
  const bool has_bias = p.bias != nullptr;
  const float neg_scale = -load_any(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);
  const int64_t bias_base = b * p.sbb + h * p.sbh;

  // Padding columns of the K tile (head dims kD .. kDpad) stay zero.
  if constexpr (Geo::kDpad > kD) {
    for (int i = tid; i < kKeys * (Geo::kDpad - kD); i += n_threads) {
      const int key = i / (Geo::kDpad - kD);
      const int d = kD + i % (Geo::kDpad - kD);
      k_lds[key * Geo::kKStride + d] = static_cast<T>(0.f);
    }
  }

  // This lane's slice of Q^T (the B operand of the first product) and the
  // query norm.  Dims past kD and rows past Nq are zero.
  Vec8 q_frag[Geo::kKSteps];
  float q_norm = 0.f;
#pragma unroll
  for (int s = 0; s < Geo::kKSteps; ++s) {
    const int d0 = 32 * s + 8 * grp;
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (q_live && d0 < kD) raw = load16(q_plane + q_row * p.sq[2] + d0);
    q_frag[s] = __builtin_bit_cast(Vec8, raw);
    q_norm = dot_chunk<T>(raw, raw, q_norm);
  }
  q_norm = allreduce_bit32(allreduce_bit16(q_norm, OpSum()), OpSum());

  float run_max = -INFINITY;
  float run_sum = 0.f;  // this lane's share; summed over the 4 lanes at the end
  f32x4 acc[kDvTiles];
#pragma unroll
  for (int u = 0; u < kDvTiles; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int32_t j0 = 0; j0 < n_k; j0 += kKeys) {
    __syncthreads();  // the previous tile is no longer read
    // K rows (row-major) and their norms.
    for (int c = tid; c < kKeys * kDChunks; c += n_threads) {
      const int key = c / kDChunks;
      const int part = c - key * kDChunks;
      const int32_t j = j0 + key;
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (j < n_k) raw = load16_stream(k_plane + j * p.sk[2] + part * 8);
      *reinterpret_cast<uint4*>(k_lds + key * Geo::kKStride + part * 8) = raw;
      float sq = reduce_low<kDChunks>(dot_chunk<T>(raw, raw, 0.f), OpSum());
      if (part == 0) kn_lds[key] = sq;
    }
    // V rows, written transposed: V^T[d][key].
    for (int c = tid; c < kKeys * kDvChunks; c += n_threads) {
      const int key = c / kDvChunks;
      const int part = c - key * kDvChunks;
      const int32_t j = j0 + key;
      uint4 raw = make_uint4(0, 0, 0, 0);
      if (j < n_k) raw = load16_stream(v_plane + j * p.sv[2] + part * 8);
      const T* vals = reinterpret_cast<const T*>(&raw);
#pragma unroll
      for (int e = 0; e < 8; ++e) vt_lds[(part * 8 + e) * Geo::kVStride + key] = vals[e];
    }
    // Key bias as fp32; keys past Nk are -inf.
    for (int key = tid; key < kKeys; key += n_threads) {
      const int32_t j = j0 + key;
      float x = -INFINITY;
      if (j < n_k) x = has_bias ? load_any(p.bias, bias_base + j * p.sbn, p.bias_dtype) : 0.f;
      bias_lds[key] = x;
    }
    __syncthreads();

    // Scores S^T for this lane's query against keys 16t + 4g + r.
    float logit[kNTiles][4];
    float tile_max = -INFINITY;
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < Geo::kKSteps; ++ks) {
        const Vec8 a = *reinterpret_cast<const Vec8*>(k_lds + (16 * t + col) * Geo::kKStride +
                                                      32 * ks + 8 * grp);
        s = Mfma<T>::run(a, q_frag[ks], s);
      }
      const float4 kn = *reinterpret_cast<const float4*>(kn_lds + 16 * t + 4 * grp);
      const float4 bias = *reinterpret_cast<const float4*>(bias_lds + 16 * t + 4 * grp);
      const float knv[4] = {kn.x, kn.y, kn.z, kn.w};
      const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float dist = fmaxf((q_norm + knv[r]) - 2.f * s[r], 0.f);
        const float x = neg_scale * dist + bv[r];
        logit[t][r] = x;
        tile_max = fmaxf(tile_max, x);
      }
    }
    tile_max = allreduce_bit32(allreduce_bit16(tile_max, OpMax()), OpMax());
    const float new_max = fmaxf(run_max, tile_max);
    const float safe_max = new_max == -INFINITY ? 0.f : new_max;
    const float alpha = __builtin_amdgcn_exp2f((run_max - safe_max) * kLog2e);
    run_max = new_max;
    run_sum *= alpha;
#pragma unroll
    for (int u = 0; u < kDvTiles; ++u) acc[u] *= alpha;

    // O^T += V^T . P^T, 32 keys per step, P as a hi + lo pair.
#pragma unroll
    for (int ps = 0; ps < kPSteps; ++ps) {
      Vec8 p_hi, p_lo;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float w = __builtin_amdgcn_exp2f((logit[2 * ps + half][r] - safe_max) * kLog2e);
          run_sum += w;
          const T hi = static_cast<T>(w);
          p_hi[4 * half + r] = hi;
          p_lo[4 * half + r] = static_cast<T>(w - static_cast<float>(hi));
        }
      }
#pragma unroll
      for (int u = 0; u < kDvTiles; ++u) {
        const T* row = vt_lds + (16 * u + col) * Geo::kVStride + 32 * ps + 4 * grp;
        const uint2 lo4 = *reinterpret_cast<const uint2*>(row);
        const uint2 hi4 = *reinterpret_cast<const uint2*>(row + 16);
        const Vec8 a = __builtin_bit_cast(Vec8, make_uint4(lo4.x, lo4.y, hi4.x, hi4.y));
        acc[u] = Mfma<T>::run(a, p_hi, acc[u]);
        acc[u] = Mfma<T>::run(a, p_lo, acc[u]);
      }
    }
  }

  const float total = allreduce_bit32(allreduce_bit16(run_sum, OpSum()), OpSum());
  if (!q_live) return;  // after the last barrier
  // A fully masked row has total 0: 0 * inf = NaN, as eager softmax gives.
  const float inv = __builtin_amdgcn_rcpf(total);
  OutT* o = static_cast<OutT*>(p.out) + b * p.so[0] + h * p.so[1] + q_row * p.so[2];
#pragma unroll
  for (int u = 0; u < kDvTiles; ++u) {
#pragma unroll
    for (int r = 0; r < 4; ++r) o[(16 * u + 4 * grp + r) * p.so[3]] = from_float<OutT>(acc[u][r] * inv);
  }
}

// ------------------------------------------------------------------- host

namespace {

template <typename T, typename OutT, int kD, int kKeys>
hipError_t launch_mfma_k(Problem& p, hipStream_t s) {
  using Geo = MfmaTile<T, kD, kD, kKeys>;
  const int waves = p.Nq >= 128 ? 8 : static_cast<int>((p.Nq + 15) / 16);
  const int32_t q_blocks = static_cast<int32_t>((p.Nq + waves * 16 - 1) / (waves * 16));
  const int64_t blocks = p.B * p.H * q_blocks;
  // The kernel decomposes its block id with the Nq divisor slots.
  Problem k = p;
  uint32_t mul = 0, shift = 0;
  {
    uint32_t l = 0;
    while ((int64_t{1} << l) < q_blocks) ++l;
    if ((int64_t{1} << l) == q_blocks) {
      mul = 0;
      shift = l;
    } else {
      mul = static_cast<uint32_t>(((uint64_t{1} << (31 + l)) + q_blocks - 1) / q_blocks);
      shift = l - 1;
    }
  }
  k.nq_mul = mul;
  k.nq_shift = shift;
  void* args[] = {&k, const_cast<int32_t*>(&q_blocks)};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_mfma_kernel<T, OutT, kD, kD, kKeys>),
                         dim3(static_cast<unsigned>(blocks)), dim3(64 * waves), args, Geo::kBytes, s);
}

template <typename T, typename OutT, int kD>
hipError_t launch_mfma_d(Problem& p, hipStream_t s) {
  // Key axes up to 128 run as one tile (one global round trip, two barriers)
  // of the smallest multiple of 32 keys that covers them; longer axes stream
  // tiles of 64 keys (128 up to 64 head dims; the LDS tile stays under 64 KB).
  const int64_t n_k = p.Nk;
  if (n_k <= 32) return launch_mfma_k<T, OutT, kD, 32>(p, s);
  if (n_k <= 64) return launch_mfma_k<T, OutT, kD, 64>(p, s);
  if (n_k <= 96) return launch_mfma_k<T, OutT, kD, 96>(p, s);
  if (kD <= 64) return launch_mfma_k<T, OutT, kD, 128>(p, s);
  return launch_mfma_k<T, OutT, kD, 64>(p, s);
}

template <typename T, typename OutT>
hipError_t launch_mfma_t(Problem& p, hipStream_t s) {
  switch (p.D) {
    case 16: return launch_mfma_d<T, OutT, 16>(p, s);
    case 32: return launch_mfma_d<T, OutT, 32>(p, s);
    case 64: return launch_mfma_d<T, OutT, 64>(p, s);
    case 128: return launch_mfma_d<T, OutT, 128>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool mfma_supports(const Problem& p, int in_dtype, int out_dtype) {
  if (in_dtype != VECTRA_BF16 && in_dtype != VECTRA_F16) return false;
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
  // Block ids (planes x query blocks) are 32-bit.
  return p.B * p.H * ((p.Nq + 15) / 16) < (int64_t{1} << 31);
}

hipError_t launch_mfma(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  if (in_dt == VECTRA_BF16)
    return out_dt == VECTRA_F32 ? launch_mfma_t<__bf16, float>(p, s) : launch_mfma_t<__bf16, __bf16>(p, s);
  return out_dt == VECTRA_F32 ? launch_mfma_t<_Float16, float>(p, s)
                              : launch_mfma_t<_Float16, _Float16>(p, s);
}

}  // namespace vectra
