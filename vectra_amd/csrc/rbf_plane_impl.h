// Single-tile RBF attention on gfx950 matrix cores, one workgroup per (b, h)
// plane and one wave per two 16-query blocks: the kernel template,
// instantiated per dtype pair in rbf_plane_<in>_<out>.hip.
//
// For planes whose query and key axes both fit one tile (self-attention over
// a comparable set: Lq = Lk = 65, head dims 16 and 32) the workgroup stages
// the plane's K and V in LDS once, and each of its waves then computes two
// blocks of 16 queries against every key:
//
//   S^T = K . Q^T     (16 keys x 16 queries per instruction)
//   O^T = V^T . P^T   (16 value dims x 16 queries)
//
// with the lane layouts listed in rbf_mfma_ops.h (l = lane, g = l / 16).  A
// lane holds the scores of one query (column l % 16) against keys
// 16t + 4g + r; those of key blocks 2p and 2p + 1 are the B operand of one
// 16x16x32 step of the second product over keys read in the order
// {32p + 4g .. +3, 32p + 16 + 4g .. +3}, and an odd last block takes a
// 16x16x16 step.  K rows sit in LDS as loaded (the A operand of the first
// product is row l % 16 of a key block, head dims 8g .. 8g+7, or 4g .. 4g+3
// for 16-dim heads; read where it is used); V is written transposed; q goes
// from HBM straight into the B operand.
//
// Per-score arithmetic is one FMA, one exp2 and the 16-bit split of the
// weight:
//  * gamma |k|^2 / 2 and the key bias are folded once per plane into one
//    value per key,
//      c_j = log2(e) (bias_j - gamma |k_j|^2),
//    and the per-query constant -gamma |q|^2 is left out (a softmax row does
//    not see a shift), so the exp2 argument is one FMA of the product,
//      x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j);
//  * the softmax sum comes from the second product itself: a row of ones in
//    the A operand sums the same hi + lo weights the values are weighted by,
//    so the denominator needs no VALU add and no cross-lane reduction;
//  * no running maximum is kept: if a query's weight sum leaves the range in
//    which the 16-bit split is accurate and the value products cannot
//    overflow (gamma < 0, a query far from every key, biases far from 0), its
//    block is computed once more with each query's exact maximum subtracted.
// The distance is not clamped at zero: where rounding makes the expansion
// negative (a query on top of a key), -d and the reference's max(d, 0) = 0
// are both within the expansion's rounding error of the true distance.
//
// Weights are fed to the second product as hi + lo 16-bit pairs (~2^-17 of
// the weight), as in rbf_mfma_kernel.  Keys past Nk have c_j = -inf, and
// their K and V rows read as zeros, so they contribute nothing.  A fully masked
// row ends as 0 * (1 / 0) = NaN, as eager softmax gives.
//
// Scheduling: one workgroup per plane, a wave per two query blocks (three
// waves for 65 queries).  The waves share the staging of K and V and then
// run their blocks independently, the two blocks of a wave interleaved; the
// hardware balances planes over the compute units as workgroups finish, and
// the load latency of one workgroup is covered by the products of the others
// resident on the same compute unit.  Workgroup w is mapped to a plane so
// that an XCD works on contiguous planes.
#pragma once

#include <type_traits>

#include "rbf_common.h"
#include "rbf_kernels.h"
#include "rbf_mfma_ops.h"

namespace vectra {

template <int kBytes>
struct PlaneFrag;
template <>
struct PlaneFrag<16> {
  typedef uint4 type;
  static __device__ __forceinline__ uint4 zero() { return make_uint4(0, 0, 0, 0); }
  static __device__ __forceinline__ uint4 load_stream(const void* p) { return load16_stream(p); }
  static __device__ __forceinline__ uint4 load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return load16_buf(r, off);
  }
};
template <>
struct PlaneFrag<8> {
  typedef uint2 type;
  static __device__ __forceinline__ uint2 zero() { return make_uint2(0, 0); }
  static __device__ __forceinline__ uint2 load_stream(const void* p) {
    typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
    const u32x2 r = __builtin_nontemporal_load(static_cast<const u32x2*>(p));
    return make_uint2(r.x, r.y);
  }
  static __device__ __forceinline__ uint2 load_buf(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNt);
    return make_uint2(v[0], v[1]);
  }
};

template <typename T>
__device__ __forceinline__ float dot_pair(uint32_t a, uint32_t b, float acc);
template <>
__device__ __forceinline__ float dot_pair<__bf16>(uint32_t a, uint32_t b, float acc) {
  typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), acc,
                                         false);
}
template <>
__device__ __forceinline__ float dot_pair<_Float16>(uint32_t a, uint32_t b, float acc) {
  typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), acc, false);
}

template <typename T>
__device__ __forceinline__ float frag_norm(uint4 f) {
  return dot_pair<T>(f.w, f.w, dot_pair<T>(f.z, f.z, dot_pair<T>(f.y, f.y, dot_pair<T>(f.x, f.x, 0.f))));
}
template <typename T>
__device__ __forceinline__ float frag_norm(uint2 f) {
  return dot_pair<T>(f.y, f.y, dot_pair<T>(f.x, f.x, 0.f));
}

// One 16-key block of S^T: 16x16x32 for 32-dim heads, 16x16x16 for 16-dim.
template <typename T>
__device__ __forceinline__ f32x4 plane_qk(uint4 k, uint4 q, f32x4 c) {
  using Qk = typename MfmaOps<T>::Qk;
  return MfmaOps<T>::qk(__builtin_bit_cast(Qk, k), __builtin_bit_cast(Qk, q), c);
}
template <typename T>
__device__ __forceinline__ f32x4 plane_qk(uint2 k, uint2 q, f32x4 c) {
  using Pv = typename MfmaOps<T>::Pv;
  return MfmaOps<T>::pv(__builtin_bit_cast(Pv, k), __builtin_bit_cast(Pv, q), c);
}
template <typename T, int kD, int kKeys>
struct PlaneGeo {
  static_assert(sizeof(T) == 2, "16-bit inputs");
  static_assert((kD == 16 || kD == 32) && kKeys % 16 == 0 && kKeys >= 32 && kKeys <= 128, "tile shape");
  static constexpr int kNB = kKeys / 16;              // 16-key blocks (and at most as many query blocks)
  static constexpr int kFragBytes = kD == 32 ? 16 : 8;  // a lane's share of a K or q row
  using Frag = typename PlaneFrag<kFragBytes>::type;
  static constexpr int kChunks = kD / 8;  // 16-byte chunks per K or V row
  // K rows in LDS: an odd number of 16-byte units, so the 16 rows of one
  // operand read start in distinct bank groups.
  static constexpr int kKStride = kD * 2 + 16;
  static constexpr int kKChunks = kKeys * kChunks;
  // V^T rows: a multiple of 8 elements, an odd number of 16-byte units.
  static constexpr int kVStride = kKeys + 8;
  static constexpr int kPairKeys = 32 * (kNB / 2);  // keys read by 16x16x32 steps
  static constexpr int kVPairSlots = kKeys / 2 * kChunks;
  static constexpr int kDTiles = kD / 16;
  // Position of key j in a V^T row.  Below kPairKeys each 32-key group is
  // stored as the 8-key runs {4g .. 4g+3, 16+4g .. 16+4g+3}, g = 0..3, so the
  // A operand of a 16x16x32 step is one 16-byte read; the keys of an odd
  // last block keep their order (8-byte reads of 4 keys).
  static __device__ __forceinline__ int vt_pos(int j) {
    return j >= kPairKeys ? j : (j & ~31) | (((j >> 2) & 3) << 3) | (((j >> 4) & 1) << 2) | (j & 3);
  }
};

// Query blocks per wave: two, computed interleaved (their products share the
// V^T operand reads, and each one's latencies are covered by the other's
// instructions).
constexpr int kPlaneBlocksPerWave = 2;

// 16-dim heads over at most 80 keys fit 8 waves per SIMD (64 VGPRs) with no
// spills; more resident workgroups keep more of HBM's latency covered.
template <typename T, typename OutT, int kD, int kKeys>
__global__ __launch_bounds__(64 * ((kKeys / 16 + 1) / 2))
__attribute__((amdgpu_waves_per_eu(kD == 16 && kKeys <= 80 ? 8 : 6))) void rbf_plane_kernel(Problem p) {
  using G = PlaneGeo<T, kD, kKeys>;
  using Ops = MfmaOps<T>;
  using Frag = typename G::Frag;
  using FragOps = PlaneFrag<G::kFragBytes>;
  using Qk = typename Ops::Qk;
  using Pv = typename Ops::Pv;
  constexpr int kNB = G::kNB;
  constexpr int kPer = kPlaneBlocksPerWave;
  constexpr int kChunks = G::kChunks;
  constexpr int kFragBytes = G::kFragBytes;
  constexpr uint32_t kOutSize = sizeof(OutT);
  // Range of a query's weight sum that needs no shift.  bf16: weights of at
  // most 2^32 (value products stay far from overflow) and a largest weight
  // of at least 2^-32 / Nk, well inside the normal range, where the hi + lo
  // split keeps 2^-17 of it.  fp16: every weight below 2^15, under the
  // format's 65504, and a sum of at least 2^-3, so the 2^-24 steps of its
  // subnormals are below 2^-21 of the sum.
  constexpr bool kBf16 = __is_same(T, __bf16);
  constexpr float kSumHi = kBf16 ? 0x1p32f : 0x1p15f;
  constexpr float kSumLo = kBf16 ? 0x1p-32f : 0x1p-3f;
  // K pieces a lane loads before the first wait: the whole of K when the
  // workgroup has at least kKeys * kD / 1024 waves (three for 65 queries
  // over 80 keys of 32 dims); smaller workgroups loop for the rest.
  constexpr int kKRounds = 2;

  __shared__ __align__(16) T vt_lds[kD * G::kVStride];
  __shared__ __align__(16) char k_lds[kKeys * G::kKStride];
  __shared__ __align__(16) float c_lds[kKeys];  // folded key values
  // Per key: whether it can contribute (not masked with a finite K row), and
  // per key and 16-byte chunk of V, whether the chunk holds an inf or NaN.
  __shared__ __align__(4) uint8_t k_live[kKeys];
  __shared__ __align__(4) uint8_t v_bad[kKeys * kChunks];

  const int tid = static_cast<int>(threadIdx.x);
  const int nthreads = static_cast<int>(blockDim.x);
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int col = lane & 15;
  const int grp = lane >> 4;

  // XCD-local plane order.  Workgroups are dispatched round-robin over the 8
  // XCDs, so with a plane count that is a multiple of 8, workgroup w runs on
  // XCD w % 8; giving XCD x the contiguous planes x * planes / 8 .. puts the
  // heads of one batch entry on one XCD at the same time.  Where q, k and v
  // are head-transposed views of one projection (the model's sites), a cache
  // line holds rows of several heads, and its L2 then fetches it from HBM
  // once instead of once per XCD.  A bijection of [0, planes).
  const int32_t planes = static_cast<int32_t>(p.B * p.H);
  const int32_t w = static_cast<int32_t>(blockIdx.x);
  const int32_t plane = planes % 8 == 0 ? (w & 7) * (planes / 8) + (w >> 3) : w;
  const int32_t b = static_cast<int32_t>(fast_div(static_cast<uint32_t>(plane), p.h_mul, p.h_shift));
  const int32_t h = plane - b * static_cast<int32_t>(p.H);

  const int32_t n_q = static_cast<int32_t>(p.Nq);
  const int32_t n_k = static_cast<int32_t>(p.Nk);
  const int32_t q_blocks = (n_q + 15) / 16;
  const bool has_bias = p.bias != nullptr;
  const int32_t bias_esize = p.bias_dtype == VECTRA_F32 ? 4 : 2;
  const uint32_t q_row_bytes = static_cast<uint32_t>(p.sq[2]) * 2u;
  const uint32_t k_row_bytes = static_cast<uint32_t>(p.sk[2]) * 2u;
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.sv[2]) * 2u;
  const uint32_t o_row = static_cast<uint32_t>(p.so[2]);
  const uint32_t o_dim = static_cast<uint32_t>(p.so[3]);
  const bool out_vec = p.so[3] == 1 && p.so[2] % 4 == 0 && p.so[1] % 4 == 0 && p.so[0] % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0;

  // Loads go through buffer resources whose extent ends at the last row of
  // the plane (rows past Nq or Nk read as zeros, a bounds check of the
  // hardware), with one per-lane offset computed once and per-round parts in
  // scalar registers.  Piece i of K is row i / kChunks, 16-byte chunk
  // i % kChunks; V pair slot i is rows 2 (i / kChunks) and + 1 of the same
  // chunk.  No row offset reaches 2^32 (the host checks 144 rows of each stride).
  const char* kp = static_cast<const char*>(p.k) + (b * p.sk[0] + h * p.sk[1]) * 2;
  const char* vp = static_cast<const char*>(p.v) + (b * p.sv[0] + h * p.sv[1]) * 2;
  const char* qp = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * 2;
  const auto k_rsrc = plane_rsrc(kp, static_cast<uint32_t>(n_k - 1) * k_row_bytes + kD * 2);
  const auto v_rsrc = plane_rsrc(vp, static_cast<uint32_t>(n_k - 1) * v_row_bytes + kD * 2);
  const auto q_rsrc = plane_rsrc(qp, static_cast<uint32_t>(n_q - 1) * q_row_bytes + kD * 2);
  const uint32_t chunk_off = static_cast<uint32_t>(lane % kChunks) * 16u;
  const uint32_t lane_rows = static_cast<uint32_t>(lane / kChunks);  // row of a piece within a round
  const uint32_t k_lane = lane_rows * k_row_bytes + chunk_off;
  const uint32_t v_lane = 2u * lane_rows * v_row_bytes + chunk_off;
  constexpr int kRowsPerWave = kWave / kChunks;  // K rows (V row pairs) a wave covers per round

  // The coefficient and, per key, the folded value
  //   c_j = log2(e) (bias_j - gamma |k_j|^2)    (-inf past Nk)
  // computed by the lane holding the first chunk of K row j.
  const RawScalar scale_raw = load_raw_scalar(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);
  const char* const bp =
      has_bias ? static_cast<const char*>(p.bias) + (b * p.sbb + h * p.sbh) * bias_esize : nullptr;
  const uint32_t bias_key_bytes = static_cast<uint32_t>(p.sbn) * static_cast<uint32_t>(bias_esize);
  const auto b_rsrc = plane_rsrc(bp, static_cast<uint32_t>(n_k - 1) * bias_key_bytes + bias_esize);
  const uint32_t b_lane = lane_rows * bias_key_bytes;
  // Raw bits of key `row0 + lane / kChunks`'s bias (an fp32 word, or a
  // 16-bit element zero-extended).
  auto bias_of = [&](int row0) -> uint32_t {
    if (!has_bias) return 0u;
    const uint32_t off = b_lane + static_cast<uint32_t>(row0) * bias_key_bytes;
    return p.bias_dtype == VECTRA_F32 ? __builtin_amdgcn_raw_buffer_load_b32(b_rsrc, off, 0, kNt)
                                      : __builtin_amdgcn_raw_buffer_load_b16(b_rsrc, off, 0, kNt);
  };
  auto k_piece = [&](int row0) {
    return load16_buf(k_rsrc, k_lane + static_cast<uint32_t>(row0) * k_row_bytes);
  };
  auto v_pair = [&](int row0, uint4& r0, uint4& r1) {
    const uint32_t off = v_lane + static_cast<uint32_t>(row0) * v_row_bytes;
    r0 = load16_buf(v_rsrc, off);
    r1 = load16_buf(v_rsrc, off + v_row_bytes);
  };
  const int k_base = wave * kWave;  // first K piece (and V pair slot) of this wave
  uint4 kr[kKRounds];
  uint32_t bias_r[kKRounds];
#pragma unroll
  for (int r = 0; r < kKRounds; ++r) {
    kr[r] = make_uint4(0, 0, 0, 0);
    bias_r[r] = 0;
    const int base = k_base + r * nthreads;
    if (base < G::kKChunks) {
      kr[r] = k_piece(base / kChunks);
      bias_r[r] = bias_of(base / kChunks);
    }
  }
  uint4 v0a = make_uint4(0, 0, 0, 0), v0b = v0a;
  if (k_base < G::kVPairSlots) v_pair(2 * (k_base / kChunks), v0a, v0b);
  // This wave's query blocks: kPer * wave + j, j < blocks (1 or 2).
  const int first_block = kPer * wave;
  const int blocks = min(kPer, q_blocks - first_block);
  const uint32_t q_lane = static_cast<uint32_t>(col) * q_row_bytes + static_cast<uint32_t>(grp * kFragBytes);
  Frag qf[kPer];
#pragma unroll
  for (int j = 0; j < kPer; ++j)
    qf[j] = FragOps::load_buf(q_rsrc, q_lane + static_cast<uint32_t>(16 * (first_block + j)) * q_row_bytes);
  const float coef = 2.f * kLog2e * decode_raw_scalar(scale_raw, p.scale_dtype);
  const float half_coef = -0.5f * coef;

  // K into LDS as loaded, and each row's folded value (the kChunks lanes of
  // a row are adjacent; every lane of a wave takes part in the reduction).
  auto put_k = [&](int base, uint4 piece, uint32_t bias_raw) {
    const int row = base / kChunks + static_cast<int>(lane_rows);
    const float sq = reduce_low<kChunks>(frag_norm<T>(piece), OpSum());
    if (base + lane < G::kKChunks) {
      *reinterpret_cast<uint4*>(k_lds + row * G::kKStride + static_cast<int>(chunk_off)) = piece;
      if (chunk_off == 0) {
        float x = 0.f;
        if (has_bias) {
          x = p.bias_dtype == VECTRA_F32    ? __uint_as_float(bias_raw)
              : p.bias_dtype == VECTRA_BF16 ? __uint_as_float(bias_raw << 16)
                                            : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bias_raw)));
        }
        const float c = row < n_k ? fmaf(half_coef, sq, x * kLog2e) : -INFINITY;
        c_lds[row] = c;
        // A key masked by its bias (or past Nk) whose K row is finite gets
        // weight exactly 0 from every finite query.
        k_live[row] = !(row >= n_k || (c == -INFINITY && __builtin_isfinite(sq)));
      }
    }
  };
  // V^T: two keys of one value dim per 32-bit word (rows past Nk read as
  // zeros: their weight is 0, and 0 * a non-finite value would not be).
  auto put_v = [&](int i, uint4 r0, uint4 r1) {
    const int row = 2 * (i / kChunks);
    const int d0 = (i % kChunks) * 8;
    // An all-ones exponent in either 16-bit half: (w & exp) + low carries
    // into that half's top bit, and into nothing else.
    constexpr uint32_t kExp = kBf16 ? 0x7f807f80u : 0x7c007c00u;
    constexpr uint32_t kLow = kBf16 ? 0x00800080u : 0x04000400u;
    auto bad = [&](uint4 r) {
      const uint32_t m = ((r.x & kExp) + kLow) | ((r.y & kExp) + kLow) | ((r.z & kExp) + kLow) | ((r.w & kExp) + kLow);
      return static_cast<uint8_t>((m & 0x80008000u) != 0);
    };
    v_bad[row * kChunks + i % kChunks] = bad(r0);
    v_bad[(row + 1) * kChunks + i % kChunks] = bad(r1);
    const uint32_t w0[4] = {r0.x, r0.y, r0.z, r0.w};
    const uint32_t w1[4] = {r1.x, r1.y, r1.z, r1.w};
    T* dst = vt_lds + d0 * G::kVStride + G::vt_pos(row);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // Elements 2e and 2e + 1 of the chunk, for keys row and row + 1.
      *reinterpret_cast<uint32_t*>(dst + 2 * e * G::kVStride) = __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u);
      *reinterpret_cast<uint32_t*>(dst + (2 * e + 1) * G::kVStride) = __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u);
    }
  };
#pragma unroll
  for (int r = 0; r < kKRounds; ++r) {
    const int base = k_base + r * nthreads;
    if (base < G::kKChunks) put_k(base, kr[r], bias_r[r]);
  }
  if (tid < G::kVPairSlots) put_v(tid, v0a, v0b);
  // Workgroups with fewer waves (fewer query blocks) stage the rest in
  // further rounds.
  for (int base = k_base + kKRounds * nthreads; base < G::kKChunks; base += nthreads)
    put_k(base, k_piece(base / kChunks), bias_of(base / kChunks));
  for (int base = k_base + nthreads; base < G::kVPairSlots; base += nthreads) {
    uint4 r0, r1;
    v_pair(2 * (base / kChunks), r0, r1);
    if (base + lane < G::kVPairSlots) put_v(base + lane, r0, r1);
  }
  static_assert(kRowsPerWave * kChunks == kWave, "pieces of whole rows per wave");

  __syncthreads();  // K, the folded key values and V^T in place

  // 16-key blocks that can contribute: a block whose every key is masked
  // with finite K and V rows adds exact zeros to every sum (bit for bit), so
  // its products are skipped.  Bit t of live_blocks is block t (uniform).
  auto key_live = [&](int j) -> bool {
    if (j >= kKeys) return false;
    uint32_t bad;
    if constexpr (kChunks == 4) {
      bad = *reinterpret_cast<const uint32_t*>(v_bad + 4 * j);
    } else {
      static_assert(kChunks == 2, "16- or 32-dim heads");
      bad = *reinterpret_cast<const uint16_t*>(v_bad + 2 * j);
    }
    return k_live[j] != 0 || bad != 0;
  };
  const uint64_t live_lo = __builtin_amdgcn_ballot_w64(key_live(lane));
  const uint64_t live_hi = kKeys > 64 ? __builtin_amdgcn_ballot_w64(key_live(lane + 64)) : 0;
  uint32_t live_blocks = 0;
#pragma unroll
  for (int t = 0; t < kNB; ++t)
    if (((t < 4 ? live_lo >> (16 * t) : live_hi >> (16 * (t - 4))) & 0xffffu) != 0) live_blocks |= 1u << t;
  live_blocks = __builtin_amdgcn_readfirstlane(live_blocks);

  // Key block t's operand of the first product (read from LDS where it is
  // used rather than held across the pass, which would cost a wave slot).
  const char* const k_op = k_lds + col * G::kKStride + grp * kFragBytes;
  auto kc = [&](int t) { return *reinterpret_cast<const Frag*>(k_op + 16 * t * G::kKStride); };

  const uint32_t one = Ops::kOnePair;
  const Qk ones8 = __builtin_bit_cast(Qk, make_uint4(one, one, one, one));
  const Pv ones4 = __builtin_bit_cast(Pv, make_uint2(one, one));

  // The wave's query blocks against every key of the plane.
  //
  // The logits are taken without the per-query constant -gamma |q|^2
  // (softmax does not see a per-row shift):
  //   x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j).
  // exp2(x) is used unshifted unless the weights' sum, read off the ones
  // product, leaves the range where the 16-bit split of the weights is
  // accurate and the value products cannot overflow; then the block is
  // computed once more with each query's exact maximum subtracted.
  f32x4 acc[kPer][G::kDTiles];
  f32x4 total[kPer];
  // Weights of block t as packed 16-bit hi / lo pairs (keys 4g + 0,1 and 4g + 2,3).
  auto weights = [&](const float (&xt)[4], uint32_t* hi, uint32_t* lo) {
    const float w0 = __builtin_amdgcn_exp2f(xt[0]), w1 = __builtin_amdgcn_exp2f(xt[1]);
    const float w2 = __builtin_amdgcn_exp2f(xt[2]), w3 = __builtin_amdgcn_exp2f(xt[3]);
    Ops::split2(w0, w1, hi[0], lo[0]);
    Ops::split2(w2, w3, hi[1], lo[1]);
  };
  // Logits of key block t for query block j (relative to `shift`, per query column).
  auto logits = [&](int j, int t, float shift, float (&xt)[4]) {
    const f32x4 s = plane_qk<T>(kc(t), qf[j], f32x4{0.f, 0.f, 0.f, 0.f});
    const float4 c = *reinterpret_cast<const float4*>(c_lds + 16 * t + 4 * grp);
    xt[0] = fmaf(coef, s[0], c.x - shift);
    xt[1] = fmaf(coef, s[1], c.y - shift);
    xt[2] = fmaf(coef, s[2], c.z - shift);
    xt[3] = fmaf(coef, s[3], c.w - shift);
  };
  // One pass over the keys for the first `n` query blocks, block pair by
  // block pair of keys, so only the logits of two key blocks per query
  // block are live at a time.
  auto pass = [&](auto n_tag, const float (&shift)[kPer]) {
    constexpr int n = decltype(n_tag)::value;
#pragma unroll
    for (int j = 0; j < n; ++j) {
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) acc[j][u] = f32x4{0.f, 0.f, 0.f, 0.f};
      total[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int pp = 0; pp < kNB / 2; ++pp) {
      if (((live_blocks >> (2 * pp)) & 3u) == 0) continue;
      Qk p_hi[n], p_lo[n];
#pragma unroll
      for (int j = 0; j < n; ++j) {
        float x0[4], x1[4];
        logits(j, 2 * pp, shift[j], x0);
        logits(j, 2 * pp + 1, shift[j], x1);
        uint32_t hi[4], lo[4];
        weights(x0, hi, lo);
        weights(x1, hi + 2, lo + 2);
        p_hi[j] = __builtin_bit_cast(Qk, make_uint4(hi[0], hi[1], hi[2], hi[3]));
        p_lo[j] = __builtin_bit_cast(Qk, make_uint4(lo[0], lo[1], lo[2], lo[3]));
      }
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const Qk a = *reinterpret_cast<const Qk*>(vt_lds + (16 * u + col) * G::kVStride + 32 * pp + 8 * grp);
#pragma unroll
        for (int j = 0; j < n; ++j) {
          acc[j][u] = Ops::qk(a, p_hi[j], acc[j][u]);
          acc[j][u] = Ops::qk(a, p_lo[j], acc[j][u]);
        }
      }
#pragma unroll
      for (int j = 0; j < n; ++j) {
        total[j] = Ops::qk(ones8, p_hi[j], total[j]);
        total[j] = Ops::qk(ones8, p_lo[j], total[j]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kNB % 2 == 1) {
      constexpr int t = kNB - 1;
      if (((live_blocks >> t) & 1u) == 0) return;
      Pv p_hi[n], p_lo[n];
#pragma unroll
      for (int j = 0; j < n; ++j) {
        float x0[4];
        logits(j, t, shift[j], x0);
        uint32_t hi[2], lo[2];
        weights(x0, hi, lo);
        p_hi[j] = __builtin_bit_cast(Pv, make_uint2(hi[0], hi[1]));
        p_lo[j] = __builtin_bit_cast(Pv, make_uint2(lo[0], lo[1]));
      }
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const Pv a = *reinterpret_cast<const Pv*>(vt_lds + (16 * u + col) * G::kVStride + 16 * t + 4 * grp);
#pragma unroll
        for (int j = 0; j < n; ++j) {
          acc[j][u] = Ops::pv(a, p_hi[j], acc[j][u]);
          acc[j][u] = Ops::pv(a, p_lo[j], acc[j][u]);
        }
      }
#pragma unroll
      for (int j = 0; j < n; ++j) {
        total[j] = Ops::pv(ones4, p_hi[j], total[j]);
        total[j] = Ops::pv(ones4, p_lo[j], total[j]);
      }
    }
  };
  // Each query's exact maximum logit in block j (the rare second pass).
  auto row_max = [&](int j) {
    float rmax = -INFINITY;
#pragma unroll
    for (int t = 0; t < kNB; ++t) {
      if (((live_blocks >> t) & 1u) == 0) continue;
      float xt[4];
      logits(j, t, 0.f, xt);
      rmax = fmaxf(rmax, fmaxf(fmaxf(xt[0], xt[1]), fmaxf(xt[2], xt[3])));
    }
    rmax = allreduce_bit32(allreduce_bit16(rmax, OpMax()), OpMax());
    return rmax == -INFINITY ? 0.f : rmax;  // every key masked: the row ends as NaN
  };
  // Every row of the ones product holds the full sum of a query's weights.
  // NaN (a NaN input) fails the test and is recomputed to NaN.  A block
  // that needs no shift is recomputed unshifted, to the same result.
  auto run = [&](auto n_tag) {
    constexpr int n = decltype(n_tag)::value;
    float shift[kPer] = {};
    pass(n_tag, shift);
    bool again = false;
#pragma unroll
    for (int j = 0; j < n; ++j) {
      if (__builtin_amdgcn_ballot_w64(!(total[j][0] >= kSumLo && total[j][0] <= kSumHi))) {
        shift[j] = row_max(j);
        again = true;
      }
    }
    if (again) pass(n_tag, shift);
  };
  if (blocks == kPer) {
    run(std::integral_constant<int, kPer>{});
  } else {
    run(std::integral_constant<int, 1>{});
  }

  char* out_plane = static_cast<char*>(p.out) + (b * p.so[0] + h * p.so[1]) * static_cast<int64_t>(kOutSize);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int32_t out_q = 16 * (first_block + j) + col;
    if (j < blocks && out_q < n_q) {
      // A fully masked row has sum 0 and ends as 0 * inf = NaN.
      const float inv = __builtin_amdgcn_rcpf(total[j][0]);
      const uint32_t row_off = static_cast<uint32_t>(out_q) * o_row;
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const uint32_t off = (row_off + static_cast<uint32_t>(16 * u + 4 * grp) * o_dim) * kOutSize;
        const float y0 = acc[j][u][0] * inv, y1 = acc[j][u][1] * inv, y2 = acc[j][u][2] * inv,
                    y3 = acc[j][u][3] * inv;
        if constexpr (kOutSize == 4) {
          if (out_vec) {
            *reinterpret_cast<float4*>(out_plane + off) = make_float4(y0, y1, y2, y3);
          } else {
            const float ys[4] = {y0, y1, y2, y3};
#pragma unroll
            for (int r = 0; r < 4; ++r) *reinterpret_cast<float*>(out_plane + off + r * o_dim * 4u) = ys[r];
          }
        } else {
          const uint32_t w01 = pack2<OutT>(y0, y1), w23 = pack2<OutT>(y2, y3);
          if (out_vec) {
            *reinterpret_cast<uint2*>(out_plane + off) = make_uint2(w01, w23);
          } else {
            const uint16_t hs[4] = {static_cast<uint16_t>(w01), static_cast<uint16_t>(w01 >> 16),
                                    static_cast<uint16_t>(w23), static_cast<uint16_t>(w23 >> 16)};
#pragma unroll
            for (int r = 0; r < 4; ++r) *reinterpret_cast<uint16_t*>(out_plane + off + r * o_dim * 2u) = hs[r];
          }
        }
      }
    }
  }
}

// ------------------------------------------------------------------- host

// One workgroup per plane, one wave per two 16-query blocks.
template <typename T, typename OutT, int kD, int kKeys>
hipError_t launch_plane_k(Problem& p, hipStream_t s) {
  const int64_t planes = p.B * p.H;
  const int64_t q_blocks = (p.Nq + 15) / 16;
  const int64_t waves = (q_blocks + kPlaneBlocksPerWave - 1) / kPlaneBlocksPerWave;
  if (planes < 1 || q_blocks < 1 || q_blocks > kKeys / 16) return hipErrorInvalidValue;
  void* args[] = {&p};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_plane_kernel<T, OutT, kD, kKeys>),
                         dim3(static_cast<unsigned>(planes)), dim3(static_cast<unsigned>(64 * waves)), args, 0, s);
}

// Tile of the longest axis: 32, 64 or 80 rows (80 covers the 65-token
// comparable sets), or 128 for 16-dim heads.
template <typename T, typename OutT, int kD>
hipError_t launch_plane_d(Problem& p, hipStream_t s) {
  const int64_t rows = p.Nq > p.Nk ? p.Nq : p.Nk;
  if (rows <= 32) return launch_plane_k<T, OutT, kD, 32>(p, s);
  if (rows <= 64) return launch_plane_k<T, OutT, kD, 64>(p, s);
  if (rows <= 80) return launch_plane_k<T, OutT, kD, 80>(p, s);
  if constexpr (kD == 16) {
    if (rows <= 128) return launch_plane_k<T, OutT, kD, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

template <typename T, typename OutT>
hipError_t launch_plane_t(Problem& p, hipStream_t s) {
  switch (p.D) {
    case 16: return launch_plane_d<T, OutT, 16>(p, s);
    case 32: return launch_plane_d<T, OutT, 32>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_plane_bf16_bf16(Problem& p, hipStream_t s);
hipError_t launch_plane_bf16_f32(Problem& p, hipStream_t s);
hipError_t launch_plane_f16_f16(Problem& p, hipStream_t s);
hipError_t launch_plane_f16_f32(Problem& p, hipStream_t s);

}  // namespace vectra
