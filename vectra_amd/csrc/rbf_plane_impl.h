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
// 16x16x16 step.  K and V rows sit in LDS as loaded: the A operand of the
// first product is row l % 16 of a key block, head dims 8g .. 8g+7 (4g ..
// 4g+3 for 16-dim heads), read where it is used; that of the second is read
// transposed from the V rows (ds_read_b64_tr_b16); q goes from HBM straight
// into the B operand.
//
// Per-score arithmetic is one FMA, one exp2 and the 16-bit split of the
// weight:
//  * gamma |k|^2 / 2 and the key bias are folded once per plane into one
//    value per key,
//      c_j = log2(e) (bias_j - gamma |k_j|^2),
//    and the per-query constant -gamma |q|^2 is left out (a softmax row does
//    not see a shift), so the exp2 argument is one FMA of the product,
//      x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j);
//  * each lane adds up the fp32 weights it computes (keys 4g + r of every
//    block), and the four lane groups of a query are summed at the end: two
//    lane swaps, where a product of ones would take a quarter of the matrix
//    instructions and eight more registers;
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
// Outputs leave as non-temporal stores, of whole rows where the layout
// allows: the plane's output is a quarter of its traffic, and written in
// 32-byte pieces through the cache it cost HBM time in the middle of the
// other workgroups' loads.
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
  static constexpr int kKChunks = kKeys * kChunks;  // 16-byte pieces of K (and of V)
  // V rows in LDS, in elements: 16 bytes of padding, as for K.
  static constexpr int kVRow = kD + 8;
  static constexpr int kDTiles = kD / 16;
};

// Query blocks per wave: two, computed interleaved (their products share the
// K and V operand reads, and each one's latencies are covered by the other's
// instructions).
constexpr int kPlaneBlocksPerWave = 2;

// Tiles of at most 80 keys fit 8 waves per SIMD (64 VGPRs) with no spills;
// more resident workgroups keep more of HBM's latency covered.
template <typename T, typename OutT, int kD, int kKeys>
__global__ __launch_bounds__(64 * ((kKeys / 16 + 1) / 2))
__attribute__((amdgpu_waves_per_eu(kKeys <= 80 ? 8 : 6))) void rbf_plane_kernel(Problem p) {
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

  constexpr int kVRow = G::kVRow;
  __shared__ __align__(16) T v_lds[kKeys * kVRow];  // V rows as loaded
  __shared__ __align__(16) char k_lds[kKeys * G::kKStride];
  __shared__ __align__(16) float c_lds[kKeys];  // folded key values
  // Per 16-key block: whether any of its keys can contribute (see below).
  __shared__ __align__(8) uint8_t block_live[8];
  static_assert(kNB <= 8, "one byte per key block");

  args_in_sgprs(p.q, p.k, p.v, p.out, p.scale, p.bias, p.scale_dtype, p.bias_dtype, p.B, p.H, p.Nq, p.Nk);
  args_in_sgprs(p.sq[0], p.sq[1], p.sq[2], p.sk[0], p.sk[1], p.sk[2], p.sv[0], p.sv[1], p.sv[2]);
  args_in_sgprs(p.so[0], p.so[1], p.so[2], p.so[3], p.ssb, p.ssh, p.sbb, p.sbh, p.sbn, p.h_mul, p.h_shift);
  const int tid = static_cast<int>(threadIdx.x);
  // The launch's workgroup size, 64 threads per two query blocks (from Nq
  // rather than blockDim.x, which would be one more dependent scalar load).
  static_assert(kPer == 2, "two query blocks (32 rows) per wave");
  const int nthreads = kWave * ((static_cast<int>(p.Nq) + 31) / 32);
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
  // scalar registers.  Piece i of K (and of V) is row i / kChunks, 16-byte
  // chunk i % kChunks.  No row offset reaches 2^32 (the host checks 144 rows
  // of each stride).
  const char* kp = static_cast<const char*>(p.k) + (b * p.sk[0] + h * p.sk[1]) * 2;
  const char* vp = static_cast<const char*>(p.v) + (b * p.sv[0] + h * p.sv[1]) * 2;
  const char* qp = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * 2;
  const auto k_rsrc = plane_rsrc(kp, static_cast<uint32_t>(n_k - 1) * k_row_bytes + kD * 2);
  const auto v_rsrc = plane_rsrc(vp, static_cast<uint32_t>(n_k - 1) * v_row_bytes + kD * 2);
  const auto q_rsrc = plane_rsrc(qp, static_cast<uint32_t>(n_q - 1) * q_row_bytes + kD * 2);
  const uint32_t chunk_off = static_cast<uint32_t>(lane % kChunks) * 16u;
  const uint32_t lane_rows = static_cast<uint32_t>(lane / kChunks);  // row of a piece within a round
  const uint32_t k_lane = lane_rows * k_row_bytes + chunk_off;
  const uint32_t v_lane = lane_rows * v_row_bytes + chunk_off;
  constexpr int kRowsPerWave = kWave / kChunks;  // K rows (V row pairs) a wave covers per round

  // The coefficient and, per key, the folded value
  //   c_j = log2(e) (bias_j - gamma |k_j|^2)    (-inf past Nk)
  // computed by the kChunks lanes holding K row j.
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
  auto v_piece = [&](int row0) {
    return load16_buf(v_rsrc, v_lane + static_cast<uint32_t>(row0) * v_row_bytes);
  };
  const int k_base = wave * kWave;  // first K and V piece of this wave
  uint4 kr[kKRounds], vr[kKRounds];
  uint32_t bias_r[kKRounds];
#pragma unroll
  for (int r = 0; r < kKRounds; ++r) {
    kr[r] = make_uint4(0, 0, 0, 0);
    vr[r] = kr[r];
    bias_r[r] = 0;
    const int base = k_base + r * nthreads;
    if (base < G::kKChunks) {
      kr[r] = k_piece(base / kChunks);
      bias_r[r] = bias_of(base / kChunks);
      vr[r] = v_piece(base / kChunks);
    }
  }
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

  // One round of staging: K and V pieces base + lane (row base / kChunks +
  // lane / kChunks, 16-byte chunk lane % kChunks) into LDS as loaded, each
  // row's folded value, and whether the round's key blocks can contribute.
  // Rows past Nk read as zeros (their weight is 0, and 0 * a non-finite
  // value would not be).  A round covers whole 16-key blocks (one for
  // 32-dim heads, two for 16-dim), and a block can be skipped if every key
  // in it is masked (by its bias, or past Nk) with finite K and V rows: it
  // gets weight exactly 0 from every finite query and adds exact zeros to
  // every sum, bit for bit.
  auto stage = [&](int base, uint4 kp_, uint4 vp_, uint32_t bias_raw) {
    const int row = base / kChunks + static_cast<int>(lane_rows);
    const bool in = G::kKChunks % kWave == 0 || base + lane < G::kKChunks;
    const float sq = reduce_low<kChunks>(frag_norm<T>(kp_), OpSum());
    float x = 0.f;
    if (has_bias) {
      x = p.bias_dtype == VECTRA_F32    ? __uint_as_float(bias_raw)
          : p.bias_dtype == VECTRA_BF16 ? __uint_as_float(bias_raw << 16)
                                        : static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bias_raw)));
    }
    const float c = row < n_k ? fmaf(half_coef, sq, x * kLog2e) : -INFINITY;
    // An all-ones exponent in either 16-bit half: (w & exp) + low carries
    // into that half's top bit, and into nothing else.
    constexpr uint32_t kExp = kBf16 ? 0x7f807f80u : 0x7c007c00u;
    constexpr uint32_t kLow = kBf16 ? 0x00800080u : 0x04000400u;
    const uint32_t m = ((vp_.x & kExp) + kLow) | ((vp_.y & kExp) + kLow) | ((vp_.z & kExp) + kLow) |
                       ((vp_.w & kExp) + kLow);
    const bool v_bad = (m & 0x80008000u) != 0;
    const bool live = in && ((row < n_k && !(c == -INFINITY && __builtin_isfinite(sq))) || v_bad);
    const uint64_t mask = __builtin_amdgcn_ballot_w64(live);
    if (in) {
      *reinterpret_cast<uint4*>(k_lds + row * G::kKStride + static_cast<int>(chunk_off)) = kp_;
      *reinterpret_cast<uint4*>(v_lds + row * kVRow + static_cast<int>(chunk_off / 2)) = vp_;
      if (chunk_off == 0) c_lds[row] = c;
    }
    if (lane == 0) {
      const int blk = base / kChunks / 16;
      if constexpr (kChunks == 4) {
        block_live[blk] = mask != 0;
      } else {
        static_assert(kChunks == 2, "16- or 32-dim heads");
        block_live[blk] = static_cast<uint32_t>(mask) != 0;
        if (blk + 1 < kNB) block_live[blk + 1] = (mask >> 32) != 0;
      }
    }
  };
#pragma unroll
  for (int r = 0; r < kKRounds; ++r) {
    const int base = k_base + r * nthreads;
    if (base < G::kKChunks) stage(base, kr[r], vr[r], bias_r[r]);
  }
  // Workgroups with fewer waves (fewer query blocks) stage the rest in
  // further rounds.
  for (int base = k_base + kKRounds * nthreads; base < G::kKChunks; base += nthreads)
    stage(base, k_piece(base / kChunks), v_piece(base / kChunks), bias_of(base / kChunks));
  static_assert(kRowsPerWave * kChunks == kWave && kRowsPerWave % 16 == 0, "pieces of whole key blocks per wave");

  __syncthreads();  // K, V, the folded key values and the live blocks in place

  // Bit t of live_blocks: key block t can contribute (uniform).
  uint32_t live_blocks = 0;
  {
    const uint2 bytes = *reinterpret_cast<const uint2*>(block_live);
#pragma unroll
    for (int t = 0; t < kNB; ++t)
      live_blocks |= (((t < 4 ? bytes.x >> (8 * t) : bytes.y >> (8 * (t - 4))) & 1u) << t);
    live_blocks = __builtin_amdgcn_readfirstlane(live_blocks);
  }

  // Key block t's operand of the first product (read from LDS where it is
  // used rather than held across the pass, which would cost a wave slot).
  const char* const k_op = k_lds + col * G::kKStride + grp * kFragBytes;
  auto kc = [&](int t) { return *reinterpret_cast<const Frag*>(k_op + 16 * t * G::kKStride); };


  // The wave's query blocks against every key of the plane.
  //
  // The logits are taken without the per-query constant -gamma |q|^2
  // (softmax does not see a per-row shift):
  //   x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j).
  // exp2(x) is used unshifted unless the weights' sum leaves the range where the 16-bit split of the weights is
  // accurate and the value products cannot overflow; then the block is
  // computed once more with each query's exact maximum subtracted.
  f32x4 acc[kPer][G::kDTiles];
  float total[kPer];  // this lane's share of a query's weight sum (keys 4g + r)
  // Weights of block t as packed 16-bit hi / lo pairs (keys 4g + 0,1 and 4g + 2,3).
  auto weights = [&](const float (&xt)[4], uint32_t* hi, uint32_t* lo, float& sum) {
    const float w0 = __builtin_amdgcn_exp2f(xt[0]), w1 = __builtin_amdgcn_exp2f(xt[1]);
    const float w2 = __builtin_amdgcn_exp2f(xt[2]), w3 = __builtin_amdgcn_exp2f(xt[3]);
    sum += (w0 + w1) + (w2 + w3);
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
  // A query's weight sum: the four lane groups hold keys 4g + r of every block.
  auto reduce_totals = [&](auto n_tag) {
#pragma unroll
    for (int j = 0; j < decltype(n_tag)::value; ++j) total[j] = allreduce_bit32(allreduce_bit16(total[j], OpSum()), OpSum());
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
      total[j] = 0.f;
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
        weights(x0, hi, lo, total[j]);
        weights(x1, hi + 2, lo + 2, total[j]);
        p_hi[j] = __builtin_bit_cast(Qk, make_uint4(hi[0], hi[1], hi[2], hi[3]));
        p_lo[j] = __builtin_bit_cast(Qk, make_uint4(lo[0], lo[1], lo[2], lo[3]));
      }
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        // Lane (dim 16u + col, group g) gets keys 32pp + 4g + 0..3 and
        // 32pp + 16 + 4g + 0..3 of that dim: within a group of 16 lanes,
        // lane i addresses key row 32pp + 4g + i / 4 (+16), dims
        // 16u + 4 (i % 4) .. +3.
        const T* va = v_lds + (32 * pp + 4 * grp + col / 4) * kVRow + 16 * u + 4 * (col % 4);
        const uint2 a0 = lds_read_tr16(va);
        const uint2 a1 = lds_read_tr16(va + 16 * kVRow);
        const Qk a = __builtin_bit_cast(Qk, make_uint4(a0.x, a0.y, a1.x, a1.y));
#pragma unroll
        for (int j = 0; j < n; ++j) {
          acc[j][u] = Ops::qk(a, p_hi[j], acc[j][u]);
          acc[j][u] = Ops::qk(a, p_lo[j], acc[j][u]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (kNB % 2 == 1) {
      constexpr int t = kNB - 1;
      if (((live_blocks >> t) & 1u) == 0) {
        reduce_totals(n_tag);
        return;
      }
      Pv p_hi[n], p_lo[n];
#pragma unroll
      for (int j = 0; j < n; ++j) {
        float x0[4];
        logits(j, t, shift[j], x0);
        uint32_t hi[2], lo[2];
        weights(x0, hi, lo, total[j]);
        p_hi[j] = __builtin_bit_cast(Pv, make_uint2(hi[0], hi[1]));
        p_lo[j] = __builtin_bit_cast(Pv, make_uint2(lo[0], lo[1]));
      }
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const Pv a = __builtin_bit_cast(Pv, lds_read_tr16(v_lds + (16 * t + 4 * grp + col / 4) * kVRow + 16 * u + 4 * (col % 4)));
#pragma unroll
        for (int j = 0; j < n; ++j) {
          acc[j][u] = Ops::pv(a, p_hi[j], acc[j][u]);
          acc[j][u] = Ops::pv(a, p_lo[j], acc[j][u]);
        }
      }
    }
    reduce_totals(n_tag);
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
  // Every lane holds the full sum of its query's weights.  NaN (a NaN
  // input) fails the test and is recomputed to NaN.  A block
  // that needs no shift is recomputed unshifted, to the same result.
  auto run = [&](auto n_tag) {
    constexpr int n = decltype(n_tag)::value;
    float shift[kPer] = {};
    pass(n_tag, shift);
    bool again = false;
#pragma unroll
    for (int j = 0; j < n; ++j) {
      if (__builtin_amdgcn_ballot_w64(!(total[j] >= kSumLo && total[j] <= kSumHi))) {
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
  if constexpr (kOutSize == 2 && G::kDTiles == 2) {
    // 16-bit outputs of 32-dim heads, dense rows: whole rows per store.  A
    // lane holds dims 16u + 4g .. +3 of its query (u = 0, 1); one swap
    // between lane groups g = 2m and 2m + 1 leaves group g with dims
    // 8t .. 8t + 7, t = 2 (g & 1) + g / 2, so each lane stores 16 bytes and
    // a wave's store covers 16 whole rows.
    if (out_vec && p.so[2] % 8 == 0 && p.so[1] % 8 == 0 && p.so[0] % 8 == 0) {
      const uint32_t t = static_cast<uint32_t>(((grp & 1) << 1) | (grp >> 1));
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        if (j >= blocks) continue;
        const float inv = __builtin_amdgcn_rcpf(total[j]);
        uint32_t w[2][2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          w[u][0] = pack2<OutT>(acc[j][u][0] * inv, acc[j][u][1] * inv);
          w[u][1] = pack2<OutT>(acc[j][u][2] * inv, acc[j][u][3] * inv);
        }
        const auto s0 = __builtin_amdgcn_permlane16_swap(w[0][0], w[1][0], false, false);
        const auto s1 = __builtin_amdgcn_permlane16_swap(w[0][1], w[1][1], false, false);
        const int32_t out_q = 16 * (first_block + j) + col;
        if (out_q < n_q) {
          const uint32_t off = (static_cast<uint32_t>(out_q) * o_row + 8u * t) * 2u;
          __builtin_nontemporal_store(u32x4{s0[0], s1[0], s0[1], s1[1]}, reinterpret_cast<u32x4*>(out_plane + off));
        }
      }
      return;
    }
  }
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int32_t out_q = 16 * (first_block + j) + col;
    if (j < blocks && out_q < n_q) {
      // A fully masked row has sum 0 and ends as 0 * inf = NaN.
      const float inv = __builtin_amdgcn_rcpf(total[j]);
      const uint32_t row_off = static_cast<uint32_t>(out_q) * o_row;
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const uint32_t off = (row_off + static_cast<uint32_t>(16 * u + 4 * grp) * o_dim) * kOutSize;
        const float y0 = acc[j][u][0] * inv, y1 = acc[j][u][1] * inv, y2 = acc[j][u][2] * inv,
                    y3 = acc[j][u][3] * inv;
        if constexpr (kOutSize == 4) {
          if (out_vec) {
            __builtin_nontemporal_store(u32x4{__float_as_uint(y0), __float_as_uint(y1), __float_as_uint(y2), __float_as_uint(y3)},
                                        reinterpret_cast<u32x4*>(out_plane + off));
          } else {
            const float ys[4] = {y0, y1, y2, y3};
#pragma unroll
            for (int r = 0; r < 4; ++r) *reinterpret_cast<float*>(out_plane + off + r * o_dim * 4u) = ys[r];
          }
        } else {
          const uint32_t w01 = pack2<OutT>(y0, y1), w23 = pack2<OutT>(y2, y3);
          if (out_vec) {
            typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
            __builtin_nontemporal_store(u32x2{w01, w23}, reinterpret_cast<u32x2*>(out_plane + off));
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
