// Single-tile RBF attention for fp32 inputs on gfx950's fp32 matrix core
// (v_mfma_f32_16x16x4_f32), one workgroup per (b, h) plane and one wave per
// two 16-query blocks: the fp32 counterpart of rbf_plane_kernel
// (rbf_plane_impl.h), instantiated in rbf_plane_f32_f32.hip.
//
// The staging, the folded key values
//   c_j = log2(e) (bias_j - gamma |k_j|^2)    (-inf past Nk)
// and the exp2 argument x = 2 gamma log2(e) q.k + c_j are those of the 16-bit
// kernel.  What differs is the arithmetic of the products, laid out for the
// 16x16x4 instruction (A: row l % 16, deep g; B: column l % 16, deep g; C:
// column l % 16, rows 4g .. 4g+3; l = lane, g = l / 16):
//  * S^T = K . Q^T, one 16-key block in kD / 4 steps.  Step s pairs head dim
//    g * kD / 4 + s of key row 16t + l % 16 (A) with the same dim of query
//    l % 16 (B): a dot product does not see the order of its terms, so each
//    lane reads its kD / 4 contiguous dims of one K row and keeps its query's
//    in registers;
//  * O^T = V^T . P^T, one 16-key block in 4 steps of 4 keys.  Step r takes
//    keys 16t + 4g + r, which are exactly the keys whose weights lane l holds
//    as row r of its part of S^T, so the weights feed the B operand where
//    they are, as fp32 (no 16-bit split); V^T sits in LDS with keys
//    contiguous, so a lane's 4 keys of one value dim are one 16-byte read;
//  * the weight sums are fp32 VALU adds (a lane's 4 keys per block) and two
//    cross-lane steps at the end, not a product;
//  * key blocks past Nk are skipped, and up to 4 keys past the last whole
//    block (65 keys: one) go through the VALU instead of a block of products
//    that would be mostly padding;
//  * as in the 16-bit kernel, a key block (or tail key) whose every key is
//    masked with finite K and V rows adds exact zeros to every sum and is
//    skipped, bit for bit.
// Weights are used unshifted while a query's sum stays in [2^-100, 2^32]
// (value products overflow only for |v| > 2^96, and subnormal weights lie
// under 2^-20 of the sum); outside
// that range (gamma < 0, a query far from every key, biases far from 0) the
// wave's blocks are computed once more with each query's exact maximum
// subtracted.  The distance is not clamped at zero, as in the 16-bit kernel.
// Keys past Nk read as zeros through the buffer bounds and have c_j = -inf.
// A fully masked row ends as 0 * (1 / 0) = NaN, as eager softmax gives.
#pragma once

#include <type_traits>

#include "rbf_common.h"
#include "rbf_kernels.h"
#include "rbf_mfma_ops.h"
#include "rbf_plane_impl.h"

namespace vectra {

template <int kD, int kKeys>
struct Plane32Geo {
  static_assert((kD == 16 || kD == 32) && kKeys % 16 == 0 && kKeys >= 32 && kKeys <= 128, "tile shape");
  static constexpr int kNB = kKeys / 16;     // 16-key blocks (and at most as many query blocks)
  static constexpr int kChunks = kD / 4;     // 16-byte chunks per K or V row
  static constexpr int kSteps = kD / 4;      // 16x16x4 steps of S^T per key block (a lane's dims)
  // K rows in LDS: an odd number of 16-byte units, so the 16 rows of one
  // operand read start in distinct bank groups.
  static constexpr int kKStride = kD * 4 + 16;
  static constexpr int kPieces = kKeys * kChunks;  // 16-byte pieces of K (and of V)
  // V^T rows (floats): keys contiguous, an odd number of 16-byte units.
  static constexpr int kVtStride = kKeys + 4;
  static constexpr int kDTiles = kD / 16;
};

template <int kD, int kKeys>
__global__ __launch_bounds__(64 * ((kKeys / 16 + 1) / 2)) void rbf_plane32_kernel(Problem p) {
  using G = Plane32Geo<kD, kKeys>;
  constexpr int kNB = G::kNB;
  constexpr int kPer = 2;  // query blocks per wave
  constexpr int kChunks = G::kChunks;
  constexpr int kSteps = G::kSteps;
  // Weights are used unshifted while a query's sum stays in [2^-100, 2^32]:
  // then |acc| <= 2^32 * max|v|, so the value products cannot overflow
  // unless |v| exceeds 2^96.  Outside the range the block is recomputed with
  // each query's maximum subtracted.
  constexpr float kSumHi = 0x1p32f;
  constexpr float kSumLo = 0x1p-100f;
  // K pieces and V pieces a lane loads before the first wait: all of them
  // when the workgroup has at least kPieces / 256 waves (three for 65 queries
  // over 80 keys of 32 dims); smaller workgroups loop for the rest.
  constexpr int kRounds = 4;

  __shared__ __align__(16) float vt_lds[kD * G::kVtStride];
  __shared__ __align__(16) char k_lds[kKeys * G::kKStride];
  __shared__ __align__(16) float c_lds[kKeys];  // folded key values
  // Per key: whether it can contribute (not masked with a finite K row), and
  // per key and 16-byte chunk of V, whether the chunk holds an inf or NaN.
  __shared__ __align__(8) uint8_t k_live[kKeys];
  __shared__ __align__(8) uint8_t v_bad[kKeys * kChunks];

  const int tid = static_cast<int>(threadIdx.x);
  const int nthreads = static_cast<int>(blockDim.x);
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int col = lane & 15;
  const int grp = lane >> 4;

  // XCD-local plane order, as in rbf_plane_kernel.
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
  const uint32_t q_row_bytes = static_cast<uint32_t>(p.sq[2]) * 4u;
  const uint32_t k_row_bytes = static_cast<uint32_t>(p.sk[2]) * 4u;
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.sv[2]) * 4u;
  const uint32_t o_row = static_cast<uint32_t>(p.so[2]);
  const uint32_t o_dim = static_cast<uint32_t>(p.so[3]);
  const bool out_vec = p.so[3] == 1 && p.so[2] % 4 == 0 && p.so[1] % 4 == 0 && p.so[0] % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0;

  // Loads through buffer resources that end at the plane's last row (rows
  // past Nq or Nk read as zeros).  Piece i of K or V is row i / kChunks,
  // 16-byte chunk i % kChunks.
  const char* kp = static_cast<const char*>(p.k) + (b * p.sk[0] + h * p.sk[1]) * 4;
  const char* vp = static_cast<const char*>(p.v) + (b * p.sv[0] + h * p.sv[1]) * 4;
  const char* qp = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * 4;
  const auto k_rsrc = plane_rsrc(kp, static_cast<uint32_t>(n_k - 1) * k_row_bytes + kD * 4);
  const auto v_rsrc = plane_rsrc(vp, static_cast<uint32_t>(n_k - 1) * v_row_bytes + kD * 4);
  const auto q_rsrc = plane_rsrc(qp, static_cast<uint32_t>(n_q - 1) * q_row_bytes + kD * 4);
  const uint32_t chunk_off = static_cast<uint32_t>(lane % kChunks) * 16u;
  const uint32_t lane_rows = static_cast<uint32_t>(lane / kChunks);
  const uint32_t k_lane = lane_rows * k_row_bytes + chunk_off;
  const uint32_t v_lane = lane_rows * v_row_bytes + chunk_off;

  const RawScalar scale_raw = load_raw_scalar(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);
  const char* const bp =
      has_bias ? static_cast<const char*>(p.bias) + (b * p.sbb + h * p.sbh) * bias_esize : nullptr;
  const uint32_t bias_key_bytes = static_cast<uint32_t>(p.sbn) * static_cast<uint32_t>(bias_esize);
  const auto b_rsrc = plane_rsrc(bp, static_cast<uint32_t>(n_k - 1) * bias_key_bytes + bias_esize);
  const uint32_t b_lane = lane_rows * bias_key_bytes;
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
  const int base0 = wave * kWave;  // this wave's first piece
  uint4 kr[kRounds], vr[kRounds];
  uint32_t bias_r[kRounds];
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    kr[r] = vr[r] = make_uint4(0, 0, 0, 0);
    bias_r[r] = 0;
    const int base = base0 + r * nthreads;
    if (base < G::kPieces) {
      kr[r] = k_piece(base / kChunks);
      vr[r] = v_piece(base / kChunks);
      bias_r[r] = bias_of(base / kChunks);
    }
  }
  // This wave's query blocks: 2 * wave + j, j < blocks (1 or 2); a lane holds
  // dims grp * kSteps .. + kSteps - 1 of query col of each.
  const int first_block = kPer * wave;
  const int blocks = min(kPer, q_blocks - first_block);
  const uint32_t q_lane = static_cast<uint32_t>(col) * q_row_bytes + static_cast<uint32_t>(grp * kSteps * 4);
  float qf[kPer][kSteps];
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
#pragma unroll
    for (int c = 0; c < kSteps / 4; ++c) {
      const uint4 r = load16_buf(q_rsrc, q_lane + static_cast<uint32_t>(16 * (first_block + j)) * q_row_bytes + 16u * c);
      qf[j][4 * c] = __uint_as_float(r.x);
      qf[j][4 * c + 1] = __uint_as_float(r.y);
      qf[j][4 * c + 2] = __uint_as_float(r.z);
      qf[j][4 * c + 3] = __uint_as_float(r.w);
    }
  }
  const float coef = 2.f * kLog2e * decode_raw_scalar(scale_raw, p.scale_dtype);
  const float half_coef = -0.5f * coef;

  // K into LDS as loaded, each row's folded value by the lane holding its
  // first chunk (a row's kChunks lanes are adjacent), and V^T.
  auto put = [&](int base, uint4 kpiece, uint4 vpiece, uint32_t bias_raw) {
    const int row = base / kChunks + static_cast<int>(lane_rows);
    const float sq = reduce_low<kChunks>(
        fmaf(__uint_as_float(kpiece.w), __uint_as_float(kpiece.w),
             fmaf(__uint_as_float(kpiece.z), __uint_as_float(kpiece.z),
                  fmaf(__uint_as_float(kpiece.y), __uint_as_float(kpiece.y),
                       __uint_as_float(kpiece.x) * __uint_as_float(kpiece.x)))),
        OpSum());
    if (base + lane < G::kPieces) {
      *reinterpret_cast<uint4*>(k_lds + row * G::kKStride + static_cast<int>(chunk_off)) = kpiece;
      const int d0 = static_cast<int>(chunk_off) / 4;
      vt_lds[(d0 + 0) * G::kVtStride + row] = __uint_as_float(vpiece.x);
      vt_lds[(d0 + 1) * G::kVtStride + row] = __uint_as_float(vpiece.y);
      vt_lds[(d0 + 2) * G::kVtStride + row] = __uint_as_float(vpiece.z);
      vt_lds[(d0 + 3) * G::kVtStride + row] = __uint_as_float(vpiece.w);
      // An all-ones exponent: (w & exp) + low carries into the sign bit.
      const uint32_t m = ((vpiece.x & 0x7f800000u) + 0x00800000u) | ((vpiece.y & 0x7f800000u) + 0x00800000u) |
                         ((vpiece.z & 0x7f800000u) + 0x00800000u) | ((vpiece.w & 0x7f800000u) + 0x00800000u);
      v_bad[row * kChunks + static_cast<int>(chunk_off) / 16] = static_cast<uint8_t>(m >> 31);
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
#pragma unroll
  for (int r = 0; r < kRounds; ++r) {
    const int base = base0 + r * nthreads;
    if (base < G::kPieces) put(base, kr[r], vr[r], bias_r[r]);
  }
  // Workgroups with fewer waves (fewer query blocks) stage the rest here.
  for (int base = base0 + kRounds * nthreads; base < G::kPieces; base += nthreads)
    put(base, k_piece(base / kChunks), v_piece(base / kChunks), bias_of(base / kChunks));

  __syncthreads();  // K, the folded key values and V^T in place

  // Keys that can contribute (bit j of live_lo / live_hi) and 16-key blocks
  // holding one (bit t of live_blocks), uniform over the wave.
  auto key_live = [&](int j) -> bool {
    if (j >= kKeys) return false;
    uint32_t bad;
    if constexpr (kChunks == 8) {
      const uint2 r = *reinterpret_cast<const uint2*>(v_bad + 8 * j);
      bad = r.x | r.y;
    } else {
      static_assert(kChunks == 4, "16- or 32-dim heads");
      bad = *reinterpret_cast<const uint32_t*>(v_bad + 4 * j);
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
  auto key_is_live = [&](int kt) { return ((kt < 64 ? live_lo >> kt : live_hi >> (kt - 64)) & 1u) != 0; };

  const char* const k_op = k_lds + col * G::kKStride + grp * kSteps * 4;
  f32x4 acc[kPer][G::kDTiles];
  float total[kPer];

  // The products of key block t for the first `n` query blocks.
  auto block = [&](auto n_tag, int t, const float (&shift)[kPer]) __attribute__((always_inline)) {
    constexpr int n = decltype(n_tag)::value;
    float kf[kSteps];
#pragma unroll
    for (int c = 0; c < kSteps / 4; ++c) {
      const float4 r = *reinterpret_cast<const float4*>(k_op + 16 * t * G::kKStride + 16 * c);
      kf[4 * c] = r.x;
      kf[4 * c + 1] = r.y;
      kf[4 * c + 2] = r.z;
      kf[4 * c + 3] = r.w;
    }
    const float4 cj = *reinterpret_cast<const float4*>(c_lds + 16 * t + 4 * grp);
    float wt[n][4];
#pragma unroll
    for (int j = 0; j < n; ++j) {
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kSteps; ++st) s = MfmaOps<float>::mma(kf[st], qf[j][st], s);
      wt[j][0] = __builtin_amdgcn_exp2f(fmaf(coef, s[0], cj.x - shift[j]));
      wt[j][1] = __builtin_amdgcn_exp2f(fmaf(coef, s[1], cj.y - shift[j]));
      wt[j][2] = __builtin_amdgcn_exp2f(fmaf(coef, s[2], cj.z - shift[j]));
      wt[j][3] = __builtin_amdgcn_exp2f(fmaf(coef, s[3], cj.w - shift[j]));
      total[j] += (wt[j][0] + wt[j][1]) + (wt[j][2] + wt[j][3]);
    }
#pragma unroll
    for (int u = 0; u < G::kDTiles; ++u) {
      const float4 vt = *reinterpret_cast<const float4*>(vt_lds + (16 * u + col) * G::kVtStride + 16 * t + 4 * grp);
      const float vr4[4] = {vt.x, vt.y, vt.z, vt.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
#pragma unroll
        for (int j = 0; j < n; ++j) acc[j][u] = MfmaOps<float>::mma(vr4[r], wt[j][r], acc[j][u]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  // Keys past the last whole 16-key block, when there are at most 4 of them
  // (65 keys: one), take the VALU instead of a block of products that would
  // be mostly padding; key blocks past Nk are skipped (their weights are 0).
  const int whole = n_k / 16;
  const int tail = n_k - 16 * whole;
  const bool valu_tail = tail > 0 && tail <= 4;
  const int mfma_blocks = valu_tail ? whole : (n_k + 15) / 16;
  // Score of tail key kt for query block j: the lane's dims, then the 4
  // lanes of its query's column.
  auto tail_score = [&](int j, int kt) __attribute__((always_inline)) {
    const char* krow = k_lds + kt * G::kKStride + grp * kSteps * 4;
    float part = 0.f;
#pragma unroll
    for (int c = 0; c < kSteps / 4; ++c) {
      const float4 r = *reinterpret_cast<const float4*>(krow + 16 * c);
      part = fmaf(r.x, qf[j][4 * c], part);
      part = fmaf(r.y, qf[j][4 * c + 1], part);
      part = fmaf(r.z, qf[j][4 * c + 2], part);
      part = fmaf(r.w, qf[j][4 * c + 3], part);
    }
    return allreduce_bit32(allreduce_bit16(part, OpSum()), OpSum());
  };
  auto tail_key = [&](auto n_tag, int kt, const float (&shift)[kPer]) __attribute__((always_inline)) {
    constexpr int n = decltype(n_tag)::value;
    // This lane's value dims 16u + 4g + r of key kt.
    float vk[G::kDTiles][4];
#pragma unroll
    for (int u = 0; u < G::kDTiles; ++u)
#pragma unroll
      for (int r = 0; r < 4; ++r) vk[u][r] = vt_lds[(16 * u + 4 * grp + r) * G::kVtStride + kt];
    const float ck = c_lds[kt];
#pragma unroll
    for (int j = 0; j < n; ++j) {
      const float wk = __builtin_amdgcn_exp2f(fmaf(coef, tail_score(j, kt), ck - shift[j]));
      total[j] += grp == 0 ? wk : 0.f;  // the sum is reduced over the 4 lanes of a column
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u)
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[j][u][r] = fmaf(wk, vk[u][r], acc[j][u][r]);
    }
  };
  auto pass = [&](auto n_tag, const float (&shift)[kPer]) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) acc[j][u] = f32x4{0.f, 0.f, 0.f, 0.f};
      total[j] = 0.f;
    }
#pragma unroll
    for (int t = 0; t < kNB; ++t)
      if (t < mfma_blocks && ((live_blocks >> t) & 1u) != 0) block(n_tag, t, shift);
    if (valu_tail)
      for (int kt = 16 * whole; kt < n_k; ++kt)
        if (key_is_live(kt)) tail_key(n_tag, kt, shift);
    // A query's sum: its lane's keys, then the 4 lanes of its column.
#pragma unroll
    for (int j = 0; j < kPer; ++j) total[j] = allreduce_bit32(allreduce_bit16(total[j], OpSum()), OpSum());
  };
  // Each query's exact maximum logit in block j (the rare second pass).
  auto row_max = [&](int j) __attribute__((always_inline)) {
    float rmax = -INFINITY;
    if (valu_tail)
      for (int kt = 16 * whole; kt < n_k; ++kt)
        if (key_is_live(kt)) rmax = fmaxf(rmax, fmaf(coef, tail_score(j, kt), c_lds[kt]));
#pragma unroll
    for (int t = 0; t < kNB; ++t) {
      if (t >= mfma_blocks || ((live_blocks >> t) & 1u) == 0) continue;
      float kf[kSteps];
#pragma unroll
      for (int c = 0; c < kSteps / 4; ++c) {
        const float4 r = *reinterpret_cast<const float4*>(k_op + 16 * t * G::kKStride + 16 * c);
        kf[4 * c] = r.x;
        kf[4 * c + 1] = r.y;
        kf[4 * c + 2] = r.z;
        kf[4 * c + 3] = r.w;
      }
      f32x4 s = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int st = 0; st < kSteps; ++st) s = MfmaOps<float>::mma(kf[st], qf[j][st], s);
      const float4 cj = *reinterpret_cast<const float4*>(c_lds + 16 * t + 4 * grp);
      rmax = fmaxf(rmax, fmaxf(fmaxf(fmaf(coef, s[0], cj.x), fmaf(coef, s[1], cj.y)),
                               fmaxf(fmaf(coef, s[2], cj.z), fmaf(coef, s[3], cj.w))));
    }
    rmax = allreduce_bit32(allreduce_bit16(rmax, OpMax()), OpMax());
    return rmax == -INFINITY ? 0.f : rmax;  // every key masked: the row ends as NaN
  };
  // NaN (a NaN input) fails the range test and is recomputed to NaN.  A
  // block that needs no shift is recomputed unshifted, to the same result.
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

  char* out_plane = static_cast<char*>(p.out) + (b * p.so[0] + h * p.so[1]) * static_cast<int64_t>(4);


#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    const int32_t out_q = 16 * (first_block + j) + col;
    if (j < blocks && out_q < n_q) {
      // A fully masked row has sum 0 and ends as 0 * inf = NaN.
      const float inv = __builtin_amdgcn_rcpf(total[j]);
      const uint32_t row_off = static_cast<uint32_t>(out_q) * o_row;
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const uint32_t off = (row_off + static_cast<uint32_t>(16 * u + 4 * grp) * o_dim) * 4u;
        const float ys[4] = {acc[j][u][0] * inv, acc[j][u][1] * inv, acc[j][u][2] * inv, acc[j][u][3] * inv};
        // Non-temporal: the output is written once and not read back here.
        if (out_vec) {
          __builtin_nontemporal_store(u32x4{__float_as_uint(ys[0]), __float_as_uint(ys[1]), __float_as_uint(ys[2]), __float_as_uint(ys[3])},
                                      reinterpret_cast<u32x4*>(out_plane + off));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) *reinterpret_cast<float*>(out_plane + off + r * o_dim * 4u) = ys[r];
        }
      }
    }
  }
}

// ------------------------------------------------------------------- host

template <int kD, int kKeys>
hipError_t launch_plane32_k(Problem& p, hipStream_t s) {
  const int64_t planes = p.B * p.H;
  const int64_t q_blocks = (p.Nq + 15) / 16;
  const int64_t waves = (q_blocks + 1) / 2;
  if (planes < 1 || q_blocks < 1 || q_blocks > kKeys / 16) return hipErrorInvalidValue;
  void* args[] = {&p};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_plane32_kernel<kD, kKeys>),
                         dim3(static_cast<unsigned>(planes)), dim3(static_cast<unsigned>(64 * waves)), args, 0, s);
}

template <int kD>
hipError_t launch_plane32_d(Problem& p, hipStream_t s) {
  const int64_t rows = p.Nq > p.Nk ? p.Nq : p.Nk;
  if (rows <= 32) return launch_plane32_k<kD, 32>(p, s);
  if (rows <= 64) return launch_plane32_k<kD, 64>(p, s);
  if (rows <= 80) return launch_plane32_k<kD, 80>(p, s);
  if constexpr (kD == 16) {
    if (rows <= 128) return launch_plane32_k<kD, 128>(p, s);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_plane_f32_f32(Problem& p, hipStream_t s);

}  // namespace vectra
