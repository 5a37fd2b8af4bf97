// Single-tile RBF attention on gfx950 matrix cores, one wave per (b, h)
// plane: the kernel template, instantiated per dtype pair in
// rbf_plane_<in>_<out>.hip.
//
// For planes whose query and key axes both fit one tile (self-attention over
// a comparable set: Lq = Lk = 65, head dims 16 and 32) the whole plane is
// one work item of one wave, so no wave ever waits for another:
//
//   S^T = K . Q^T     (16 keys x 16 queries per instruction)
//   O^T = V^T . P^T   (16 value dims x 16 queries)
//
// with the lane layouts listed in rbf_mfma_ops.h (l = lane, g = l / 16).  A
// lane holds the scores of one query (column l % 16) against keys
// 16t + 4g + r; those of key blocks 2p and 2p + 1 are the B operand of one
// 16x16x32 step of the second product over keys read in the order
// {32p + 4g .. +3, 32p + 16 + 4g .. +3}, and an odd last block takes a
// 16x16x16 step.  K stays in the registers it is loaded into as the A operand
// of the first product (row l % 16 of each key block, head dims 8g .. 8g+7,
// or 4g .. 4g+3 for 16-dim heads); V is written transposed into LDS.
//
// Per-score arithmetic is one FMA, one exp2 and the 16-bit split of the
// weight:
//  * gamma |k|^2 / 2, the key bias and the plane's largest bias M are folded
//    once per plane into one value per key,
//      c_j = log2(e) (bias_j - gamma |k_j|^2) - M,
//    and the per-query constant -gamma |q|^2 is left out (a softmax row does
//    not see a shift), so the exp2 argument is one FMA of the product,
//      x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j) - M;
//  * the softmax sum comes from the second product itself: a row of ones in
//    the A operand sums the same hi + lo weights the values are weighted by,
//    so the denominator needs no VALU add and no cross-lane reduction;
//  * no running maximum is kept: if a query's weight sum leaves the range in
//    which the 16-bit split is accurate and the value products cannot
//    overflow (gamma < 0, a query far from every key, extreme biases), its
//    block is computed once more with each query's exact maximum subtracted.
// The distance is not clamped at zero: where rounding makes the expansion
// negative (a query on top of a key), -d and the reference's max(d, 0) = 0
// are both within the expansion's rounding error of the true distance.
//
// Weights are fed to the second product as hi + lo 16-bit pairs (~2^-17 of
// the weight), as in rbf_mfma_kernel.  Keys past Nk have c_j = -inf, and
// their K and V rows are zeroed, so they contribute nothing.  A fully masked
// row ends as 0 * (1 / 0) = NaN, as eager softmax gives.
//
// Scheduling: the grid is persistent (as many one-wave workgroups as fit at
// once); a wave takes slots blockIdx.x, blockIdx.x + gridDim.x, ..., each
// slot mapped to a plane so that an XCD works on contiguous planes.  Right
// after a plane's operands are in place (K in registers; V^T, the folded
// biases and q in LDS) every load of the wave's next plane is issued into
// registers, so its HBM latency overlaps the whole of this plane's products.
// q travels with the prefetch (and waits in LDS) because vector loads return
// in issue order: a q load issued during the plane would wait for the whole
// prefetch.

#pragma once

#include <atomic>

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
  static constexpr int kNB = kKeys / 16;              // 16-key blocks (and 16-query blocks)
  static constexpr int kFragBytes = kD == 32 ? 16 : 8;  // a lane's share of a K or q row
  using Frag = typename PlaneFrag<kFragBytes>::type;
  // V^T rows: a multiple of 8 elements, an odd number of 16-byte units, so
  // the 16 rows of one operand read start in distinct bank groups.
  static constexpr int kVStride = kKeys + 8;
  static constexpr int kPairKeys = 32 * (kNB / 2);  // keys read by 16x16x32 steps
  static constexpr int kVChunks = kD / 8;           // 16-byte chunks per V row
  static constexpr int kVPairSlots = kKeys / 2 * kVChunks;
  static constexpr int kVSlots = (kVPairSlots + kWave - 1) / kWave;
  static constexpr int kBiasSlots = (kNB + 3) / 4;
  static constexpr int kDTiles = kD / 16;
  // Position of key j in a V^T row.  Below kPairKeys each 32-key group is
  // stored as the 8-key runs {4g .. 4g+3, 16+4g .. 16+4g+3}, g = 0..3, so the
  // A operand of a 16x16x32 step is one 16-byte read; the keys of an odd
  // last block keep their order (8-byte reads of 4 keys).
  static __device__ __forceinline__ int vt_pos(int j) {
    return j >= kPairKeys ? j : (j & ~31) | (((j >> 2) & 3) << 3) | (((j >> 4) & 1) << 2) | (j & 3);
  }
};

// Registers holding the loads of one plane other than K.
template <typename T, int kD, int kKeys>
struct PlaneStage {
  using G = PlaneGeo<T, kD, kKeys>;
  typename G::Frag q[G::kNB];
  uint4 v[G::kVSlots][2];
  uint32_t bias[G::kBiasSlots];
  uint32_t bias_misalign;
  RawScalar scale;
};

template <typename T, typename OutT, int kD, int kKeys>
__global__ __launch_bounds__(64) void rbf_plane_kernel(Problem p) {
  using G = PlaneGeo<T, kD, kKeys>;
  using Ops = MfmaOps<T>;
  using Frag = typename G::Frag;
  using FragOps = PlaneFrag<G::kFragBytes>;
  using Stage = PlaneStage<T, kD, kKeys>;
  using Qk = typename Ops::Qk;
  using Pv = typename Ops::Pv;
  constexpr int kNB = G::kNB;
  constexpr int kVChunks = G::kVChunks;
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

  __shared__ __align__(16) T vt_lds[kD * G::kVStride];
  __shared__ __align__(16) float bias_lds[kKeys];
  __shared__ __align__(16) Frag q_lds[kNB][kWave];

  const int lane = threadIdx.x;
  const int col = lane & 15;
  const int grp = lane >> 4;

  const int32_t planes = static_cast<int32_t>(p.B * p.H);
  int32_t slot = static_cast<int32_t>(blockIdx.x);
  if (slot >= planes) return;  // one-wave workgroups: no barrier to miss
  // XCD-local plane order.  Workgroups are dispatched round-robin over the 8
  // XCDs, so with a grid and a plane count that are multiples of 8, slot s
  // runs on XCD s % 8; giving XCD x the contiguous planes x * planes / 8 ..
  // puts the heads of one batch entry on one XCD at the same time.  Where
  // q, k and v are head-transposed views of one projection (the model's
  // sites), a cache line holds rows of several heads, and its L2 then
  // fetches it from HBM once instead of once per XCD.  A bijection of
  // [0, planes).
  const int32_t grid = static_cast<int32_t>(gridDim.x);
  const bool xcd_order = grid % 8 == 0 && planes % 8 == 0;
  const int32_t per_xcd = planes / 8;
  auto plane_of = [&](int32_t s) { return xcd_order ? (s & 7) * per_xcd + (s >> 3) : s; };
  int32_t plane = plane_of(slot);
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

  auto plane_bh = [&](int32_t pl, int32_t& b, int32_t& h) {
    b = static_cast<int32_t>(fast_div(static_cast<uint32_t>(pl), p.h_mul, p.h_shift));
    h = pl - b * static_cast<int32_t>(p.H);
  };

  // Per-lane byte offsets inside a plane of the first row each load slot
  // reads, and of the last row (every offset is clamped to it, so rows past
  // Nq or Nk read the last row, in bounds, and no load is behind a
  // data-dependent branch).  Slot t of K and q is rows 16t + col, slot s of
  // V the row pair starting at 2 * (lane / chunks) + s * 128 / chunks.
  const uint32_t frag_off = static_cast<uint32_t>(grp * kFragBytes);
  const uint32_t k_first = static_cast<uint32_t>(col) * k_row_bytes + frag_off;
  const uint32_t k_last = static_cast<uint32_t>(n_k - 1) * k_row_bytes + frag_off;
  const uint32_t q_first = static_cast<uint32_t>(col) * q_row_bytes + frag_off;
  const uint32_t q_last = static_cast<uint32_t>(n_q - 1) * q_row_bytes + frag_off;
  const uint32_t chunk_off = static_cast<uint32_t>(lane % kVChunks) * 16u;
  const uint32_t v_first = static_cast<uint32_t>(2 * (lane / kVChunks)) * v_row_bytes + chunk_off;
  const uint32_t v_last = static_cast<uint32_t>(n_k - 1) * v_row_bytes + chunk_off;

  // Issues every load of plane `pl`: K into `kdst` (the A operand of the
  // first product, as loaded), the rest into `st`.  Rows past Nk are copies
  // of row Nk - 1; their folded key value is -inf, so their weights are 0.
  auto issue = [&](Stage& st, Frag (&kdst)[kNB], int32_t pl) {
    int32_t b, h;
    plane_bh(pl, b, h);
    const char* kp = static_cast<const char*>(p.k) + (b * p.sk[0] + h * p.sk[1]) * 2;
    const char* vp = static_cast<const char*>(p.v) + (b * p.sv[0] + h * p.sv[1]) * 2;
    const char* qp = static_cast<const char*>(p.q) + (b * p.sq[0] + h * p.sq[1]) * 2;
    // Opaque copies: offsets derived from them are recomputed here (one add
    // and one min per load) instead of being hoisted into a register each.
    uint32_t kf0 = k_first, qf0 = q_first, vf0 = v_first;
    asm volatile("" : "+v"(kf0), "+v"(qf0), "+v"(vf0));
#pragma unroll
    for (int t = 0; t < kNB; ++t)
      kdst[t] = FragOps::load_stream(kp + min(kf0 + 16u * t * k_row_bytes, k_last));
#pragma unroll
    for (int t = 0; t < kNB; ++t)
      st.q[t] = FragOps::load_stream(qp + min(qf0 + 16u * t * q_row_bytes, q_last));
#pragma unroll
    for (int s = 0; s < G::kVSlots; ++s) {
      if (lane + kWave * s < G::kVPairSlots) {
        const uint32_t first = vf0 + static_cast<uint32_t>(s * 128 / kVChunks) * v_row_bytes;
        st.v[s][0] = load16_stream(vp + min(first, v_last));
        st.v[s][1] = load16_stream(vp + min(first + v_row_bytes, v_last));
      }
    }
    if (has_bias) {
      const char* bp = static_cast<const char*>(p.bias) + (b * p.sbb + h * p.sbh) * bias_esize;
      st.bias_misalign = base_misalign(bp);
#pragma unroll
      for (int i = 0; i < G::kBiasSlots; ++i) {
        const uint32_t key = static_cast<uint32_t>(min(16 * (grp + 4 * i) + col, n_k - 1));
        st.bias[i] = load_raw_scalar32(bp, st.bias_misalign, key * static_cast<uint32_t>(p.sbn), p.bias_dtype).word;
      }
    }
    st.scale = load_raw_scalar(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);
  };

  float coef = 0.f;

  // Puts a staged plane in place: V^T, the folded key values and q into LDS
  // (K stays in the registers `kc` it was loaded into).
  auto publish = [&](const Stage& st, const Frag (&kc)[kNB]) {
    coef = 2.f * kLog2e * decode_raw_scalar(st.scale, p.scale_dtype);
    float k_sq[kNB];
#pragma unroll
    for (int t = 0; t < kNB; ++t)
      k_sq[t] = allreduce_bit32(allreduce_bit16(frag_norm<T>(kc[t]), OpSum()), OpSum());
    // Biases (log2 units) of keys 16t + col for t = grp + 4i; -inf past Nk.
    float bl[G::kBiasSlots];
    float top = -INFINITY;
#pragma unroll
    for (int i = 0; i < G::kBiasSlots; ++i) {
      const int32_t key = 16 * (grp + 4 * i) + col;
      float x = -INFINITY;
      if (grp + 4 * i < kNB && key < n_k) {
        x = 0.f;
        if (has_bias) {
          const uint32_t bytes = static_cast<uint32_t>(key) * static_cast<uint32_t>(p.sbn) * bias_esize +
                                 st.bias_misalign;
          x = decode_raw_scalar(RawScalar{st.bias[i], (bytes & 2u) * 8u}, p.bias_dtype) * kLog2e;
        }
      }
      bl[i] = x;
      top = fmaxf(top, x);
    }
    top = reduce_wave(top, OpMax());
    if (top == -INFINITY) top = 0.f;  // every key masked: the rows end as NaN
#pragma unroll
    for (int i = 0; i < G::kBiasSlots; ++i) {
      const int t = grp + 4 * i;
      if (t < kNB) {
        // k_sq[4i + grp], picked by the lane group (the same three masks
        // serve every slot).
        float sq = k_sq[4 * i];
        if (4 * i + 1 < kNB) sq = grp == 1 ? k_sq[4 * i + 1] : sq;
        if (4 * i + 2 < kNB) sq = grp == 2 ? k_sq[4 * i + 2] : sq;
        if (4 * i + 3 < kNB) sq = grp == 3 ? k_sq[4 * i + 3] : sq;
        bias_lds[16 * t + col] = fmaf(-0.5f * coef, sq, bl[i] - top);
      }
    }
    // V^T: two keys of one value dim per 32-bit word; rows past Nk zeroed
    // (their weight is 0, and 0 * a non-finite copy would not be).
#pragma unroll
    for (int s = 0; s < G::kVSlots; ++s) {
      const int slot = lane + kWave * s;
      if (slot < G::kVPairSlots) {
        const int row = 2 * (slot / kVChunks);
        const int d0 = (slot % kVChunks) * 8;
        const uint4 r0 = row < n_k ? st.v[s][0] : make_uint4(0, 0, 0, 0);
        const uint4 r1 = row + 1 < n_k ? st.v[s][1] : make_uint4(0, 0, 0, 0);
        const uint32_t w0[4] = {r0.x, r0.y, r0.z, r0.w};
        const uint32_t w1[4] = {r1.x, r1.y, r1.z, r1.w};
        T* dst = vt_lds + d0 * G::kVStride + G::vt_pos(row);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // Elements 2e and 2e + 1 of the chunk, for keys row and row + 1.
          *reinterpret_cast<uint32_t*>(dst + 2 * e * G::kVStride) = __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100u);
          *reinterpret_cast<uint32_t*>(dst + (2 * e + 1) * G::kVStride) =
              __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302u);
        }
      }
    }
#pragma unroll
    for (int t = 0; t < kNB; ++t) q_lds[t][lane] = st.q[t];
  };

  const uint32_t one = Ops::kOnePair;
  const Qk ones8 = __builtin_bit_cast(Qk, make_uint4(one, one, one, one));
  const Pv ones4 = __builtin_bit_cast(Pv, make_uint2(one, one));

  // One block of 16 query rows against every key of the plane; `out_plane`
  // is the plane's output base.
  //
  // The logits are taken relative to the plane's largest bias, without the
  // per-query constant -gamma |q|^2 (softmax does not see a per-row shift):
  //   x = 2 gamma log2(e) q.k + c_j = log2(e) (-gamma (d - |q|^2) + bias_j) - M.
  // exp2(x) is used unshifted unless the weights' sum, read off the ones
  // product, leaves the range where the 16-bit split of the weights is
  // accurate and the value products cannot overflow; then the block is
  // computed once more with each query's exact maximum subtracted.
  auto query_block = [&](const Frag (&kc)[kNB], char* out_plane, int32_t qb) {
    // The folded key values are re-read from LDS per block rather than held
    // in registers across blocks.
    asm volatile("" ::: "memory");
    const Frag qf = q_lds[qb][lane];
    f32x4 acc[G::kDTiles];
    f32x4 total;
    // Weights of block t as packed 16-bit hi / lo pairs (keys 4g + 0,1 and 4g + 2,3).
    auto weights = [&](const float (&xt)[4], uint32_t* hi, uint32_t* lo) {
      const float w0 = __builtin_amdgcn_exp2f(xt[0]), w1 = __builtin_amdgcn_exp2f(xt[1]);
      const float w2 = __builtin_amdgcn_exp2f(xt[2]), w3 = __builtin_amdgcn_exp2f(xt[3]);
      Ops::split2(w0, w1, hi[0], lo[0]);
      Ops::split2(w2, w3, hi[1], lo[1]);
    };
    // Logits of key block t (relative to `shift`, per query column).
    auto logits = [&](int t, float shift, float (&xt)[4]) {
      const f32x4 s = plane_qk<T>(kc[t], qf, f32x4{0.f, 0.f, 0.f, 0.f});
      const float4 c = *reinterpret_cast<const float4*>(bias_lds + 16 * t + 4 * grp);
      xt[0] = fmaf(coef, s[0], c.x - shift);
      xt[1] = fmaf(coef, s[1], c.y - shift);
      xt[2] = fmaf(coef, s[2], c.z - shift);
      xt[3] = fmaf(coef, s[3], c.w - shift);
    };
    // One pass over the keys, block pair by block pair, so only the logits
    // of two blocks are live at a time.
    auto pass = [&](float shift) {
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      total = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int pp = 0; pp < kNB / 2; ++pp) {
        float x0[4], x1[4];
        logits(2 * pp, shift, x0);
        logits(2 * pp + 1, shift, x1);
        uint32_t hi[4], lo[4];
        weights(x0, hi, lo);
        weights(x1, hi + 2, lo + 2);
        const Qk p_hi = __builtin_bit_cast(Qk, make_uint4(hi[0], hi[1], hi[2], hi[3]));
        const Qk p_lo = __builtin_bit_cast(Qk, make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
        for (int u = 0; u < G::kDTiles; ++u) {
          const Qk a = *reinterpret_cast<const Qk*>(vt_lds + (16 * u + col) * G::kVStride + 32 * pp + 8 * grp);
          acc[u] = Ops::qk(a, p_hi, acc[u]);
          acc[u] = Ops::qk(a, p_lo, acc[u]);
        }
        total = Ops::qk(ones8, p_hi, total);
        total = Ops::qk(ones8, p_lo, total);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (kNB % 2 == 1) {
        constexpr int t = kNB - 1;
        float x0[4];
        logits(t, shift, x0);
        uint32_t hi[2], lo[2];
        weights(x0, hi, lo);
        const Pv p_hi = __builtin_bit_cast(Pv, make_uint2(hi[0], hi[1]));
        const Pv p_lo = __builtin_bit_cast(Pv, make_uint2(lo[0], lo[1]));
#pragma unroll
        for (int u = 0; u < G::kDTiles; ++u) {
          const Pv a = *reinterpret_cast<const Pv*>(vt_lds + (16 * u + col) * G::kVStride + 16 * t + 4 * grp);
          acc[u] = Ops::pv(a, p_hi, acc[u]);
          acc[u] = Ops::pv(a, p_lo, acc[u]);
        }
        total = Ops::pv(ones4, p_hi, total);
        total = Ops::pv(ones4, p_lo, total);
      }
    };
    // Each query's exact maximum logit (the rare second pass).
    auto row_max = [&]() {
      float top = -INFINITY;
#pragma unroll
      for (int t = 0; t < kNB; ++t) {
        float xt[4];
        logits(t, 0.f, xt);
        top = fmaxf(top, fmaxf(fmaxf(xt[0], xt[1]), fmaxf(xt[2], xt[3])));
      }
      top = allreduce_bit32(allreduce_bit16(top, OpMax()), OpMax());
      return top == -INFINITY ? 0.f : top;  // every key masked: the row ends as NaN
    };
    pass(0.f);
    // Every row of the ones product holds the full sum of this query's
    // weights.  NaN (a NaN input) fails the test and is recomputed to NaN.
    if (__builtin_amdgcn_ballot_w64(!(total[0] >= kSumLo && total[0] <= kSumHi))) pass(row_max());

    const int32_t q_row = 16 * qb + col;
    if (q_row < n_q) {
      // A fully masked row has sum 0 and ends as 0 * inf = NaN.
      const float inv = __builtin_amdgcn_rcpf(total[0]);
      const uint32_t row_off = static_cast<uint32_t>(q_row) * o_row;
#pragma unroll
      for (int u = 0; u < G::kDTiles; ++u) {
        const uint32_t off = (row_off + static_cast<uint32_t>(16 * u + 4 * grp) * o_dim) * kOutSize;
        const float y0 = acc[u][0] * inv, y1 = acc[u][1] * inv, y2 = acc[u][2] * inv, y3 = acc[u][3] * inv;
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
  };

  // One plane: its K is in `kc`; the next plane's K goes to `kn`.  Returns
  // false after the wave's last plane.
  Stage st;
  auto step = [&](const Frag (&kc)[kNB], Frag (&kn)[kNB]) -> bool {
    publish(st, kc);
    // LDS is private to the wave and its instructions run in order; the
    // fence only keeps the compiler from moving LDS accesses across here.
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    int32_t b, h;
    plane_bh(plane, b, h);
    char* out_plane = static_cast<char*>(p.out) + (b * p.so[0] + h * p.so[1]) * static_cast<int64_t>(kOutSize);
    const int32_t next_slot = slot + grid;
    const bool more = next_slot < planes;
    const int32_t next = more ? plane_of(next_slot) : 0;
    if (more) issue(st, kn, next);  // in flight while this plane is reduced
    for (int32_t qb = 0; qb < q_blocks; ++qb) query_block(kc, out_plane, qb);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    slot = next_slot;
    plane = next;
    return more;
  };

  Frag k0[kNB], k1[kNB];
  issue(st, k0, plane);
  while (step(k0, k1) && step(k1, k0)) {
  }
}

// ------------------------------------------------------------------- host

// One-wave workgroups of an instantiation that fit on a compute unit at once.
template <typename T, typename OutT, int kD, int kKeys>
int plane_resident_waves() {
  static std::atomic<int> cached{0};
  int n = cached.load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&rbf_plane_kernel<T, OutT, kD, kKeys>), 64, 0) != hipSuccess ||
        n < 1)
      n = 1;
    cached.store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename T, typename OutT, int kD, int kKeys>
hipError_t launch_plane_k(Problem& p, hipStream_t s) {
  const int64_t planes = p.B * p.H;
  int64_t waves = static_cast<int64_t>(plane_resident_waves<T, OutT, kD, kKeys>()) *
                  (p.compute_units > 0 ? p.compute_units : 1);
  if (waves > planes) waves = planes;
  if (waves >= 8) waves -= waves % 8;  // whole XCD rounds (see the kernel)
  void* args[] = {&p};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_plane_kernel<T, OutT, kD, kKeys>),
                         dim3(static_cast<unsigned>(waves)), dim3(64), args, 0, s);
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
