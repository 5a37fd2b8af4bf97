// Streamed key tiles for long key axes on gfx950 matrix cores: the kernel
// template, instantiated per dtype pair in rbf_tile_<in>_<out>.hip.
//
// A work item is one (b, h) plane and a block of 16 * kCB * kWaves query
// rows; a workgroup of kWaves waves streams the plane's keys through LDS in
// tiles of kKeys, and every wave reduces 16 * kCB queries (kCB 16-column
// blocks) against each tile:
//
//   S^T = K . Q^T     (16 keys x 16 queries per instruction, 32-deep steps)
//   O^T = V^T . P^T   (16 value dims x 16 queries)
//
// with the lane layouts of rbf_mfma_ops.h.  A K fragment read from LDS feeds
// the products of every query block of the wave, and so does a V^T fragment:
// two blocks per wave halve the LDS traffic per product, four quarter it.
//
// Per-score arithmetic is one FMA, one exp2 and the 16-bit split of the
// weight:
//  * -|q|^2 / 2 is the accumulator the first product starts from (one value
//    per query column), so S = q.k - |q|^2 / 2;
//  * gamma |k|^2 / 2 and the key bias are folded per tile into one value per
//    key, c_j = log2(e) bias_j - gamma log2(e) |k_j|^2 (-inf past Nk);
//  * x = 2 gamma log2(e) S + c_j = log2(e) (-gamma d + bias_j);
//  * the softmax sum comes from the second product: a row of ones in its A
//    operand sums the same hi + lo weights the values are weighted by.
// Without a bias and with gamma >= 0, x <= 0 (d >= 0 up to rounding), so
// exp2(x) is used as the weight directly: one pass over the keys, no running
// maximum and no rescaling.  If a query's weight sum then ends below the
// range in which the 16-bit split is accurate (the query is far from every
// key), and always with a bias or gamma < 0, the item is computed exactly:
// one pass finds each query's largest logit, a second subtracts it.
// Weights are fed to the second product as hi + lo 16-bit pairs (~2^-17 of
// each weight).  The distance is not clamped at zero: where rounding makes
// the expansion negative, -d and the reference's max(d, 0) = 0 are both
// within the expansion's rounding error of the true distance.
//
// Fast pass (one pass, long key axes): with at least kFastKeys keys, the
// single pass first runs with each weight rounded once to fp16 (to nearest,
// 2^-11 of the weight) and fp16 values (bf16 values converted to nearest as
// they are staged: exact in fp16's normal range, within 2^-25 below it), one
// product instead of the hi and lo pair and no split.  The result is the
// exact weighted mean under the rounded weights w^_j = w_j + r_j, so output
// o^ differs from o by sum_j r_j (v_j - o) / T (T = sum_j w^_j): the
// rounding errors of independent weights add up like a random walk.  With
// |r_j| <= 2^-11 w_j (normal fp16 weights; an error uniform over that step
// has deviation 2^-11 w_j / sqrt(3)) and |v_j - o| <= max|v| + |o^|, the
// walk's deviation is at most
//     sigma = 2^-11 / sqrt(3) (max|v| + |o^|) sqrt(sum_j w^_j^2) / T,
// plus 2^-25 per key (weights below fp16's normal range, worst case) and
// 2^-25 for the values' conversion.  The item keeps the fast result only if
// kFastSigmas * sigma + those terms fit the 16-bit paths' accuracy contract
// (kGateAtol + kGateRtol |o^|) for every output, every weight sum T is at
// least kFastSum (weights are at most 1, so at least T keys carry the sum
// and the walk has that many terms), and every accumulator is finite (a bf16
// value of 2^16 or more becomes inf in fp16, and inf times any weight, 0
// included, is not finite); otherwise the item takes the split pass above.
// sum_j w^_j^2 is the diagonal of the fp16 weights' product with
// themselves (one more product per query block and key pair, the weight
// fragment as both operands), and max|v| is taken over the values as they
// are staged.
//
// Scheduling: persistent workgroups take items in a fixed order.  With a
// grid and an item count that are multiples of the 8 XCDs (workgroups are
// dispatched round-robin over them), the items are ordered so that every
// item of a plane runs on one XCD, whose L2 then serves the plane's K and V
// to all of them.  K and V tiles are stored row-major in LDS, as loaded; the
// A operand of O^T is read with gfx950's transposing LDS read.  Tiles are
// double-buffered: while a tile is reduced the next one is in flight into
// registers and is written to the other buffer afterwards, with one barrier
// per tile.

#pragma once

#include <atomic>

#include "rbf_common.h"
#include "rbf_kernels.h"
#include "rbf_mfma_ops.h"

namespace vectra {

template <typename T, int kD, int kKeys, int kWaves, int kCB>
struct TileGeo {
  static_assert(sizeof(T) == 2, "16-bit inputs");
  static_assert(kD % 32 == 0 && kKeys % 32 == 0, "whole 32-deep steps and key pairs");
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kQRows = 16 * kCB * kWaves;  // query rows per item
  static constexpr int kKSteps = kD / 32;     // 32-deep steps of S^T
  static constexpr int kPairs = kKeys / 32;   // 32-key steps of O^T
  static constexpr int kDTiles = kD / 16;
  static constexpr int kChunks = kD / 8;  // 16-byte chunks per K or V row
  // K and V are stored row-major, as loaded.  K rows: a multiple of 8
  // elements and an odd multiple of 16 bytes, so the 16 rows one 16-byte
  // operand read touches start in distinct bank groups.  V rows: an odd
  // multiple of 32 bytes, so the 4 x 32-byte row pieces of one transposing
  // read (8 rows per 256 bytes of banks) do not collide.
  static constexpr int kKStride = kD + 8;
  static constexpr int kVStride = kD + 16;
  static constexpr int kKBytes = kKeys * kKStride * 2;
  static constexpr int kVBytes = kKeys * kVStride * 2;
  static constexpr int kBufBytes = kKBytes + kVBytes + kKeys * 4;  // + c_j
  static constexpr int kSlots = (kKeys * kChunks + kThreads - 1) / kThreads;
  static constexpr bool kFull = kSlots * kThreads == kKeys * kChunks;
};

// Registers holding one tile's loads.  Slot s of a thread is chunk
// slot % kChunks of key slot / kChunks (slot = tid + s * threads), of K and
// of V; the thread holding chunk 0 of a key also loads its bias.
template <typename T, int kD, int kKeys, int kWaves, int kCB>
struct TileStage {
  using G = TileGeo<T, kD, kKeys, kWaves, kCB>;
  uint4 k[G::kSlots];
  uint4 v[G::kSlots];
  uint32_t bias[G::kSlots];
  uint32_t bias_misalign;
};

// Pass kinds of one item, as template arguments of the pass code.
enum TilePass : int { kPassSum = 0, kPassMax = 1, kPassShifted = 2, kPassFast = 3 };
template <int kKind>
struct PassKind {
  static constexpr int value = kKind;
};

// The fast pass: tried for key axes of at least kFastKeys keys, kept if every
// query's weight sum is at least kFastSum and kFastSigmas deviations of its
// rounding error fit the accuracy contract of the 16-bit paths (rtol 1e-3,
// atol 1e-4 against the eager fp32 result) at every output (see the header
// comment).
constexpr int32_t kFastKeys = 1024;
constexpr float kFastSum = 256.f;
constexpr float kFastSigmas = 4.f;
constexpr float kGateAtol = 1e-4f, kGateRtol = 1e-3f;
constexpr float kFastWalk = kFastSigmas * 0x1p-11f * 0.57735026919f;  // kFastSigmas 2^-11 / sqrt(3)

// Two query blocks per wave at three waves per SIMD (at most 168 VGPRs)
// for 32-dim heads; four blocks at two waves per SIMD for 64-dim heads (each
// K and V^T fragment, and each tile's staging, then serve 64 queries per
// wave: 10 % faster at config 4 than two blocks at three waves); 128-dim
// heads keep two blocks at two waves.
template <typename T, typename OutT, int kD, int kKeys, int kWaves, int kCB>
__global__ __launch_bounds__(64 * kWaves) __attribute__((amdgpu_waves_per_eu(kD <= 64 && kCB <= 2 ? 3 : 2))) void
rbf_tile_kernel(Problem p, int32_t q_blocks) {
  using G = TileGeo<T, kD, kKeys, kWaves, kCB>;
  using Ops = MfmaOps<T>;
  using Stage = TileStage<T, kD, kKeys, kWaves, kCB>;
  using Qk = typename Ops::Qk;
  constexpr int kThreads = G::kThreads;
  constexpr int kChunks = G::kChunks;
  constexpr int kKSteps = G::kKSteps;
  constexpr int kDTiles = G::kDTiles;
  constexpr uint32_t kOutSize = sizeof(OutT);
  // Weight sums that need no exact pass: bf16 weights are at most 1 and the
  // largest one at least 2^-32 / Nk, far inside the normal range, where the
  // hi + lo split keeps 2^-17 of it; fp16's subnormal steps of 2^-24 stay
  // below 2^-21 of a sum of at least 2^-3.
  constexpr bool kBf16 = __is_same(T, __bf16);
  constexpr float kSumLo = kBf16 ? 0x1p-32f : 0x1p-3f;
  typedef _Float16 h2v __attribute__((ext_vector_type(2)));
  // Fast pass statistic: the largest |v| this thread staged in the pass (fp32
  // for bf16 inputs, packed fp16 for fp16 inputs).
  float vmax = 0.f;
  h2v vmax16 = {0, 0};

  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ int32_t exact_flag[2];
  __shared__ int32_t split_flag[2];  // the fast pass did not hold
  __shared__ float vmax_wave[2][kWaves];  // the fast pass's max |v| per wave
  __shared__ int32_t abort_flag[2];  // the fast pass was abandoned early

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;
  const int grp = lane >> 4;

  const int32_t n_q = static_cast<int32_t>(p.Nq);
  const int32_t n_k = static_cast<int32_t>(p.Nk);
  const int32_t items = static_cast<int32_t>(p.B * p.H) * q_blocks;
  const int32_t tiles = (n_k + kKeys - 1) / kKeys;
  const bool has_bias = p.bias != nullptr;
  const int32_t bias_esize = p.bias_dtype == VECTRA_F32 ? 4 : 2;
  const uint32_t q_row_bytes = static_cast<uint32_t>(p.sq[2]) * 2u;
  const uint32_t k_row_bytes = static_cast<uint32_t>(p.sk[2]) * 2u;
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.sv[2]) * 2u;
  const uint32_t o_row = static_cast<uint32_t>(p.so[2]);
  const uint32_t o_dim = static_cast<uint32_t>(p.so[3]);
  const bool out_vec = p.so[3] == 1 && p.so[2] % 4 == 0 && p.so[1] % 4 == 0 && p.so[0] % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0;
  // XCD-local item order (see the header comment); a bijection of [0, items).
  const int32_t grid = static_cast<int32_t>(gridDim.x);
  const bool xcd_order = grid % 8 == 0 && items % 8 == 0;
  const int32_t per_xcd = items / 8;
  auto item_of = [&](int32_t slot) { return xcd_order ? (slot & 7) * per_xcd + (slot >> 3) : slot; };

  struct Coords {
    int32_t b, h, qb;
  };
  auto coords = [&](int32_t item) {
    Coords c;
    const int32_t bh = static_cast<int32_t>(fast_div(static_cast<uint32_t>(item), p.nq_mul, p.nq_shift));
    c.qb = item - bh * q_blocks;
    c.b = static_cast<int32_t>(fast_div(static_cast<uint32_t>(bh), p.h_mul, p.h_shift));
    c.h = bh - c.b * static_cast<int32_t>(p.H);
    return c;
  };

  // Byte offsets of a thread's first K and V chunk within a tile; slot s
  // adds s * kThreads / kChunks rows.
  static_assert(G::kFull && kThreads % kChunks == 0, "whole rows per slot");
  const uint32_t k_lane = static_cast<uint32_t>(tid / kChunks) * k_row_bytes + static_cast<uint32_t>(tid % kChunks) * 16u;
  const uint32_t v_lane = static_cast<uint32_t>(tid / kChunks) * v_row_bytes + static_cast<uint32_t>(tid % kChunks) * 16u;

  // Issues the loads of tile `tile` of the plane of `c` into `st`: buffer
  // loads over the plane's rows, so rows past Nk read zeros (or, where rows
  // overlap, bytes of the plane's own rows; no offset wraps, which the
  // launch checks) and are masked when published.
  auto issue = [&](Stage& st, const Coords& c, int32_t tile) {
    const char* kp = static_cast<const char*>(p.k) + (c.b * p.sk[0] + c.h * p.sk[1]) * 2;
    const char* vp = static_cast<const char*>(p.v) + (c.b * p.sv[0] + c.h * p.sv[1]) * 2;
    const auto k_rsrc = plane_rsrc(kp, static_cast<uint32_t>(n_k - 1) * k_row_bytes + kD * 2);
    const auto v_rsrc = plane_rsrc(vp, static_cast<uint32_t>(n_k - 1) * v_row_bytes + kD * 2);
    const int32_t j0 = tile * kKeys;
#pragma unroll
    for (int s = 0; s < G::kSlots; ++s) {
      const uint32_t row0 = static_cast<uint32_t>(j0 + s * (kThreads / kChunks));
      st.k[s] = load16_buf(k_rsrc, k_lane + row0 * k_row_bytes);
      st.v[s] = load16_buf(v_rsrc, v_lane + row0 * v_row_bytes);
    }
    if (has_bias) {
      const char* bp = static_cast<const char*>(p.bias) + (c.b * p.sbb + c.h * p.sbh) * bias_esize;
      st.bias_misalign = base_misalign(bp);
#pragma unroll
      for (int s = 0; s < G::kSlots; ++s) {
        const int slot = tid + s * kThreads;
        const uint32_t key = static_cast<uint32_t>(min(j0 + slot / kChunks, n_k - 1));
        st.bias[s] = load_raw_scalar32(bp, st.bias_misalign, key * static_cast<uint32_t>(p.sbn), p.bias_dtype).word;
      }
    }
  };

  // Writes a staged tile into LDS buffer `buf`: K and V rows, and per key
  // c_j = log2(e) bias_j - coef |k_j|^2 / 2 (-inf past Nk).  A fast pass
  // stores bf16 values as fp16 (to nearest).
  auto publish = [&](const Stage& st, int32_t tile, int buf, float coef, auto kind_c) {
    constexpr bool kFast = decltype(kind_c)::value == kPassFast;
    constexpr bool kToF16 = kFast && kBf16;
    const int32_t j0 = tile * kKeys;
    T* kl = reinterpret_cast<T*>(lds + buf * G::kBufBytes);
    T* vl = reinterpret_cast<T*>(lds + buf * G::kBufBytes + G::kKBytes);
    float* cl = reinterpret_cast<float*>(lds + buf * G::kBufBytes + G::kKBytes + G::kVBytes);
#pragma unroll
    for (int s = 0; s < G::kSlots; ++s) {
      const int slot = tid + s * kThreads;
      if (G::kFull || slot < kKeys * kChunks) {
        const int key = slot / kChunks;
        const int d0 = (slot % kChunks) * 8;
        *reinterpret_cast<uint4*>(kl + key * G::kKStride + d0) = st.k[s];
        // Rows past Nk are zeroed in V: their weight is 0, and 0 times a
        // non-finite copy would not be.
        uint4 vw = st.v[s];
        if constexpr (kToF16) {
          typedef _Float16 h2 __attribute__((ext_vector_type(2)));
          uint32_t* w = reinterpret_cast<uint32_t*>(&vw);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float f0 = __uint_as_float(w[e] << 16), f1 = __uint_as_float(w[e] & 0xffff0000u);
            // IEEE maximum (v_maximum3_f32): no quieting copies of the inputs.
            vmax = __builtin_elementwise_maximum(
                vmax, __builtin_elementwise_maximum(__builtin_fabsf(f0), __builtin_fabsf(f1)));
            w[e] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{f0, f1}, h2));
          }
        } else if constexpr (kFast) {
          // fp16 values: |v| by clearing the sign bits, a packed maximum.
          const uint32_t* w = reinterpret_cast<const uint32_t*>(&vw);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            vmax16 = __builtin_elementwise_maximum(vmax16, __builtin_bit_cast(h2v, w[e] & 0x7fff7fffu));
        }
        if (j0 + kKeys > n_k && j0 + key >= n_k) vw = make_uint4(0, 0, 0, 0);  // the last tile only
        *reinterpret_cast<uint4*>(vl + key * G::kVStride + d0) = vw;
        // |k|^2 over the chunks of the row (kChunks adjacent lanes).
        const float sq = reduce_low<kChunks>(dot_chunk<T>(st.k[s], st.k[s], 0.f), OpSum());
        if (slot % kChunks == 0) {
          float bias = 0.f;
          if (has_bias) {
            const uint32_t j = static_cast<uint32_t>(min(j0 + key, n_k - 1));
            const uint32_t bytes = j * static_cast<uint32_t>(p.sbn) * bias_esize + st.bias_misalign;
            bias = decode_raw_scalar(RawScalar{st.bias[s], (bytes & 2u) * 8u}, p.bias_dtype) * kLog2e;
          }
          cl[key] = j0 + key < n_k ? fmaf(-0.5f * coef, sq, bias) : -INFINITY;
        }
      }
    }
  };

  const uint32_t one = Ops::kOnePair;
  const Qk ones8 = __builtin_bit_cast(Qk, make_uint4(one, one, one, one));

  // Per-wave query state of the current item: the B operands of the two
  // 16-column blocks, -|q|^2 / 2, and the accumulators.
  uint4 qf[kCB][kKSteps];
  f32x4 q_half[kCB];  // -|q|^2 / 2 in every row: the first product's accumulator
  float row_max[kCB];
  f32x4 acc[kCB][kDTiles];
  f32x4 total[kCB];
  // Fast pass statistic: each query block's fp16 weights times themselves;
  // the diagonal holds every query's sum of squared weights.
  f32x4 wsq[kCB];

  // Reduces tile `buf` for the wave's 16 * kCB queries.
  auto compute = [&](int buf, float coef, auto kind_c) {
    constexpr int kind = decltype(kind_c)::value;
    const T* kl = reinterpret_cast<const T*>(lds + buf * G::kBufBytes);
    const T* vl = reinterpret_cast<const T*>(lds + buf * G::kBufBytes + G::kKBytes);
    const float* cl = reinterpret_cast<const float*>(lds + buf * G::kBufBytes + G::kKBytes + G::kVBytes);
#pragma unroll
    for (int kp = 0; kp < G::kPairs; ++kp) {
      // S^T for key blocks 2kp, 2kp + 1 and both query blocks.
      f32x4 s[kCB][2];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
          const Qk a = *reinterpret_cast<const Qk*>(kl + (32 * kp + 16 * hb + col) * G::kKStride + 32 * ks + 8 * grp);
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb)
            s[cb][hb] = Ops::qk(a, __builtin_bit_cast(Qk, qf[cb][ks]), ks == 0 ? q_half[cb] : s[cb][hb]);
        }
      }
      float x[kCB][2][4];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        const float4 c = *reinterpret_cast<const float4*>(cl + 32 * kp + 16 * hb + 4 * grp);
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
          x[cb][hb][0] = fmaf(coef, s[cb][hb][0], c.x);
          x[cb][hb][1] = fmaf(coef, s[cb][hb][1], c.y);
          x[cb][hb][2] = fmaf(coef, s[cb][hb][2], c.z);
          x[cb][hb][3] = fmaf(coef, s[cb][hb][3], c.w);
        }
      }
      if constexpr (kind == kPassMax) {
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb)
#pragma unroll
          for (int hb = 0; hb < 2; ++hb)
            row_max[cb] = fmaxf(row_max[cb], fmaxf(fmaxf(x[cb][hb][0], x[cb][hb][1]), fmaxf(x[cb][hb][2], x[cb][hb][3])));
        continue;
      }
      if constexpr (kind == kPassFast) {
        // One fp16 weight per score (round to nearest) against fp16 values.
        using H = MfmaOps<_Float16>;
        typedef _Float16 h2 __attribute__((ext_vector_type(2)));
        typename H::Qk pw[kCB];
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
          uint32_t wp[4];
#pragma unroll
          for (int hb = 0; hb < 2; ++hb) {
            float w[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) w[r] = __builtin_amdgcn_exp2f(x[cb][hb][r]);
            wp[2 * hb] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{w[0], w[1]}, h2));
            wp[2 * hb + 1] = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{w[2], w[3]}, h2));
          }

          pw[cb] = __builtin_bit_cast(typename H::Qk, make_uint4(wp[0], wp[1], wp[2], wp[3]));
        }
#pragma unroll
        for (int u = 0; u < kDTiles; ++u) {
          // The A operand as in the split pass below.
          const T* va = vl + (32 * kp + 4 * grp + col / 4) * G::kVStride + 16 * u + 4 * (col % 4);
          const uint2 a0 = lds_read_tr16(va);
          const uint2 a1 = lds_read_tr16(va + 16 * G::kVStride);
          const auto a = __builtin_bit_cast(typename H::Qk, make_uint4(a0.x, a0.y, a1.x, a1.y));
#pragma unroll
          for (int cb = 0; cb < kCB; ++cb) acc[cb][u] = H::qk(a, pw[cb], acc[cb][u]);
        }
        const uint32_t one_h = MfmaOps<_Float16>::kOnePair;
        const auto ones_h = __builtin_bit_cast(typename H::Qk, make_uint4(one_h, one_h, one_h, one_h));
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
          total[cb] = H::qk(ones_h, pw[cb], total[cb]);
          wsq[cb] = H::qk(pw[cb], pw[cb], wsq[cb]);  // A = B^T (the same lane layout)
        }
        __builtin_amdgcn_sched_barrier(0);
        continue;
      }
      Qk p_hi[kCB], p_lo[kCB];
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const float shift = kind == kPassShifted ? row_max[cb] : 0.f;
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          float w[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) w[r] = __builtin_amdgcn_exp2f(x[cb][hb][r] - shift);
          Ops::split2_sub(w[0], w[1], hi[2 * hb], lo[2 * hb]);
          Ops::split2_sub(w[2], w[3], hi[2 * hb + 1], lo[2 * hb + 1]);
        }
        p_hi[cb] = __builtin_bit_cast(Qk, make_uint4(hi[0], hi[1], hi[2], hi[3]));
        p_lo[cb] = __builtin_bit_cast(Qk, make_uint4(lo[0], lo[1], lo[2], lo[3]));
      }
#pragma unroll
      for (int u = 0; u < kDTiles; ++u) {
        // A operand of O^T: lane (dim 16u + col, group g) gets keys
        // 32kp + 4g + 0..3 and 32kp + 16 + 4g + 0..3 of that dim.  Within a
        // group of 16 lanes, ds_read_b64_tr_b16 gives lane i element i % 4
        // of the 4-element pieces addressed by lanes i / 4, 4 + i / 4,
        // 8 + i / 4 and 12 + i / 4, so lane i addresses key row
        // 32kp + 4g + i / 4 (+16), dims 16u + 4 (i % 4) .. +3.
        const T* va = vl + (32 * kp + 4 * grp + col / 4) * G::kVStride + 16 * u + 4 * (col % 4);
        const uint2 a0 = lds_read_tr16(va);
        const uint2 a1 = lds_read_tr16(va + 16 * G::kVStride);
        const Qk a = __builtin_bit_cast(Qk, make_uint4(a0.x, a0.y, a1.x, a1.y));
#pragma unroll
        for (int cb = 0; cb < kCB; ++cb) {
          acc[cb][u] = Ops::qk(a, p_hi[cb], acc[cb][u]);
          acc[cb][u] = Ops::qk(a, p_lo[cb], acc[cb][u]);
        }
      }
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        total[cb] = Ops::qk(ones8, p_hi[cb], total[cb]);
        total[cb] = Ops::qk(ones8, p_lo[cb], total[cb]);
      }
      // One key pair at a time: keeps the next pair's operands from being
      // hoisted over this pair's products (register pressure).
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Whether, with the fast pass's sums so far over `seen` keys, the bound on
  // its error misses the accuracy contract at one of this lane's outputs:
  // kFastSigmas deviations of the walk (its bound per unit of spread scaled
  // from `seen` keys to all n_k, as sqrt(sum w^2) / T falls like one over
  // the root of the key count), 2^-25 per key and for the values, against
  // `slack` times the allowance; also a weight sum (scaled to n_k keys) below
  // kFastSum / slack, or a non-finite output.
  auto fast_misses = [&](float v_max, float seen, float slack) {
    const float grow = static_cast<float>(n_k) / seen;
    bool miss = false;
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      const float t = total[cb][0];
      miss = miss || !(t * grow * slack >= kFastSum);
      // Sum of squared weights of this lane's query: row `col` of the
      // product, held by lane col + 16 (col / 4) in register col % 4.
      const float diag = wsq[cb][col & 3];
      const float sq_w = __shfl(diag, col + 16 * (col >> 2), kWave);
      const float inv_t = 1.f / t;
      const float per_spread = (kFastWalk * __builtin_sqrtf(sq_w / grow) + 0x1p-25f * seen) * inv_t;
#pragma unroll
      for (int u = 0; u < kDTiles; ++u) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float o = __builtin_fabsf(acc[cb][u][r] * inv_t);
          miss = miss || !__builtin_isfinite(o) ||
                 !(fmaf(per_spread, v_max + o, 0x1p-25f) <= slack * fmaf(kGateRtol, o, kGateAtol));
        }
      }
    }
    return miss;
  };

  // One pass of an item over every key tile (double-buffered, one barrier
  // per tile).  Every wave of the workgroup runs it.  The fast pass checks
  // its course after the first eighth of the tiles and is abandoned (returns
  // false, nothing left in flight) where its bound, so far, misses the
  // contract by more than twice: the split pass then runs instead.  That is
  // a prediction, not the test: a fast pass that runs to the end is kept
  // only if its final sums pass it.
  Stage st;
  int32_t parity = 0;
  auto run_pass = [&](const Coords& c, float coef, auto kind_c) {
    constexpr bool kFast = decltype(kind_c)::value == kPassFast;
    if constexpr (decltype(kind_c)::value != kPassMax) {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
#pragma unroll
        for (int u = 0; u < kDTiles; ++u) acc[cb][u] = f32x4{0.f, 0.f, 0.f, 0.f};
        total[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
    }
    if constexpr (decltype(kind_c)::value == kPassFast) {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) wsq[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
      vmax = 0.f;
      vmax16 = h2v{0, 0};
    }
    issue(st, c, 0);
    publish(st, 0, 0, coef, kind_c);
    __syncthreads();
    if (tiles > 1) issue(st, c, 1);
    const int32_t probe = tiles / 8;  // tiles reduced when the fast pass checks its course
    for (int32_t t = 0; t < tiles; ++t) {
      compute(t & 1, coef, kind_c);
      if (t + 1 < tiles) publish(st, t + 1, (t + 1) & 1, coef, kind_c);
      if constexpr (kFast) {
        // After the staging registers are written out: no loads in flight.
        if (t + 1 == probe) {
          const float m = kBf16 ? vmax : fmaxf(static_cast<float>(vmax16.x), static_cast<float>(vmax16.y));
          const float seen = static_cast<float>(min(probe * kKeys, n_k));
          if (__builtin_amdgcn_ballot_w64(fast_misses(reduce_wave(m, OpMax()), seen, 2.f)) && lane == 0)
            abort_flag[parity] = 1;
        }
      }
      __syncthreads();
      if constexpr (kFast) {
        // Every wave reads the flag after the barrier: a uniform exit, with
        // tile t + 1 already staged and nothing issued past it.
        if (t + 1 == probe && abort_flag[parity] != 0) return false;
      }
      if (t + 2 < tiles) issue(st, c, t + 2);
    }
    return true;
  };

  for (int32_t slot = static_cast<int32_t>(blockIdx.x); slot < items; slot += grid, parity ^= 1) {
    const Coords c = coords(item_of(slot));
    if (tid == 0) {  // read after the first barrier of this item
      exact_flag[parity] = 0;
      split_flag[parity] = 0;
      abort_flag[parity] = 0;
    }
    const float coef = 2.f * kLog2e * load_any(p.scale, c.b * p.ssb + c.h * p.ssh, p.scale_dtype);
    // Query rows of this wave: item rows (wave * kCB + cb) * 16 + col (rows
    // past Nq read row Nq - 1 and are not stored).
    {
      const char* qp = static_cast<const char*>(p.q) + (c.b * p.sq[0] + c.h * p.sq[1]) * 2;
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const uint32_t row = static_cast<uint32_t>(min(c.qb * G::kQRows + (wave * kCB + cb) * 16 + col, n_q - 1));
        float sq = 0.f;
#pragma unroll
        for (int ks = 0; ks < kKSteps; ++ks) {
          qf[cb][ks] = load16(qp + row * q_row_bytes + static_cast<uint32_t>(64 * ks + 16 * grp));
          sq = dot_chunk<T>(qf[cb][ks], qf[cb][ks], sq);
        }
        const float h = -0.5f * allreduce_bit32(allreduce_bit16(sq, OpSum()), OpSum());
        q_half[cb] = f32x4{h, h, h, h};
      }
    }
    // The single pass needs x <= 0: no bias and gamma >= 0.
    bool exact = has_bias || !(coef >= 0.f);
    bool split = true;
    if (!exact && n_k >= kFastKeys && !(p.flags & VECTRA_FLAG_SPLIT_WEIGHTS)) {
      // The fast result stands if the whole pass ran and its final sums pass
      // the check anywhere in the workgroup: every weight sum at least
      // kFastSum, every output finite and within the contract by its bound.
      if (run_pass(c, coef, PassKind<kPassFast>{})) {
        // The workgroup's max |v| (every wave staged a share of every tile).
        const float m = kBf16 ? vmax : fmaxf(static_cast<float>(vmax16.x), static_cast<float>(vmax16.y));
        const float mw = reduce_wave(m, OpMax());
        if (lane == 0) vmax_wave[parity][wave] = mw;
        __syncthreads();
        float v_max = vmax_wave[parity][0];
#pragma unroll
        for (int w = 1; w < kWaves; ++w) v_max = fmaxf(v_max, vmax_wave[parity][w]);
        const bool redo = fast_misses(v_max, static_cast<float>(n_k), 1.f);
        if (__builtin_amdgcn_ballot_w64(redo) && lane == 0) split_flag[parity] = 1;
        __syncthreads();
        split = split_flag[parity] != 0;
      }
    }
    if (!exact && split) {
      run_pass(c, coef, PassKind<kPassSum>{});
      // A weight sum below the accurate range (or NaN) anywhere in the
      // workgroup sends the item to the exact passes.
      bool low = false;
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) low = low || !(total[cb][0] >= kSumLo);
      if (__builtin_amdgcn_ballot_w64(low) && lane == 0) exact_flag[parity] = 1;
      __syncthreads();
      exact = exact_flag[parity] != 0;
    }
    if (exact) {
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) row_max[cb] = -INFINITY;
      run_pass(c, coef, PassKind<kPassMax>{});
#pragma unroll
      for (int cb = 0; cb < kCB; ++cb) {
        const float m = allreduce_bit32(allreduce_bit16(row_max[cb], OpMax()), OpMax());
        row_max[cb] = m == -INFINITY ? 0.f : m;  // every key masked: the row ends as NaN
      }
      run_pass(c, coef, PassKind<kPassShifted>{});
    }

    // Store: every row of the ones product holds the query's weight sum; a
    // fully masked row has sum 0 and ends as 0 * inf = NaN.
    char* out_plane = static_cast<char*>(p.out) + (c.b * p.so[0] + c.h * p.so[1]) * static_cast<int64_t>(kOutSize);
#pragma unroll
    for (int cb = 0; cb < kCB; ++cb) {
      const int32_t q_row = c.qb * G::kQRows + (wave * kCB + cb) * 16 + col;
      if (q_row < n_q) {
        const float inv = __builtin_amdgcn_rcpf(total[cb][0]);
        const uint32_t row_off = static_cast<uint32_t>(q_row) * o_row;
#pragma unroll
        for (int u = 0; u < kDTiles; ++u) {
          const uint32_t off = (row_off + static_cast<uint32_t>(16 * u + 4 * grp) * o_dim) * kOutSize;
          const float y0 = acc[cb][u][0] * inv, y1 = acc[cb][u][1] * inv;
          const float y2 = acc[cb][u][2] * inv, y3 = acc[cb][u][3] * inv;
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
}

// ------------------------------------------------------------------- host

template <typename T, typename OutT, int kD, int kKeys, int kWaves, int kCB>
int tile_resident_blocks() {
  static std::atomic<int> cached{0};
  int n = cached.load(std::memory_order_relaxed);
  if (n == 0) {
    using G = TileGeo<T, kD, kKeys, kWaves, kCB>;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&rbf_tile_kernel<T, OutT, kD, kKeys, kWaves, kCB>), 64 * kWaves,
            2 * G::kBufBytes) != hipSuccess ||
        n < 1)
      n = 1;
    cached.store(n, std::memory_order_relaxed);
  }
  return n;
}

template <typename T, typename OutT, int kD, int kKeys, int kWaves, int kCB>
hipError_t launch_tile_k(Problem& p, hipStream_t s) {
  using G = TileGeo<T, kD, kKeys, kWaves, kCB>;
  const int32_t q_blocks = static_cast<int32_t>((p.Nq + G::kQRows - 1) / G::kQRows);
  const int64_t items = p.B * p.H * q_blocks;
  int64_t blocks = static_cast<int64_t>(tile_resident_blocks<T, OutT, kD, kKeys, kWaves, kCB>()) *
                   (p.compute_units > 0 ? p.compute_units : 1);
  if (blocks > items) blocks = items;
  if (blocks >= 8) blocks -= blocks % 8;  // whole XCD rounds (see the kernel)
  if (items + blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  Problem k = p;  // the kernel divides work items by q_blocks with the Nq slots
  make_fast_div(q_blocks, &k.nq_mul, &k.nq_shift);
  int32_t qb = q_blocks;
  void* args[] = {&k, &qb};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_tile_kernel<T, OutT, kD, kKeys, kWaves, kCB>),
                         dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves), args, 2 * G::kBufBytes, s);
}

template <typename T, typename OutT>
hipError_t launch_tile_t(Problem& p, hipStream_t s) {
  switch (p.D) {
    case 32: return launch_tile_k<T, OutT, 32, 64, 4, 2>(p, s);
    case 64: return launch_tile_k<T, OutT, 64, 64, 4, 4>(p, s);
    case 128: return launch_tile_k<T, OutT, 128, 32, 4, 2>(p, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_tile_bf16_bf16(Problem& p, hipStream_t s);
hipError_t launch_tile_bf16_f32(Problem& p, hipStream_t s);
hipError_t launch_tile_f16_f16(Problem& p, hipStream_t s);
hipError_t launch_tile_f16_f32(Problem& p, hipStream_t s);

}  // namespace vectra
