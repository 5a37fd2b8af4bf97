// Query-tile RBF attention on gfx950 matrix cores: the kernel template.
// Instantiated per dtype pair in rbf_mfma_<in>_<out>.hip.
//
// For query tiles (Nq >= 16: self-attention over a comparable set, long key
// axes) both products run on MFMA, transposed so that no operand has to move
// between lanes:
//
//   S^T = K . Q^T     (16 keys x 16 queries per instruction)
//   O^T = V^T . P^T   (16 value dims x 16 queries)
//
// Lane layouts of the instructions used are listed in rbf_mfma_ops.h
// (wave64, l = lane, g = l / 16).
//
// S^T puts in each lane the scores of ONE query (column l % 16) against keys
// 16t + 4g + r (r = 0..3) of every 16-key block t.  Those of blocks 2p and
// 2p + 1 together are exactly the B operand of a 16x16x32 step over keys
// 32p .. 32p + 31 read in the order {4g .. 4g+3, 16+4g .. 16+4g+3} (V^T is
// read in the same order); an odd last block takes a 16x16x16 step (deep
// index 4g + r), and fp32 takes 16x16x4 steps, one r at a time (deep index
// g).  So P stays in the registers it was computed in, and the softmax state
// of a query lives in its four lanes l, l+16, l+32, l+48, reduced with gfx950
// permlane swaps.
//
// The distance is folded into the first product: its accumulator starts at
// -(|q|^2 + |k|^2) / 2, so the result is S' = q.k - (|q|^2 + |k|^2) / 2 =
// -d / 2, and the logit (in log2 units) is
//   2 gamma log2(e) min(S', 0) + bias log2(e)  =  log2(e) (-gamma max(d, 0) + bias).
//
// 16-bit inputs: P is fed to the second product as a hi + lo pair of 16-bit
// values (two MFMAs), so the weights keep ~16 more bits than one rounding
// would; rounding P once (as the reference's Triton kernel does) misses the
// rtol 1e-3 gate at a few tens of keys.  fp32 inputs: both products run on
// the fp32 MFMA, exact products with fp32 accumulation.
//
// Semantics are those of rbf_stream_kernel: clamp of the distance at 0,
// -scale * d + bias, keys >= Nk masked, a running max replaced by 0 while it
// is -inf (fully masked rows end as 0/0 = NaN), fp32 accumulation.

#pragma once

#include <atomic>

#include "rbf_common.h"
#include "rbf_kernels.h"
#include "rbf_mfma_ops.h"

namespace vectra {

// LDS tile geometry.
//   K: row-major [key][head dim], 16-bit rows padded to whole 32-deep steps
//      (zeros) plus 8, fp32 rows plus 4: the 16 rows one operand read touches
//      start in distinct banks.
//   V: 16-bit transposed [value dim][key] (row stride kKeys + 4), read as
//      4 consecutive keys; fp32 as [key / 4][value dim][key % 4], read as the
//      4 keys 16t + 4g + 0..3 of one value dim.
//   Then -|k|^2 / 2 and the bias (log2 units, -inf past Nk) per key.
template <typename T, int kD, int kKeys>
struct MfmaTile {
  static constexpr bool kHalf = sizeof(T) == 2;
  static constexpr int kKSteps = kHalf ? (kD + 31) / 32 : kD / 4;  // deep steps of S^T
  static constexpr int kDpad = kHalf ? (kD + 31) / 32 * 32 : kD;
  static constexpr int kKStride = kDpad + (kHalf ? 8 : 4);
  static constexpr int kVStride = kKeys + 4;  // 16-bit V^T rows
  static constexpr int kKBytes = kKeys * kKStride * static_cast<int>(sizeof(T));
  static constexpr int kVBytes = kHalf ? kD * kVStride * 2 : kKeys * kD * 4;
  static constexpr int kBytes = kKBytes + kVBytes + 2 * kKeys * static_cast<int>(sizeof(float));
};

// Work item: one (b, h) plane and one block of kWaves * 16 query rows; the
// plane's keys are streamed in tiles of kKeys.  The grid is persistent: a
// workgroup takes items blockIdx.x, blockIdx.x + gridDim.x, ...  Every
// thread owns fixed load slots of a tile (16-byte chunks of K rows, of V rows
// -- pairs of rows for 16-bit inputs, which are transposed two keys per
// 32-bit LDS write -- and biases, plus at an item's first tile its q
// fragment).  All of them are issued together into registers as soon as the
// previous tile is in LDS, so the next tile's HBM latency overlaps this
// tile's products and softmax.
template <typename T, int kD, int kKeys, int kWaves>
struct MfmaStage {
  static constexpr bool kHalf = sizeof(T) == 2;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kVec = 16 / static_cast<int>(sizeof(T));
  static constexpr int kDChunks = kD / kVec;  // 16-byte chunks per row
  static constexpr int kVRows = kHalf ? 2 : 1;
  static constexpr int kKSlots = (kKeys * kDChunks + kThreads - 1) / kThreads;
  static constexpr int kVSlots = ((kKeys / kVRows) * kDChunks + kThreads - 1) / kThreads;
  static constexpr int kBSlots = (kKeys + kThreads - 1) / kThreads;
  // q chunks per lane: 16-bit, one per 32-deep step; fp32, the D / 4
  // consecutive dims of lane group g.
  static constexpr int kQChunks = kHalf ? (kD + 31) / 32 : kD / 16;
  uint4 k[kKSlots];
  uint4 v[kVSlots][kVRows];
  uint32_t bias[kBSlots];
  uint32_t bias_misalign;  // address & 3 of the item's bias plane
  uint4 q[kQChunks];
  RawScalar scale;
};

// Byte offsets, inside a (b, h) plane, of a thread's load slots for one tile.
template <typename T, int kD, int kKeys, int kWaves>
struct MfmaOffsets {
  using Stage = MfmaStage<T, kD, kKeys, kWaves>;
  uint32_t k[Stage::kKSlots];
  uint32_t v[Stage::kVSlots][Stage::kVRows];
  uint32_t bias[Stage::kBSlots];  // elements
};

template <typename T, typename OutT, int kD, int kKeys, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void rbf_mfma_kernel(Problem p, int32_t q_blocks) {
  using Geo = MfmaTile<T, kD, kKeys>;
  using Stage = MfmaStage<T, kD, kKeys, kWaves>;
  using Offsets = MfmaOffsets<T, kD, kKeys, kWaves>;
  constexpr bool kHalf = Geo::kHalf;
  constexpr int kThreads = Stage::kThreads;
  constexpr int kVec = Stage::kVec;
  constexpr int kDChunks = Stage::kDChunks;
  constexpr int kVRows = Stage::kVRows;
  constexpr int kNTiles = kKeys / 16;  // 16-key blocks per tile
  constexpr int kDvTiles = kD / 16;
  constexpr int kESize = static_cast<int>(sizeof(T));
  static_assert(kD % 16 == 0 && kKeys % 16 == 0 && kKeys <= 128, "tile shape");
  static_assert(64 % kDChunks == 0, "a K row's chunks stay inside one wave");

  extern __shared__ __align__(16) unsigned char lds[];
  T* k_lds = reinterpret_cast<T*>(lds);
  T* v_lds = reinterpret_cast<T*>(lds + Geo::kKBytes);
  float* kn_lds = reinterpret_cast<float*>(lds + Geo::kKBytes + Geo::kVBytes);
  float* bias_lds = kn_lds + kKeys;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 15;  // query within the wave's 16
  const int grp = lane >> 4;  // lane group g

  const int32_t n_q = static_cast<int32_t>(p.Nq);
  const int32_t n_k = static_cast<int32_t>(p.Nk);
  const int32_t items = static_cast<int32_t>(p.B * p.H) * q_blocks;
  const int32_t tiles = (n_k + kKeys - 1) / kKeys;
  const bool has_bias = p.bias != nullptr;
  const int32_t bias_esize = p.bias_dtype == VECTRA_F32 ? 4 : 2;
  const uint32_t k_row_bytes = static_cast<uint32_t>(p.sk[2]) * kESize;
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.sv[2]) * kESize;
  const uint32_t q_row_bytes = static_cast<uint32_t>(p.sq[2]) * kESize;
  // Contiguous output rows take one vector store per 4 values.
  const bool out_vec = p.so[3] == 1 && p.so[2] % 4 == 0 && p.so[1] % 4 == 0 && p.so[0] % 4 == 0 &&
                       (reinterpret_cast<uintptr_t>(p.out) & 15u) == 0;

  struct Coords {
    int32_t b, h, qb;
  };
  auto coords = [&](int32_t item) {
    Coords c;
    const int32_t bh = static_cast<int32_t>(fast_div(item, p.nq_mul, p.nq_shift));  // / q_blocks
    c.qb = item - bh * q_blocks;
    c.b = static_cast<int32_t>(fast_div(bh, p.h_mul, p.h_shift));
    c.h = bh - c.b * static_cast<int32_t>(p.H);
    return c;
  };

  // Rows past Nk read row Nk - 1 (in bounds) and are masked in LDS.
  auto tile_offsets = [&](int32_t tile) {
    Offsets o;
    const int32_t j0 = tile * kKeys;
#pragma unroll
    for (int s = 0; s < Stage::kKSlots; ++s) {
      const int slot = tid + s * kThreads;
      const uint32_t j = static_cast<uint32_t>(min(j0 + slot / kDChunks, n_k - 1));
      o.k[s] = j * k_row_bytes + (slot % kDChunks) * 16u;
    }
#pragma unroll
    for (int s = 0; s < Stage::kVSlots; ++s) {
      const int slot = tid + s * kThreads;
#pragma unroll
      for (int e = 0; e < kVRows; ++e) {
        const uint32_t j = static_cast<uint32_t>(min(j0 + kVRows * (slot / kDChunks) + e, n_k - 1));
        o.v[s][e] = j * v_row_bytes + (slot % kDChunks) * 16u;
      }
    }
#pragma unroll
    for (int s = 0; s < Stage::kBSlots; ++s) {
      const uint32_t j = static_cast<uint32_t>(min(j0 + tid + s * kThreads, n_k - 1));
      o.bias[s] = j * static_cast<uint32_t>(p.sbn);
    }
    return o;
  };
  const Offsets first = tile_offsets(0);

  // Padding columns of 16-bit K rows (head dims kD .. kDpad) stay zero.
  if constexpr (Geo::kDpad > kD) {
    for (int i = tid; i < kKeys * (Geo::kDpad - kD); i += kThreads) {
      const int key = i / (Geo::kDpad - kD);
      k_lds[key * Geo::kKStride + kD + i % (Geo::kDpad - kD)] = static_cast<T>(0.f);
    }
  }

  // Issues every load of (item, tile) into `st`.
  auto issue = [&](Stage& st, int32_t item, int32_t tile) {
    const Coords c = coords(item);
    const char* kp = static_cast<const char*>(p.k) + (c.b * p.sk[0] + c.h * p.sk[1]) * kESize;
    const char* vp = static_cast<const char*>(p.v) + (c.b * p.sv[0] + c.h * p.sv[1]) * kESize;
    const Offsets o = tile == 0 ? first : tile_offsets(tile);
#pragma unroll
    for (int s = 0; s < Stage::kKSlots; ++s)
      if (tid + s * kThreads < kKeys * kDChunks) st.k[s] = load16_stream(kp + o.k[s]);
#pragma unroll
    for (int s = 0; s < Stage::kVSlots; ++s) {
      if (tid + s * kThreads < (kKeys / kVRows) * kDChunks) {
#pragma unroll
        for (int e = 0; e < kVRows; ++e) st.v[s][e] = load16_stream(vp + o.v[s][e]);
      }
    }
    if (has_bias) {
      const char* bp = static_cast<const char*>(p.bias) + (c.b * p.sbb + c.h * p.sbh) * bias_esize;
      st.bias_misalign = base_misalign(bp);
#pragma unroll
      for (int s = 0; s < Stage::kBSlots; ++s)
        if (tid + s * kThreads < kKeys)
          st.bias[s] = load_raw_scalar32(bp, st.bias_misalign, o.bias[s], p.bias_dtype).word;
    }
    if (tile == 0) {
      const int32_t q_row = min((c.qb * kWaves + wave) * 16 + col, n_q - 1);
      const char* qp = static_cast<const char*>(p.q) + (c.b * p.sq[0] + c.h * p.sq[1]) * kESize;
      const uint32_t q_off = static_cast<uint32_t>(q_row) * q_row_bytes;
#pragma unroll
      for (int i = 0; i < Stage::kQChunks; ++i) {
        const int d0 = kHalf ? 32 * i + 8 * grp : grp * (kD / 4) + 4 * i;
        if (d0 < kD) st.q[i] = load16(qp + q_off + d0 * kESize);
      }
      st.scale = load_raw_scalar(p.scale, c.b * p.ssb + c.h * p.ssh, p.scale_dtype);
    }
  };

  // Copies a staged tile into LDS: K rows and -|k|^2 / 2, V, and biases.
  auto publish = [&](const Stage& st, int32_t tile) {
    const int32_t j0 = tile * kKeys;
#pragma unroll
    for (int s = 0; s < Stage::kKSlots; ++s) {
      const int slot = tid + s * kThreads;
      // The cross-lane reduction runs on every lane, outside any branch, and
      // only the stores are guarded: under a branch that some waves skip (a
      // slot only partly filled, as with eight waves and 80-key tiles of
      // 64-dim rows) its DPP reads gave wrong values on the device.
      const bool live = Stage::kKSlots * kThreads == kKeys * kDChunks || slot < kKeys * kDChunks;
      const int key = slot / kDChunks;
      const uint4 raw = live && j0 + key < n_k ? st.k[s] : make_uint4(0, 0, 0, 0);
      if (live) *reinterpret_cast<uint4*>(k_lds + key * Geo::kKStride + (slot % kDChunks) * kVec) = raw;
      const float sq = reduce_low<kDChunks>(dot_chunk<T>(raw, raw, 0.f), OpSum());
      if (live && slot % kDChunks == 0) kn_lds[key] = -0.5f * sq;
    }
#pragma unroll
    for (int s = 0; s < Stage::kVSlots; ++s) {
      const int slot = tid + s * kThreads;
      if (slot < (kKeys / kVRows) * kDChunks) {
        const int row = kVRows * (slot / kDChunks);  // first key of the slot
        const int d0 = (slot % kDChunks) * kVec;
        if constexpr (kHalf) {
          const uint4 r0 = j0 + row < n_k ? st.v[s][0] : make_uint4(0, 0, 0, 0);
          const uint4 r1 = j0 + row + 1 < n_k ? st.v[s][1] : make_uint4(0, 0, 0, 0);
          const uint32_t w0[4] = {r0.x, r0.y, r0.z, r0.w};
          const uint32_t w1[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            // Elements 2e and 2e+1 of the chunk for keys row (low half) and row + 1.
            const uint32_t even = (w0[e] & 0xffffu) | (w1[e] << 16);
            const uint32_t odd = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
            *reinterpret_cast<uint32_t*>(v_lds + (d0 + 2 * e) * Geo::kVStride + row) = even;
            *reinterpret_cast<uint32_t*>(v_lds + (d0 + 2 * e + 1) * Geo::kVStride + row) = odd;
          }
        } else {
          const uint4 r0 = j0 + row < n_k ? st.v[s][0] : make_uint4(0, 0, 0, 0);
          float* dst = reinterpret_cast<float*>(v_lds) + ((row >> 2) * kD + d0) * 4 + (row & 3);
          dst[0] = __uint_as_float(r0.x);
          dst[4] = __uint_as_float(r0.y);
          dst[8] = __uint_as_float(r0.z);
          dst[12] = __uint_as_float(r0.w);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < Stage::kBSlots; ++s) {
      const int key = tid + s * kThreads;
      if (key < kKeys) {
        float x = -INFINITY;
        if (j0 + key < n_k) {
          x = 0.f;
          if (has_bias) {
            const uint32_t j = static_cast<uint32_t>(j0 + key);
            const uint32_t bytes = j * static_cast<uint32_t>(p.sbn) * bias_esize + st.bias_misalign;
            x = decode_raw_scalar(RawScalar{st.bias[s], (bytes & 2u) * 8u}, p.bias_dtype) * kLog2e;
          }
        }
        bias_lds[key] = x;
      }
    }
  };

  uint4 q_frag[Stage::kQChunks];
  float q_half = 0.f, coef = 0.f, run_max = -INFINITY, run_sum = 0.f;
  f32x4 acc[kDvTiles];

  Stage st;
  int32_t item = static_cast<int32_t>(blockIdx.x), tile = 0;
  if (item >= items) return;  // before any barrier: the whole workgroup leaves
  issue(st, item, 0);
  while (true) {
    int32_t next_item = item, next_tile = tile + 1;
    if (next_tile == tiles) {
      next_tile = 0;
      next_item += static_cast<int32_t>(gridDim.x);
    }
    __syncthreads();  // the previous tile is no longer read from LDS
    publish(st, tile);
    if (tile == 0) {
      const Coords c = coords(item);
      const bool q_live = (c.qb * kWaves + wave) * 16 + col < n_q;
      float q_norm = 0.f;
#pragma unroll
      for (int i = 0; i < Stage::kQChunks; ++i) {
        const int d0 = kHalf ? 32 * i + 8 * grp : grp * (kD / 4) + 4 * i;
        q_frag[i] = (q_live && d0 < kD) ? st.q[i] : make_uint4(0, 0, 0, 0);
        q_norm = dot_chunk<T>(q_frag[i], q_frag[i], q_norm);
      }
      q_half = -0.5f * allreduce_bit32(allreduce_bit16(q_norm, OpSum()), OpSum());
      coef = 2.f * kLog2e * decode_raw_scalar(st.scale, p.scale_dtype);
      run_max = -INFINITY;
      run_sum = 0.f;
#pragma unroll
      for (int u = 0; u < kDvTiles; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    const bool more = next_item < items;
    if (more) issue(st, next_item, next_tile);  // in flight while this tile is reduced

    // Logits (log2 units) of this lane's query against keys 16t + 4g + r.
    float logit[kNTiles][4];
    float tile_max = -INFINITY;
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
      const float4 kn = *reinterpret_cast<const float4*>(kn_lds + 16 * t + 4 * grp);
      f32x4 sc = f32x4{kn.x + q_half, kn.y + q_half, kn.z + q_half, kn.w + q_half};
      if constexpr (kHalf) {
        using Qk = typename MfmaOps<T>::Qk;
#pragma unroll
        for (int ks = 0; ks < Geo::kKSteps; ++ks) {
          const Qk a = *reinterpret_cast<const Qk*>(k_lds + (16 * t + col) * Geo::kKStride + 32 * ks + 8 * grp);
          sc = MfmaOps<T>::qk(a, __builtin_bit_cast(Qk, q_frag[ks]), sc);
        }
      } else {
#pragma unroll
        for (int i = 0; i < kD / 16; ++i) {
          const float4 kf = *reinterpret_cast<const float4*>(
              reinterpret_cast<const float*>(k_lds) + (16 * t + col) * Geo::kKStride + grp * (kD / 4) + 4 * i);
          sc = MfmaOps<float>::mma(kf.x, __uint_as_float(q_frag[i].x), sc);
          sc = MfmaOps<float>::mma(kf.y, __uint_as_float(q_frag[i].y), sc);
          sc = MfmaOps<float>::mma(kf.z, __uint_as_float(q_frag[i].z), sc);
          sc = MfmaOps<float>::mma(kf.w, __uint_as_float(q_frag[i].w), sc);
        }
      }
      const float4 bias = *reinterpret_cast<const float4*>(bias_lds + 16 * t + 4 * grp);
      const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
      // min(-d/2, 0) keeping NaN (v_minimum3_f32), so a NaN in q or k makes
      // the row NaN as in the eager chain, even for a masked key.
#pragma unroll
      for (int r = 0; r < 4; ++r) logit[t][r] = fmaf(coef, __builtin_elementwise_minimum(sc[r], 0.f), bv[r]);
      tile_max = fmaxf(tile_max, fmaxf(fmaxf(logit[t][0], logit[t][1]), fmaxf(logit[t][2], logit[t][3])));
    }
    tile_max = allreduce_bit32(allreduce_bit16(tile_max, OpMax()), OpMax());
    const float new_max = fmaxf(run_max, tile_max);
    const float safe_max = new_max == -INFINITY ? 0.f : new_max;
    const float alpha = __builtin_amdgcn_exp2f(run_max - safe_max);
    run_max = new_max;
    // Rescale only when some query's maximum moved (alpha == 1 is exact).
    if (__builtin_amdgcn_ballot_w64(alpha != 1.f)) {
      run_sum *= alpha;
#pragma unroll
      for (int u = 0; u < kDvTiles; ++u) acc[u] *= alpha;
    }

    // O^T += V^T . P^T.
    if constexpr (kHalf) {
      using Qk = typename MfmaOps<T>::Qk;
      using Pv = typename MfmaOps<T>::Pv;
      // Weights of block t as packed 16-bit hi / lo pairs (keys 4g + 0,1 and 4g + 2,3).
      auto weights = [&](int t, uint32_t* hi, uint32_t* lo) {
        float w[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = __builtin_amdgcn_exp2f(logit[t][r] - safe_max);
        run_sum += (w[0] + w[1]) + (w[2] + w[3]);
        MfmaOps<T>::split2(w[0], w[1], hi[0], lo[0]);
        MfmaOps<T>::split2(w[2], w[3], hi[1], lo[1]);
      };
#pragma unroll
      for (int pp = 0; pp < kNTiles / 2; ++pp) {
        uint32_t hi[4], lo[4];
        weights(2 * pp, hi, lo);
        weights(2 * pp + 1, hi + 2, lo + 2);
        const Qk p_hi = __builtin_bit_cast(Qk, make_uint4(hi[0], hi[1], hi[2], hi[3]));
        const Qk p_lo = __builtin_bit_cast(Qk, make_uint4(lo[0], lo[1], lo[2], lo[3]));
#pragma unroll
        for (int u = 0; u < kDvTiles; ++u) {
          const T* row = v_lds + (16 * u + col) * Geo::kVStride + 32 * pp + 4 * grp;
          const uint2 a0 = *reinterpret_cast<const uint2*>(row);
          const uint2 a1 = *reinterpret_cast<const uint2*>(row + 16);
          const Qk a = __builtin_bit_cast(Qk, make_uint4(a0.x, a0.y, a1.x, a1.y));
          acc[u] = MfmaOps<T>::qk(a, p_hi, acc[u]);
          acc[u] = MfmaOps<T>::qk(a, p_lo, acc[u]);
        }
      }
      if constexpr (kNTiles % 2 == 1) {
        constexpr int t = kNTiles - 1;
        uint32_t hi[2], lo[2];
        weights(t, hi, lo);
        const Pv p_hi = __builtin_bit_cast(Pv, make_uint2(hi[0], hi[1]));
        const Pv p_lo = __builtin_bit_cast(Pv, make_uint2(lo[0], lo[1]));
#pragma unroll
        for (int u = 0; u < kDvTiles; ++u) {
          const Pv a = *reinterpret_cast<const Pv*>(v_lds + (16 * u + col) * Geo::kVStride + 16 * t + 4 * grp);
          acc[u] = MfmaOps<T>::pv(a, p_hi, acc[u]);
          acc[u] = MfmaOps<T>::pv(a, p_lo, acc[u]);
        }
      }
    } else {
#pragma unroll
      for (int t = 0; t < kNTiles; ++t) {
        float w[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) w[r] = __builtin_amdgcn_exp2f(logit[t][r] - safe_max);
        run_sum += (w[0] + w[1]) + (w[2] + w[3]);
#pragma unroll
        for (int u = 0; u < kDvTiles; ++u) {
          const float4 vv = *reinterpret_cast<const float4*>(
              reinterpret_cast<const float*>(v_lds) + ((4 * t + grp) * kD + 16 * u + col) * 4);
          acc[u] = MfmaOps<float>::mma(vv.x, w[0], acc[u]);
          acc[u] = MfmaOps<float>::mma(vv.y, w[1], acc[u]);
          acc[u] = MfmaOps<float>::mma(vv.z, w[2], acc[u]);
          acc[u] = MfmaOps<float>::mma(vv.w, w[3], acc[u]);
        }
      }
    }

    if (tile == tiles - 1) {
      const float total = allreduce_bit32(allreduce_bit16(run_sum, OpSum()), OpSum());
      const Coords c = coords(item);
      const int32_t q_row = (c.qb * kWaves + wave) * 16 + col;
      if (q_row < n_q) {
        // A fully masked row has total 0: 0 * inf = NaN, as eager softmax gives.
        const float inv = __builtin_amdgcn_rcpf(total);
        OutT* o = static_cast<OutT*>(p.out) + c.b * p.so[0] + c.h * p.so[1] + q_row * p.so[2];
#pragma unroll
        for (int u = 0; u < kDvTiles; ++u) {
          OutT vals[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) vals[r] = from_float<OutT>(acc[u][r] * inv);
          OutT* dst = o + (16 * u + 4 * grp) * p.so[3];
          if (out_vec) {
            if constexpr (sizeof(OutT) == 4) {
              *reinterpret_cast<uint4*>(dst) = *reinterpret_cast<const uint4*>(vals);
            } else {
              *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(vals);
            }
          } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) dst[r * p.so[3]] = vals[r];
          }
        }
      }
    }
    if (!more) break;
    item = next_item;
    tile = next_tile;
  }
}

// ------------------------------------------------------------------- host

// Workgroups of one MFMA instantiation that fit on a compute unit at once
// (registers and LDS), asked of the runtime once per process.
template <typename T, typename OutT, int kD, int kKeys, int kWaves>
int mfma_resident_blocks() {
  static std::atomic<int> cached{0};
  int n = cached.load(std::memory_order_relaxed);
  if (n == 0) {
    using Geo = MfmaTile<T, kD, kKeys>;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&rbf_mfma_kernel<T, OutT, kD, kKeys, kWaves>), 64 * kWaves,
            Geo::kBytes) != hipSuccess ||
        n < 1)
      n = 1;
    cached.store(n, std::memory_order_relaxed);
  }
  return n;
}

// The grid is persistent: as many workgroups as are resident at once, each
// looping over work items, so one item's loads overlap the previous one's
// products.
template <typename T, typename OutT, int kD, int kKeys, int kWaves>
hipError_t launch_mfma_w(Problem& p, hipStream_t s) {
  using Geo = MfmaTile<T, kD, kKeys>;
  const int32_t q_blocks = static_cast<int32_t>((p.Nq + kWaves * 16 - 1) / (kWaves * 16));
  const int64_t items = p.B * p.H * q_blocks;
  int64_t blocks = static_cast<int64_t>(mfma_resident_blocks<T, OutT, kD, kKeys, kWaves>()) *
                   (p.compute_units > 0 ? p.compute_units : 1);
  if (blocks > items) blocks = items;
  // Item indices (and item + grid size) stay below 2^31.
  if (items + blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  Problem k = p;  // the kernel divides work items by q_blocks with the Nq slots
  make_fast_div(q_blocks, &k.nq_mul, &k.nq_shift);
  int32_t qb = q_blocks;
  void* args[] = {&k, &qb};
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_mfma_kernel<T, OutT, kD, kKeys, kWaves>),
                         dim3(static_cast<unsigned>(blocks)), dim3(64 * kWaves), args, Geo::kBytes, s);
}

// Waves per workgroup: one per 16-row query tile of a plane, at least 4 (the
// loaders' register staging of a tile is split over the workgroup) and at
// most 8; 5 covers the 65-token comparable sets.
template <typename T, typename OutT, int kD, int kKeys>
hipError_t launch_mfma_k(Problem& p, hipStream_t s) {
  const int64_t tiles = (p.Nq + 15) / 16;
  if (tiles <= 4) return launch_mfma_w<T, OutT, kD, kKeys, 4>(p, s);
  if (tiles <= 5) return launch_mfma_w<T, OutT, kD, kKeys, 5>(p, s);
  return launch_mfma_w<T, OutT, kD, kKeys, 8>(p, s);
}

// Longest key tile per input type and head dim (register staging and LDS,
// chosen so that no instantiation spills): 128 keys, 64 for 16-bit 128-dim
// heads and fp32 64-dim heads, 32 for fp32 128-dim heads.
template <typename T, int kD>
constexpr int mfma_max_keys() {
  if constexpr (sizeof(T) == 2) return kD <= 64 ? 128 : 64;
  return kD <= 32 ? 128 : (kD == 64 ? 64 : 32);
}

template <typename T, typename OutT, int kD>
hipError_t launch_mfma_d(Problem& p, hipStream_t s) {
  // Key axes that fit one tile run as one tile (one global round trip per
  // item) of 32, 64, 80 or 128 keys, the smallest that covers them; longer
  // axes stream tiles of the longest size.
  constexpr int kMax = mfma_max_keys<T, kD>();
  if constexpr (kMax == 32) {
    return launch_mfma_k<T, OutT, kD, 32>(p, s);
  } else {
    if (p.Nk <= 32) return launch_mfma_k<T, OutT, kD, 32>(p, s);
    if constexpr (kMax >= 128) {
      if (p.Nk <= 64) return launch_mfma_k<T, OutT, kD, 64>(p, s);
      if (p.Nk <= 80) return launch_mfma_k<T, OutT, kD, 80>(p, s);
      return launch_mfma_k<T, OutT, kD, 128>(p, s);
    } else {
      return launch_mfma_k<T, OutT, kD, 64>(p, s);
    }
  }
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

// One instantiation per (input, output) dtype pair, each in its own file.
hipError_t launch_mfma_bf16_bf16(Problem& p, hipStream_t s);
hipError_t launch_mfma_bf16_f32(Problem& p, hipStream_t s);
hipError_t launch_mfma_f16_f16(Problem& p, hipStream_t s);
hipError_t launch_mfma_f16_f32(Problem& p, hipStream_t s);
hipError_t launch_mfma_f32_f32(Problem& p, hipStream_t s);

}  // namespace vectra
