// Query-tile RBF attention on gfx950 matrix cores (bf16 / fp16 inputs):
// the kernel template.  Instantiated per dtype pair in rbf_mfma_<in>_<out>.hip.
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

#pragma once

#include <atomic>

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

// Work item: one (b, h) plane and one block of kWaves * 16 query rows; the
// plane's keys are streamed in tiles of kKeys.  The grid is persistent: a
// workgroup takes items blockIdx.x, blockIdx.x + gridDim.x, ...  Every
// thread owns fixed load slots of a tile (K rows, V row pairs, biases, and
// at an item's first tile its q fragment).  All of them are issued together
// into registers as soon as the previous tile has been copied to LDS, so the
// next tile's HBM latency overlaps this tile's products and softmax.
template <typename T, int kD, int kDv, int kKeys, int kWaves>
struct MfmaStage {
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int kDChunks = kD / 8;
  static constexpr int kDvChunks = kDv / 8;
  static constexpr int kKSteps = (kD + 31) / 32;
  static constexpr int kKSlots = (kKeys * kDChunks + kThreads - 1) / kThreads;
  static constexpr int kVSlots = ((kKeys / 2) * kDvChunks + kThreads - 1) / kThreads;
  static constexpr int kBSlots = (kKeys + kThreads - 1) / kThreads;
  uint4 k[kKSlots];
  uint4 v[kVSlots][2];  // rows 2p and 2p + 1 of one 16-byte column chunk
  uint32_t bias[kBSlots];
  uint32_t bias_misalign;  // address & 3 of the item's bias plane
  uint4 q[kKSteps];
  RawScalar scale;
};

template <typename T, typename OutT, int kD, int kDv, int kKeys, int kWaves>
__global__ __launch_bounds__(64 * kWaves) void rbf_mfma_kernel(Problem p, int32_t q_blocks) {
  using Geo = MfmaTile<T, kD, kDv, kKeys>;
  using Stage = MfmaStage<T, kD, kDv, kKeys, kWaves>;
  using Vec8 = typename Mfma<T>::vec8;
  constexpr int kThreads = Stage::kThreads;
  constexpr int kNTiles = kKeys / 16;   // 16-key blocks per tile
  constexpr int kPSteps = kKeys / 32;   // deep steps of O^T = V^T . P^T
  constexpr int kDvTiles = kDv / 16;
  constexpr int kDChunks = Stage::kDChunks;
  constexpr int kDvChunks = Stage::kDvChunks;
  static_assert(kD % 8 == 0 && kDv % 16 == 0 && kKeys % 32 == 0 && kKeys <= 128, "tile shape");
  static_assert(64 % kDChunks == 0, "a K row's chunks stay inside one wave");

  extern __shared__ __align__(16) unsigned char lds[];
  T* k_lds = reinterpret_cast<T*>(lds);
  T* vt_lds = reinterpret_cast<T*>(lds + Geo::kKBytes);
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

  // Padding columns of the K tile (head dims kD .. kDpad) stay zero.
  if constexpr (Geo::kDpad > kD) {
    for (int i = tid; i < kKeys * (Geo::kDpad - kD); i += kThreads) {
      const int key = i / (Geo::kDpad - kD);
      k_lds[key * Geo::kKStride + kD + i % (Geo::kDpad - kD)] = static_cast<T>(0.f);
    }
  }

  // Issues every load of (item, tile) into `st`.  Rows past Nk read row
  // Nk - 1 (in bounds) and are masked when written to LDS.
  auto issue = [&](Stage& st, int32_t item, int32_t tile) {
    const Coords c = coords(item);
    const T* k_plane = static_cast<const T*>(p.k) + c.b * p.sk[0] + c.h * p.sk[1];
    const T* v_plane = static_cast<const T*>(p.v) + c.b * p.sv[0] + c.h * p.sv[1];
    const int32_t j0 = tile * kKeys;
#pragma unroll
    for (int s = 0; s < Stage::kKSlots; ++s) {
      const int slot = tid + s * kThreads;
      const int key = slot / kDChunks;
      const int32_t j = min(j0 + key, n_k - 1);
      if (slot < kKeys * kDChunks) st.k[s] = load16_stream(k_plane + j * p.sk[2] + (slot % kDChunks) * 8);
    }
#pragma unroll
    for (int s = 0; s < Stage::kVSlots; ++s) {
      const int slot = tid + s * kThreads;
      const int pair = slot / kDvChunks;
      const int32_t j = j0 + 2 * pair;
      if (slot < (kKeys / 2) * kDvChunks) {
        const T* src = v_plane + (slot % kDvChunks) * 8;
        st.v[s][0] = load16_stream(src + min(j, n_k - 1) * p.sv[2]);
        st.v[s][1] = load16_stream(src + min(j + 1, n_k - 1) * p.sv[2]);
      }
    }
    if (has_bias) {
      const char* bp = reinterpret_cast<const char*>(p.bias) + (c.b * p.sbb + c.h * p.sbh) * bias_esize;
      st.bias_misalign = base_misalign(bp);
#pragma unroll
      for (int s = 0; s < Stage::kBSlots; ++s) {
        const int key = tid + s * kThreads;
        const uint32_t j = static_cast<uint32_t>(min(j0 + key, n_k - 1));
        if (key < kKeys)
          st.bias[s] = load_raw_scalar32(bp, st.bias_misalign, j * static_cast<uint32_t>(p.sbn), p.bias_dtype).word;
      }
    }
    if (tile == 0) {
      const int32_t q_row = (c.qb * kWaves + wave) * 16 + col;
      const T* q_src = static_cast<const T*>(p.q) + c.b * p.sq[0] + c.h * p.sq[1] +
                       min(q_row, n_q - 1) * p.sq[2];
#pragma unroll
      for (int ks = 0; ks < Geo::kKSteps; ++ks) {
        const int d0 = 32 * ks + 8 * grp;
        if (d0 < kD) st.q[ks] = load16(q_src + d0);
      }
      st.scale = load_raw_scalar(p.scale, c.b * p.ssb + c.h * p.ssh, p.scale_dtype);
    }
  };

  // Copies a staged tile into LDS: K rows and their norms, V transposed (two
  // keys per 32-bit write), biases as fp32 with keys past Nk at -inf.
  auto publish = [&](const Stage& st, int32_t tile) {
    const int32_t j0 = tile * kKeys;
#pragma unroll
    for (int s = 0; s < Stage::kKSlots; ++s) {
      const int slot = tid + s * kThreads;
      if (Stage::kKSlots * kThreads == kKeys * kDChunks || slot < kKeys * kDChunks) {
        const int key = slot / kDChunks;
        const uint4 raw = j0 + key < n_k ? st.k[s] : make_uint4(0, 0, 0, 0);
        *reinterpret_cast<uint4*>(k_lds + key * Geo::kKStride + (slot % kDChunks) * 8) = raw;
        const float sq = reduce_low<kDChunks>(dot_chunk<T>(raw, raw, 0.f), OpSum());
        if (slot % kDChunks == 0) kn_lds[key] = sq;
      }
    }
#pragma unroll
    for (int s = 0; s < Stage::kVSlots; ++s) {
      const int slot = tid + s * kThreads;
      if (slot < (kKeys / 2) * kDvChunks) {
        const int pair = slot / kDvChunks;
        const int d0 = (slot % kDvChunks) * 8;
        const uint4 r0 = j0 + 2 * pair < n_k ? st.v[s][0] : make_uint4(0, 0, 0, 0);
        const uint4 r1 = j0 + 2 * pair + 1 < n_k ? st.v[s][1] : make_uint4(0, 0, 0, 0);
        const uint32_t w0[4] = {r0.x, r0.y, r0.z, r0.w};
        const uint32_t w1[4] = {r1.x, r1.y, r1.z, r1.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // Elements 2e and 2e+1 of the chunk, for keys 2p (low half) and 2p+1.
          const uint32_t even = (w0[e] & 0xffffu) | (w1[e] << 16);
          const uint32_t odd = (w0[e] >> 16) | (w1[e] & 0xffff0000u);
          *reinterpret_cast<uint32_t*>(vt_lds + (d0 + 2 * e) * Geo::kVStride + 2 * pair) = even;
          *reinterpret_cast<uint32_t*>(vt_lds + (d0 + 2 * e + 1) * Geo::kVStride + 2 * pair) = odd;
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
            x = decode_raw_scalar(RawScalar{st.bias[s], (bytes & 2u) * 8u}, p.bias_dtype);
          }
        }
        bias_lds[key] = x;
      }
    }
  };

  Vec8 q_frag[Geo::kKSteps];
  float q_norm = 0.f, neg_scale = 0.f, run_max = -INFINITY, run_sum = 0.f;
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
      q_norm = 0.f;
#pragma unroll
      for (int ks = 0; ks < Geo::kKSteps; ++ks) {
        const bool in_d = 32 * ks + 8 * grp < kD;
        const uint4 raw = (q_live && in_d) ? st.q[ks] : make_uint4(0, 0, 0, 0);
        q_frag[ks] = __builtin_bit_cast(Vec8, raw);
        q_norm = dot_chunk<T>(raw, raw, q_norm);
      }
      q_norm = allreduce_bit32(allreduce_bit16(q_norm, OpSum()), OpSum());
      neg_scale = -decode_raw_scalar(st.scale, p.scale_dtype);
      run_max = -INFINITY;
      run_sum = 0.f;
#pragma unroll
      for (int u = 0; u < kDvTiles; ++u) acc[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    const bool more = next_item < items;
    if (more) issue(st, next_item, next_tile);  // in flight while this tile is reduced

    // Scores S^T for this lane's query against keys 16t + 4g + r.
    float logit[kNTiles][4];
    float tile_max = -INFINITY;
#pragma unroll
    for (int t = 0; t < kNTiles; ++t) {
      f32x4 sc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < Geo::kKSteps; ++ks) {
        const Vec8 a = *reinterpret_cast<const Vec8*>(k_lds + (16 * t + col) * Geo::kKStride + 32 * ks + 8 * grp);
        sc = Mfma<T>::run(a, q_frag[ks], sc);
      }
      const float4 kn = *reinterpret_cast<const float4*>(kn_lds + 16 * t + 4 * grp);
      const float4 bias = *reinterpret_cast<const float4*>(bias_lds + 16 * t + 4 * grp);
      const float knv[4] = {kn.x, kn.y, kn.z, kn.w};
      const float bv[4] = {bias.x, bias.y, bias.z, bias.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float dist = fmaxf((q_norm + knv[r]) - 2.f * sc[r], 0.f);
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
#pragma unroll
          for (int r = 0; r < 4; ++r) o[(16 * u + 4 * grp + r) * p.so[3]] = from_float<OutT>(acc[u][r] * inv);
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
    using Geo = MfmaTile<T, kD, kD, kKeys>;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &n, reinterpret_cast<const void*>(&rbf_mfma_kernel<T, OutT, kD, kD, kKeys, kWaves>), 64 * kWaves,
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
  using Geo = MfmaTile<T, kD, kD, kKeys>;
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
  return hipLaunchKernel(reinterpret_cast<const void*>(&rbf_mfma_kernel<T, OutT, kD, kD, kKeys, kWaves>),
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

template <typename T, typename OutT, int kD>
hipError_t launch_mfma_d(Problem& p, hipStream_t s) {
  // Key axes up to 128 run as one tile (one global round trip per item) of
  // 64, 96 or 128 keys, the smallest that covers them; longer axes stream
  // 128-key tiles.  128 head dims use 64-key tiles (register staging).
  if constexpr (kD >= 128) {
    return launch_mfma_k<T, OutT, kD, 64>(p, s);
  } else {
    if (p.Nk <= 64) return launch_mfma_k<T, OutT, kD, 64>(p, s);
    if (p.Nk <= 96) return launch_mfma_k<T, OutT, kD, 96>(p, s);
    return launch_mfma_k<T, OutT, kD, 128>(p, s);
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

}  // namespace vectra
