// Fused RBF attention for MI355X (gfx950 / CDNA4, wave64).
//
//   out[b,h,i,:] = sum_j softmax_j(-scale[b,h] * max(|q_i|^2 + |k_j|^2 - 2 q_i.k_j, 0)
//                                  + key_bias[b,h,j]) * v[b,h,j,:]
//
// Semantics follow the reference operator (kernels/vectra_kernels/
// spatial_rbf_attention.py:47-174 and custom_ops.py:52-72):
//  * distances by the Euclidean expansion with a clamp at zero (:137);
//  * logits -scale*d plus the key bias; without a bias only keys < Nk count
//    (:139-150);
//  * an online softmax whose running maximum is replaced by 0 while it is
//    still -inf, so a row whose keys are all masked ends as 0/0 = NaN, as
//    eager softmax gives (:152-157);
//  * fp32 accumulation throughout, the result divided by the running sum and
//    converted once to the output dtype (:168-174).
// Unlike the reference kernel, the attention weights are never rounded to
// the input dtype before the value product: P.V accumulates in fp32.
//
// Kernels in this file:
//  * rbf_stream_kernel  -- few query rows per (b,h) plane (the serving shape:
//    one subject query against tens of comparables).  HBM-bound: each wave
//    owns one query row, streams the plane's K and V once with coalesced
//    128-bit loads straight into registers and reduces with DPP.
//  * rbf_generic_kernel -- any strides, head dims and alignments.
//  * rbf_mfma_kernel (rbf_mfma.hip) -- query tiles on bf16/fp16 MFMA.

#include "rbf_common.h"
#include "rbf_kernels.h"

namespace vectra {

// ------------------------------------------------------------------------
// Stream kernel.
//
// Layout: a 64-key tile of K is 64 rows of D = kChunks * Vec<T> elements.
// Lane l holds chunk (l % kChunks) of key rows  p * (64 / kChunks) + l / kChunks
// for the kChunks passes p, so each pass is one fully coalesced 1 KiB wave
// load.  V is held the same way (requires Dv == D), so a lane owns the value
// chunk of exactly the keys whose weights it computed and P.V needs no
// shuffle until the final reduction.
//
// Scheduling: the grid is persistent (a fixed number of waves, each taking
// query rows wave, wave + waves, ...).  A wave always has its next work item
// (a row and 64-key tile) in flight while it reduces the current one, so the
// softmax and P.V arithmetic of one row overlaps the HBM stream of the next;
// a one-shot grid instead leaves every wave waiting for its last bytes until
// the end of the stream and then serialises all of its arithmetic.  Every
// load of a work item (K, V, the key bias, and at a row's first tile q and
// the coefficient) is issued together; rows past Nk are loaded from row
// Nk - 1 (always in bounds) and masked afterwards, so no load is behind a
// branch.  Per-lane addresses are 32-bit offsets from wave-uniform bases.
// ------------------------------------------------------------------------

// Sums kVec accumulators per lane over the row-group lane bits (kChunks ..
// 32) of the stream layout.  Lane bits 32 and 16 use butterfly steps: a
// permlane swap of the value pair (a_i, a_{i+n/2}) hands each half of the
// wave the partner's copy of the half it keeps, so one swap and one add
// halve the values per lane.  The remaining row-group bits (below 16) are
// all-reduced with DPP.  On return res[0 .. kVec/4) are the finished sums of
// elements first_e .. first_e + kVec/4 of the lane's chunk.
template <int kChunks, int kVec>
__device__ __forceinline__ void reduce_rows_butterfly(const float* acc, float* res, int& first_e) {
  const int lane = threadIdx.x & (kWave - 1);
  constexpr int kHalf = kVec / 2, kQuarter = kVec / 4;
  float half[kHalf];
#pragma unroll
  for (int i = 0; i < kHalf; ++i) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[i]),
                                                    __float_as_uint(acc[i + kHalf]), false, false);
    half[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);  // lanes < 32: a_i, else a_{i+n/2}
  }
#pragma unroll
  for (int i = 0; i < kQuarter; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(half[i]),
                                                    __float_as_uint(half[i + kQuarter]), false, false);
    res[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
  first_e = ((lane & 32) ? kHalf : 0) + ((lane & 16) ? kQuarter : 0);
  if constexpr (kChunks < 16) {
#pragma unroll
    for (int i = 0; i < kQuarter; ++i) {
      float x = res[i];
      if constexpr (kChunks <= 1) x += dpp<0xB1>(x);
      if constexpr (kChunks <= 2) x += dpp<0x4E>(x);
      if constexpr (kChunks <= 4) {
        x += dpp<0x124>(x);
        x += dpp<0x128>(x);
      } else {
        x += dpp<0x128>(x);
      }
      res[i] = x;
    }
  }
}

template <int kPasses>
struct StreamSlot {
  uint4 k[kPasses];
  uint4 v[kPasses];
  uint32_t bias[kPasses];  // aligned words holding the key biases
  uint32_t bias_misalign;  // address & 3 of the row's bias plane (wave-uniform)
  uint4 q;
  RawScalar scale;
};

struct RowCoords {
  int32_t b, h, i;
};

__device__ __forceinline__ RowCoords row_coords(int32_t row, const Problem& p) {
  RowCoords c;
  const int32_t bh = static_cast<int32_t>(fast_div(row, p.nq_mul, p.nq_shift));
  c.i = row - bh * static_cast<int32_t>(p.Nq);
  c.b = static_cast<int32_t>(fast_div(bh, p.h_mul, p.h_shift));
  c.h = bh - c.b * static_cast<int32_t>(p.H);
  return c;
}

template <typename T, typename OutT, int kChunks, int kRows>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void rbf_stream_kernel(Problem p) {
  // kRows > 0: the wave takes rows wave * kRows .. + kRows - 1, each one key
  // tile (Nk <= 64), in a fully unrolled pipeline with no loop and no branch
  // around a load, so the compiler can wait for exactly the loads each step
  // needs.  Rows past the end are clamped to the last row: the duplicate
  // wave recomputes that row and stores the same bytes.
  // kRows == 0: rows wave, wave + grid_waves, ..., any number of key tiles.
  constexpr bool kSingleTile = kRows > 0;
  constexpr int kVec = Vec<T>::kN;
  constexpr int kRowsPerPass = kWave / kChunks;
  constexpr int kPasses = kChunks;  // kPasses * kRowsPerPass == 64 keys
  using Slot = StreamSlot<kPasses>;

  // Every argument read below, loaded in one batch (measured at the serving
  // shape: 12.4 -> 12.0 us back to back, 12.9 -> 12.65 us per isolated launch).
  args_in_sgprs(p.q, p.k, p.v, p.out, p.scale, p.bias, p.scale_dtype, p.bias_dtype, p.H, p.Nq, p.Nk);
  args_in_sgprs(p.sq[0], p.sq[1], p.sq[2], p.sk[0], p.sk[1], p.sk[2], p.sv[0], p.sv[1], p.sv[2]);
  args_in_sgprs(p.so[0], p.so[1], p.so[2], p.ssb, p.ssh, p.sbb, p.sbh, p.sbn, p.total_rows);
  args_in_sgprs(p.grid_waves, p.nq_mul, p.nq_shift, p.h_mul, p.h_shift);
  const int lane = threadIdx.x & (kWave - 1);
  const int32_t wave_id =
      static_cast<int32_t>(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t total_rows = static_cast<int32_t>(p.total_rows);
  // No barriers below: early exit is safe.
  if (wave_id * (kRows > 0 ? kRows : 1) >= total_rows) return;

  const int32_t n_waves = p.grid_waves;
  const int32_t n_k = static_cast<int32_t>(p.Nk);
  const int chunk = lane % kChunks;
  const int group = lane / kChunks;
  const uint32_t chunk_bytes = chunk * 16u;
  const uint32_t k_row_bytes = static_cast<uint32_t>(p.sk[2]) * sizeof(T);
  const uint32_t v_row_bytes = static_cast<uint32_t>(p.sv[2]) * sizeof(T);
  const bool has_bias = p.bias != nullptr;
  const int32_t bias_esize = p.bias_dtype == VECTRA_F32 ? 4 : 2;

  if (n_k == 0) {  // softmax over no keys contributes nothing (eager gives 0)
    for (int32_t row = wave_id; row < total_rows; row += n_waves) {
      const RowCoords c = row_coords(row, p);
      float zero[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) zero[e] = 0.f;
      if (group == 0)
        store_chunk<OutT, kVec>(static_cast<OutT*>(p.out) + c.b * p.so[0] + c.h * p.so[1] +
                                    c.i * p.so[2] + chunk * kVec,
                                zero);
    }
    return;
  }
  const int32_t tiles = kSingleTile ? 1 : (n_k + kWave - 1) / kWave;

  // Per-lane byte offsets of a tile's keys inside a (b, h) plane.  Those of
  // tile 0 are the same for every row, so they are computed once: issuing
  // the next row's loads then only changes wave-uniform base addresses.
  struct Offsets {
    uint32_t k[kPasses], v[kPasses], bias[kPasses];
  };
  auto tile_offsets = [&](int32_t tile) {
    Offsets o;
#pragma unroll
    for (int s = 0; s < kPasses; ++s) {
      const int32_t j = tile * kWave + s * kRowsPerPass + group;
      const uint32_t key = static_cast<uint32_t>(j < n_k - 1 ? j : n_k - 1);
      o.k[s] = key * k_row_bytes + chunk_bytes;
      o.v[s] = key * v_row_bytes + chunk_bytes;
      o.bias[s] = key * static_cast<uint32_t>(p.sbn);
    }
    return o;
  };
  const Offsets first = tile_offsets(0);

  // Issues every load of work item (row, tile) into `slot`.
  auto issue = [&](Slot& slot, int32_t row, int32_t tile) {
    const RowCoords c = row_coords(row, p);
    const char* kp = reinterpret_cast<const char*>(p.k) + (c.b * p.sk[0] + c.h * p.sk[1]) * sizeof(T);
    const char* vp = reinterpret_cast<const char*>(p.v) + (c.b * p.sv[0] + c.h * p.sv[1]) * sizeof(T);
    // With one tile per row (Nk <= 64) the offsets are loop invariant.
    const Offsets o = (kSingleTile || tile == 0) ? first : tile_offsets(tile);
    // Issue order is use order: vector loads complete in order, so q, the
    // coefficient and the biases go first and K before V; the scores are
    // then computed while V is still arriving, and only the value product
    // waits for the last bytes.
    if (tile == 0) {
      const char* qp = reinterpret_cast<const char*>(p.q) +
                       (c.b * p.sq[0] + c.h * p.sq[1] + c.i * p.sq[2]) * sizeof(T);
      slot.q = load16(qp + chunk_bytes);
      slot.scale = load_raw_scalar(p.scale, c.b * p.ssb + c.h * p.ssh, p.scale_dtype);
    }
    if (has_bias) {
      const char* bp = reinterpret_cast<const char*>(p.bias) +
                       (c.b * p.sbb + c.h * p.sbh) * bias_esize;
      slot.bias_misalign = base_misalign(bp);
#pragma unroll
      for (int s = 0; s < kPasses; ++s)
        slot.bias[s] = load_raw_scalar32(bp, slot.bias_misalign, o.bias[s], p.bias_dtype).word;
    }
#pragma unroll
    for (int s = 0; s < kPasses; ++s) slot.k[s] = load16_stream(kp + o.k[s]);
#pragma unroll
    for (int s = 0; s < kPasses; ++s) slot.v[s] = load16_stream(vp + o.v[s]);
    // Nothing that waits for a load may be scheduled among them (a wait for
    // q or a bias there would hold back the V loads by a memory latency).
    __builtin_amdgcn_sched_barrier(0);
  };

  // Per-row running state.
  uint4 q_raw = make_uint4(0, 0, 0, 0);
  float q_norm = 0.f, neg_scale = 0.f, run_max = -INFINITY, run_sum = 0.f;
  float acc[kVec];

  // Reduces work item (row, tile) held in `slot`.
  auto consume = [&](const Slot& slot, int32_t row, int32_t tile) {
    if (tile == 0) {
      q_raw = slot.q;
      q_norm = reduce_low<kChunks>(dot_chunk<T>(q_raw, q_raw, 0.f), OpSum());
      neg_scale = -decode_raw_scalar(slot.scale, p.scale_dtype);
      run_max = -INFINITY;
      run_sum = 0.f;
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[e] = 0.f;
    }
    float logit[kPasses];
    bool live[kPasses];
    float tile_max = -INFINITY;
#pragma unroll
    for (int s = 0; s < kPasses; ++s) {
      const int32_t j = tile * kWave + s * kRowsPerPass + group;
      live[s] = j < n_k;
      const float dot = reduce_low<kChunks>(dot_chunk<T>(q_raw, slot.k[s], 0.f), OpSum());
      const float k_norm = reduce_low<kChunks>(dot_chunk<T>(slot.k[s], slot.k[s], 0.f), OpSum());
      const float dist = clamp_distance((q_norm + k_norm) - 2.f * dot);
      float x = neg_scale * dist;
      if (has_bias) {
        // Position of a 2-byte bias inside its word, from the key index
        // (the same arithmetic as the load).
        const uint32_t key = static_cast<uint32_t>(j < n_k - 1 ? j : n_k - 1);
        const uint32_t bytes = key * static_cast<uint32_t>(p.sbn) * bias_esize + slot.bias_misalign;
        x += decode_raw_scalar(RawScalar{slot.bias[s], (bytes & 2u) * 8u}, p.bias_dtype);
      }
      x = live[s] ? x : -INFINITY;
      logit[s] = x;
      tile_max = fmaxf(tile_max, x);
    }
    tile_max = reduce_high<kChunks>(tile_max, OpMax());
    const float new_max = fmaxf(run_max, tile_max);
    const float safe_max = new_max == -INFINITY ? 0.f : new_max;
    const float alpha = __builtin_amdgcn_exp2f((run_max - safe_max) * kLog2e);
    float tile_sum = 0.f;
#pragma unroll
    for (int e = 0; e < kVec; ++e) acc[e] *= alpha;
    // Rows past Nk do not exist: their (clamped) values must not reach the
    // sum even as 0 * inf, so a tile with such rows zeroes them.
    const bool ragged = (tile + 1) * kWave > n_k;
#pragma unroll
    for (int s = 0; s < kPasses; ++s) {
      const float w = __builtin_amdgcn_exp2f((logit[s] - safe_max) * kLog2e);
      tile_sum += w;
      uint4 vr = slot.v[s];
      if (ragged && !live[s]) vr = make_uint4(0, 0, 0, 0);
      float vf[kVec];
      unpack<T>(vr, vf);
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[e] = fmaf(w, vf[e], acc[e]);
    }
    // Each weight is replicated over the kChunks lanes of its key row; sum
    // over row groups only.
    run_sum = run_sum * alpha + reduce_high<kChunks>(tile_sum, OpSum());
    run_max = new_max;
    if (tile == tiles - 1) {
      // Sum the accumulators over row groups; lane `lane` ends with
      // kVec / 4 finished values of its chunk, starting at element `first_e`.
      constexpr int kOut = kVec / 4;
      float res[kOut];
      int first_e;
      reduce_rows_butterfly<kChunks, kVec>(acc, res, first_e);
      // A row whose keys are all masked has run_sum 0: 0 * inf = NaN, as eager.
      const float inv = __builtin_amdgcn_rcpf(run_sum);
#pragma unroll
      for (int e = 0; e < kOut; ++e) res[e] *= inv;
      // Row groups below lane bit 16 hold copies; one of them stores.
      if ((lane & (16 - kChunks)) == 0) {
        const RowCoords c = row_coords(row, p);
        store_small<OutT, kOut>(static_cast<OutT*>(p.out) + c.b * p.so[0] + c.h * p.so[1] +
                                    c.i * p.so[2] + chunk * kVec + first_e,
                                res);
      }
    }
  };

  auto advance = [&](int32_t& row, int32_t& tile) {
    if (kSingleTile) {
      row += n_waves;
      return;
    }
    if (++tile == tiles) {
      tile = 0;
      row += n_waves;
    }
  };

  if constexpr (kRows > 0) {
    Slot slots[2];
    auto row_at = [&](int r) {
      const int32_t row = wave_id * kRows + r;
      return row < total_rows ? row : total_rows - 1;
    };
    issue(slots[0], row_at(0), 0);
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
      if (r + 1 < kRows) issue(slots[(r + 1) & 1], row_at(r + 1), 0);
      consume(slots[r & 1], row_at(r), 0);
    }
    return;
  }

  // Two slots alternate roles, so the prefetch needs no register copies.
  // Each branch has its own copy of the reduction: after a join of a path
  // that issued the prefetch and one that did not, the compiler could only
  // wait for every outstanding load, the prefetch included.
  Slot a, b;
  int32_t row = wave_id, tile = 0;
  issue(a, row, tile);
  while (true) {
    int32_t next_row = row, next_tile = tile;
    advance(next_row, next_tile);
    if (next_row < total_rows) {
      issue(b, next_row, next_tile);
      consume(a, row, tile);
    } else {
      consume(a, row, tile);
      break;
    }
    row = next_row;
    tile = next_tile;
    advance(next_row, next_tile);
    if (next_row < total_rows) {
      issue(a, next_row, next_tile);
      consume(b, row, tile);
    } else {
      consume(b, row, tile);
      break;
    }
    row = next_row;
    tile = next_tile;
  }
}

// ------------------------------------------------------------------------
// Generic kernel: one wave per (b, h, query row) and per 256-wide slice of
// the value dimension (blockIdx.y).  Scores: lane = key within a 64-key
// tile.  Value product: lane = value column, weights broadcast with
// readlane.  Handles any strides (including zero), any D and Dv.  Waves
// loop over rows with a grid stride, so the grid stays within HIP's
// per-dimension thread limit however many rows there are.
// ------------------------------------------------------------------------
template <typename T, typename OutT>
__device__ void generic_row(const Problem& p, int64_t row_id, int lane);

template <typename T, typename OutT>
__global__ __launch_bounds__(256) void rbf_generic_kernel(Problem p) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t stride = static_cast<int64_t>(gridDim.x) * 4;
  // Wave-uniform loop (no barriers inside).
  for (int64_t row_id = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6); row_id < p.total_rows;
       row_id += stride)
    generic_row<T, OutT>(p, row_id, lane);
}

template <typename T, typename OutT>
__device__ void generic_row(const Problem& p, int64_t row_id, int lane) {
  constexpr int kCols = 4;  // value columns per lane: 4 * 64 = 256 per slice
  const int64_t i = row_id % p.Nq;
  const int64_t bh = row_id / p.Nq;
  const int64_t h = bh % p.H;
  const int64_t b = bh / p.H;
  const int64_t dv0 = static_cast<int64_t>(blockIdx.y) * (kCols * kWave);

  const T* q_row = static_cast<const T*>(p.q) + b * p.sq[0] + h * p.sq[1] + i * p.sq[2];
  const T* k_plane = static_cast<const T*>(p.k) + b * p.sk[0] + h * p.sk[1];
  const T* v_plane = static_cast<const T*>(p.v) + b * p.sv[0] + h * p.sv[1];

  float q_norm = 0.f;
  for (int64_t d = lane; d < p.D; d += kWave) {
    const float x = to_float<T>(q_row[d * p.sq[3]]);
    q_norm += x * x;
  }
  q_norm = reduce_wave(q_norm, OpSum());

  const float neg_scale = -load_any(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);
  const bool has_bias = p.bias != nullptr;
  const int64_t bias_base = b * p.sbb + h * p.sbh;

  float run_max = -INFINITY, run_sum = 0.f;
  float acc[kCols];
#pragma unroll
  for (int c = 0; c < kCols; ++c) acc[c] = 0.f;

  for (int64_t j0 = 0; j0 < p.Nk; j0 += kWave) {
    const int64_t j = j0 + lane;
    const bool live = j < p.Nk;
    float logit = -INFINITY;
    if (live) {
      const T* k_row = k_plane + j * p.sk[2];
      float dot = 0.f, k_norm = 0.f;
      for (int64_t d = 0; d < p.D; ++d) {
        const float qd = to_float<T>(q_row[d * p.sq[3]]);
        const float kd = to_float<T>(k_row[d * p.sk[3]]);
        dot += qd * kd;
        k_norm += kd * kd;
      }
      const float dist = clamp_distance((q_norm + k_norm) - 2.f * dot);
      logit = neg_scale * dist;
      if (has_bias) logit += load_any(p.bias, bias_base + j * p.sbn, p.bias_dtype);
    }
    const float new_max = fmaxf(run_max, reduce_wave(logit, OpMax()));
    const float safe_max = new_max == -INFINITY ? 0.f : new_max;
    const float alpha = __builtin_amdgcn_exp2f((run_max - safe_max) * kLog2e);
    const float w = __builtin_amdgcn_exp2f((logit - safe_max) * kLog2e);
    run_sum = run_sum * alpha + reduce_wave(w, OpSum());
#pragma unroll
    for (int c = 0; c < kCols; ++c) acc[c] *= alpha;
    const int n_live = static_cast<int>(p.Nk - j0 < kWave ? p.Nk - j0 : kWave);
    for (int jj = 0; jj < n_live; ++jj) {
      const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), jj));
      const T* v_row = v_plane + (j0 + jj) * p.sv[2];
#pragma unroll
      for (int c = 0; c < kCols; ++c) {
        const int64_t d = dv0 + c * kWave + lane;
        if (d < p.Dv) acc[c] += wj * to_float<T>(v_row[d * p.sv[3]]);
      }
    }
    run_max = new_max;
  }

  OutT* o = static_cast<OutT*>(p.out) + b * p.so[0] + h * p.so[1] + i * p.so[2];
#pragma unroll
  for (int c = 0; c < kCols; ++c) {
    const int64_t d = dv0 + c * kWave + lane;
    if (d < p.Dv) o[d * p.so[3]] = from_float<OutT>(p.Nk > 0 ? acc[c] / run_sum : 0.f);
  }
}

// Row norms |x_j|^2 in fp32 (norm_precompute.py:34-64): one thread per row.
struct NormArgs {
  const void* x;
  float* out;
  int64_t B, H, N, D;
  int64_t s[4];
};

// Threads loop over rows with a grid stride.
template <typename T>
__global__ __launch_bounds__(256) void squared_norms_kernel(NormArgs a) {
  const int64_t total = a.B * a.H * a.N;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; r < total; r += stride) {
    const int64_t n = r % a.N;
    const int64_t bh = r / a.N;
    const T* row = static_cast<const T*>(a.x) + (bh / a.H) * a.s[0] + (bh % a.H) * a.s[1] + n * a.s[2];
    float acc = 0.f;
    for (int64_t d = 0; d < a.D; ++d) {
      const float t = to_float<T>(row[d * a.s[3]]);
      acc += t * t;
    }
    a.out[r] = acc;
  }
}

// ------------------------------------------------------------------------
// Launch helpers (host).
// ------------------------------------------------------------------------

static hipError_t launch(const void* fn, dim3 grid, dim3 block, Problem& p, hipStream_t s) {
  void* args[] = {&p};
  return hipLaunchKernel(fn, grid, block, args, 0, s);
}

template <typename T, typename OutT, int kChunks, int kRows>
static hipError_t launch_stream_k(Problem& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.grid_waves + 3) / 4));
  return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, kChunks, kRows>), grid,
                dim3(256), p, s);
}

// Rows per wave for one-tile rows: about `budget` waves, at most kMaxRows
// rows each (the register footprint of two slots bounds it for wide heads).
template <typename T, typename OutT, int kChunks, int kMaxRows>
static hipError_t launch_stream_c(Problem& p, hipStream_t s) {
  const int64_t budget = p.grid_waves;
  // Rows of 8 or 16 chunks with several key tiles would spill registers in
  // the looping variant: the host sends them to another kernel instead.
  if (kChunks >= 8 && p.Nk > kWave) return hipErrorInvalidValue;
  if (kChunks < 8 && p.Nk > kWave) {
    p.grid_waves = static_cast<int32_t>(p.total_rows < budget ? p.total_rows : budget);
    return launch_stream_k<T, OutT, kChunks, (kChunks < 8 ? 0 : 1)>(p, s);
  }
  const int64_t rows = p.total_rows;
  int rows_per_wave = rows > 2 * budget ? 4 : (rows > budget ? 2 : 1);
  if (rows_per_wave > kMaxRows) rows_per_wave = kMaxRows;
  p.grid_waves = static_cast<int32_t>((rows + rows_per_wave - 1) / rows_per_wave);
  if (kMaxRows >= 4 && rows_per_wave == 4) return launch_stream_k<T, OutT, kChunks, (kMaxRows >= 4 ? 4 : 1)>(p, s);
  if (kMaxRows >= 2 && rows_per_wave == 2) return launch_stream_k<T, OutT, kChunks, (kMaxRows >= 2 ? 2 : 1)>(p, s);
  return launch_stream_k<T, OutT, kChunks, 1>(p, s);
}

// p.grid_waves holds the persistent wave budget on entry; it is replaced by
// the number of waves launched.
template <typename T, typename OutT>
static hipError_t launch_stream_t(Problem& p, int chunks, hipStream_t s) {
  switch (chunks) {
    case 2: return launch_stream_c<T, OutT, 2, 4>(p, s);
    case 4: return launch_stream_c<T, OutT, 4, 4>(p, s);
    case 8: return launch_stream_c<T, OutT, 8, 4>(p, s);
    case 16: return launch_stream_c<T, OutT, 16, 1>(p, s);
    default: return hipErrorInvalidValue;
  }
}

// Workgroups of the grid-stride kernels: at most this many (of 256 threads).
constexpr int64_t kMaxGridStrideBlocks = int64_t{1} << 20;

template <typename T, typename OutT>
static hipError_t launch_generic_t(Problem& p, hipStream_t s) {
  const int64_t blocks = (p.total_rows + 3) / 4;
  const int64_t slices = (p.Dv + 255) / 256;
  if (slices > kMaxGenericSlices) return hipErrorInvalidValue;  // the host rejects these first
  const dim3 grid(static_cast<unsigned>(blocks < kMaxGridStrideBlocks ? blocks : kMaxGridStrideBlocks),
                  static_cast<unsigned>(slices));
  return launch(reinterpret_cast<const void*>(&rbf_generic_kernel<T, OutT>), grid, dim3(256), p, s);
}

// Dispatch on (input dtype, output dtype).
template <template <typename, typename> class F, typename... A>
static hipError_t by_dtype(int in_dt, int out_dt, A&&... a) {
#define VECTRA_CASE(IN_ENUM, IN_T)                                             \
  if (in_dt == IN_ENUM) {                                                      \
    if (out_dt == VECTRA_F32) return F<IN_T, float>::run(a...);                \
    if (out_dt == VECTRA_F16) return F<IN_T, _Float16>::run(a...);             \
    if (out_dt == VECTRA_BF16) return F<IN_T, __bf16>::run(a...);              \
  }
  VECTRA_CASE(VECTRA_F32, float)
  VECTRA_CASE(VECTRA_F16, _Float16)
  VECTRA_CASE(VECTRA_BF16, __bf16)
#undef VECTRA_CASE
  return hipErrorInvalidValue;
}

template <typename T, typename OutT>
struct GenericLauncher {
  static hipError_t run(Problem& p, hipStream_t s) { return launch_generic_t<T, OutT>(p, s); }
};

hipError_t launch_stream(Problem& p, int in_dt, int out_dt, int chunks, hipStream_t s) {
  // Output in the input dtype (the operator) or fp32 (parity harnesses).
  switch (in_dt) {
    case VECTRA_BF16:
      return out_dt == VECTRA_F32 ? launch_stream_t<__bf16, float>(p, chunks, s)
                                  : launch_stream_t<__bf16, __bf16>(p, chunks, s);
    case VECTRA_F16:
      return out_dt == VECTRA_F32 ? launch_stream_t<_Float16, float>(p, chunks, s)
                                  : launch_stream_t<_Float16, _Float16>(p, chunks, s);
    default:
      return launch_stream_t<float, float>(p, chunks, s);
  }
}

hipError_t launch_generic(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  return by_dtype<GenericLauncher>(in_dt, out_dt, p, s);
}

hipError_t launch_squared_norms(const void* x, int dtype, int64_t B, int64_t H, int64_t N,
                                int64_t D, const int64_t* st, float* out, hipStream_t s) {
  NormArgs a{x, out, B, H, N, D, {st[0], st[1], st[2], st[3]}};
  const int64_t blocks = (B * H * N + 255) / 256;
  const dim3 grid(static_cast<unsigned>(blocks < kMaxGridStrideBlocks ? blocks : kMaxGridStrideBlocks));
  void* args[] = {&a};
  const void* fn = nullptr;
  switch (dtype) {
    case VECTRA_F32: fn = reinterpret_cast<const void*>(&squared_norms_kernel<float>); break;
    case VECTRA_F16: fn = reinterpret_cast<const void*>(&squared_norms_kernel<_Float16>); break;
    case VECTRA_BF16: fn = reinterpret_cast<const void*>(&squared_norms_kernel<__bf16>); break;
    default: return hipErrorInvalidValue;
  }
  return hipLaunchKernel(fn, grid, dim3(256), args, 0, s);
}

}  // namespace vectra
