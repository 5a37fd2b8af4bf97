// Fused RBF attention for MI355X (gfx950 / CDNA4, wave64).
//
//   out[b,h,i,:] = sum_j softmax_j(-scale[b,h] * max(|q_i|^2 + |k_j|^2 - 2 q_i.k_j, 0)
//                                  + key_bias[b,h,j]) * v[b,h,j,:]
//
// Semantics follow the reference operator (kernels/vectra_kernels/
// spatial_rbf_attention.py:47-174 and custom_ops.py:70-115):
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
// Scheduling: the plane decomposition is wave-uniform (scalar registers);
// every load of a tile (K, V, the key bias, and for the first tile q and the
// coefficient) is issued before the first wait, and the next tile's loads
// are issued before the current tile is reduced.  Rows past Nk are loaded
// from row Nk-1 (always in bounds) and masked afterwards, so no load sits
// behind a branch.
// ------------------------------------------------------------------------

template <typename T, int kPasses, int kRowsPerPass>
struct StreamTile {
  uint4 k[kPasses];
  uint4 v[kPasses];
  RawScalar bias[kPasses];
};

template <typename T, int kPasses, int kRowsPerPass>
__device__ __forceinline__ void load_tile(StreamTile<T, kPasses, kRowsPerPass>& t, const Problem& p,
                                          const char* k_base, const char* v_base,
                                          int64_t k_row_bytes, int64_t v_row_bytes,
                                          int64_t bias_base, int64_t j0, int group) {
  const int64_t last = p.Nk - 1;
  int64_t row[kPasses];
#pragma unroll
  for (int s = 0; s < kPasses; ++s) {
    const int64_t j = j0 + s * kRowsPerPass + group;
    row[s] = j < last ? j : last;
  }
#pragma unroll
  for (int s = 0; s < kPasses; ++s) t.k[s] = load16_stream(k_base + row[s] * k_row_bytes);
#pragma unroll
  for (int s = 0; s < kPasses; ++s) t.v[s] = load16_stream(v_base + row[s] * v_row_bytes);
  if (p.bias != nullptr) {
#pragma unroll
    for (int s = 0; s < kPasses; ++s)
      t.bias[s] = load_raw_scalar(p.bias, bias_base + row[s] * p.sbn, p.bias_dtype);
  }
}

template <typename T, typename OutT, int kChunks>
__global__ __launch_bounds__(256) void rbf_stream_kernel(Problem p) {
  constexpr int kVec = Vec<T>::kN;
  constexpr int kRowsPerPass = kWave / kChunks;
  constexpr int kPasses = kChunks;  // kPasses * kRowsPerPass == 64 keys
  using Tile = StreamTile<T, kPasses, kRowsPerPass>;

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int32_t row_id = static_cast<int32_t>(blockIdx.x) * 4 + wave;
  if (row_id >= p.total_rows) return;  // no barriers below: early exit is safe

  // Wave-uniform decomposition (the host guarantees B*H*Nq < 2^31).
  const int32_t n_q = static_cast<int32_t>(p.Nq);
  const int32_t heads = static_cast<int32_t>(p.H);
  const int32_t bh = n_q == 1 ? row_id : row_id / n_q;
  const int32_t i = row_id - bh * n_q;
  const int32_t b = __builtin_amdgcn_readfirstlane(bh / heads);
  const int32_t h = __builtin_amdgcn_readfirstlane(bh - b * heads);
  const int chunk = lane % kChunks;
  const int group = lane / kChunks;

  const char* k_base = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + b * p.sk[0] +
                                                     h * p.sk[1] + chunk * kVec);
  const char* v_base = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + b * p.sv[0] +
                                                     h * p.sv[1] + chunk * kVec);
  const int64_t k_row_bytes = p.sk[2] * static_cast<int64_t>(sizeof(T));
  const int64_t v_row_bytes = p.sv[2] * static_cast<int64_t>(sizeof(T));
  const int64_t bias_base = b * p.sbb + h * p.sbh;
  const bool has_bias = p.bias != nullptr;

  float run_max = -INFINITY;
  float run_sum = 0.f;
  float acc[kVec];
#pragma unroll
  for (int e = 0; e < kVec; ++e) acc[e] = 0.f;

  if (p.Nk > 0) {
    // First tile, q and the coefficient: all in flight before any wait.
    Tile cur;
    load_tile(cur, p, k_base, v_base, k_row_bytes, v_row_bytes, bias_base, 0, group);
    const uint4 q_raw = load16(static_cast<const T*>(p.q) + b * p.sq[0] + h * p.sq[1] +
                               i * p.sq[2] + chunk * kVec);
    const RawScalar scale_raw = load_raw_scalar(p.scale, b * p.ssb + h * p.ssh, p.scale_dtype);

    float qf[kVec];
    unpack<T>(q_raw, qf);
    float q_norm = 0.f;
#pragma unroll
    for (int e = 0; e < kVec; ++e) q_norm += qf[e] * qf[e];
    q_norm = reduce_low<kChunks>(q_norm, OpSum());
    const float neg_scale = -decode_raw_scalar(scale_raw, p.scale_dtype);

    for (int64_t j0 = 0; j0 < p.Nk; j0 += kWave) {
      Tile next;
      const bool more = j0 + kWave < p.Nk;
      if (more)
        load_tile(next, p, k_base, v_base, k_row_bytes, v_row_bytes, bias_base, j0 + kWave, group);

      float logit[kPasses];
      bool live[kPasses];
      float tile_max = -INFINITY;
#pragma unroll
      for (int s = 0; s < kPasses; ++s) {
        live[s] = j0 + s * kRowsPerPass + group < p.Nk;
        float kf[kVec];
        unpack<T>(cur.k[s], kf);
        float dot = 0.f, k_norm = 0.f;
#pragma unroll
        for (int e = 0; e < kVec; ++e) {
          dot += qf[e] * kf[e];
          k_norm += kf[e] * kf[e];
        }
        dot = reduce_low<kChunks>(dot, OpSum());
        k_norm = reduce_low<kChunks>(k_norm, OpSum());
        const float dist = fmaxf((q_norm + k_norm) - 2.f * dot, 0.f);
        float x = neg_scale * dist;
        if (has_bias) x += decode_raw_scalar(cur.bias[s], p.bias_dtype);
        x = live[s] ? x : -INFINITY;
        logit[s] = x;
        tile_max = fmaxf(tile_max, x);
      }
      tile_max = reduce_high<kChunks>(tile_max, OpMax());
      const float new_max = fmaxf(run_max, tile_max);
      const float safe_max = new_max == -INFINITY ? 0.f : new_max;
      const float alpha = __builtin_amdgcn_exp2f((run_max - safe_max) * kLog2e);

      float tile_sum = 0.f;
      float pv[kVec];
#pragma unroll
      for (int e = 0; e < kVec; ++e) pv[e] = 0.f;
#pragma unroll
      for (int s = 0; s < kPasses; ++s) {
        const float w = __builtin_amdgcn_exp2f((logit[s] - safe_max) * kLog2e);
        tile_sum += w;
        float vf[kVec];
        unpack<T>(cur.v[s], vf);
        // Rows past Nk do not exist: their (clamped) values must not reach
        // the sum even as 0 * inf.
#pragma unroll
        for (int e = 0; e < kVec; ++e) pv[e] += w * (live[s] ? vf[e] : 0.f);
      }
      // Each weight is replicated over the kChunks lanes of its key row; sum
      // over row groups only.
      tile_sum = reduce_high<kChunks>(tile_sum, OpSum());
      run_sum = run_sum * alpha + tile_sum;
#pragma unroll
      for (int e = 0; e < kVec; ++e) acc[e] = acc[e] * alpha + pv[e];
      run_max = new_max;
      if (more) cur = next;
    }
  }

#pragma unroll
  for (int e = 0; e < kVec; ++e) acc[e] = reduce_high<kChunks>(acc[e], OpSum());

  if (group == 0) {
    float res[kVec];
#pragma unroll
    for (int e = 0; e < kVec; ++e) res[e] = p.Nk > 0 ? acc[e] / run_sum : 0.f;
    OutT* o = static_cast<OutT*>(p.out) + b * p.so[0] + h * p.so[1] + i * p.so[2] + chunk * kVec;
    store_chunk<OutT, kVec>(o, res);
  }
}

// ------------------------------------------------------------------------
// Generic kernel: one wave per (b, h, query row) and per 256-wide slice of
// the value dimension (blockIdx.y).  Scores: lane = key within a 64-key
// tile.  Value product: lane = value column, weights broadcast with
// readlane.  Handles any strides (including zero), any D and Dv.
// ------------------------------------------------------------------------
template <typename T, typename OutT>
__global__ __launch_bounds__(256) void rbf_generic_kernel(Problem p) {
  constexpr int kCols = 4;  // value columns per lane: 4 * 64 = 256 per slice
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row_id = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row_id >= p.total_rows) return;  // no barriers below

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
      const float dist = fmaxf((q_norm + k_norm) - 2.f * dot, 0.f);
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

template <typename T>
__global__ __launch_bounds__(256) void squared_norms_kernel(NormArgs a) {
  const int64_t r = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (r >= a.B * a.H * a.N) return;
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

// ------------------------------------------------------------------------
// Launch helpers (host).
// ------------------------------------------------------------------------

static hipError_t launch(const void* fn, dim3 grid, dim3 block, Problem& p, hipStream_t s) {
  void* args[] = {&p};
  return hipLaunchKernel(fn, grid, block, args, 0, s);
}

template <typename T, typename OutT>
static hipError_t launch_stream_t(Problem& p, int chunks, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.total_rows + 3) / 4));
  const dim3 block(256);
  switch (chunks) {
    case 1: return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, 1>), grid, block, p, s);
    case 2: return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, 2>), grid, block, p, s);
    case 4: return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, 4>), grid, block, p, s);
    case 8: return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, 8>), grid, block, p, s);
    case 16: return launch(reinterpret_cast<const void*>(&rbf_stream_kernel<T, OutT, 16>), grid, block, p, s);
    default: return hipErrorInvalidValue;
  }
}

template <typename T, typename OutT>
static hipError_t launch_generic_t(Problem& p, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((p.total_rows + 3) / 4),
                  static_cast<unsigned>((p.Dv + 255) / 256));
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
struct StreamLauncher {
  static hipError_t run(Problem& p, int chunks, hipStream_t s) {
    return launch_stream_t<T, OutT>(p, chunks, s);
  }
};
template <typename T, typename OutT>
struct GenericLauncher {
  static hipError_t run(Problem& p, hipStream_t s) { return launch_generic_t<T, OutT>(p, s); }
};

hipError_t launch_stream(Problem& p, int in_dt, int out_dt, int chunks, hipStream_t s) {
  return by_dtype<StreamLauncher>(in_dt, out_dt, p, chunks, s);
}

hipError_t launch_generic(Problem& p, int in_dt, int out_dt, hipStream_t s) {
  return by_dtype<GenericLauncher>(in_dt, out_dt, p, s);
}

hipError_t launch_squared_norms(const void* x, int dtype, int64_t B, int64_t H, int64_t N,
                                int64_t D, const int64_t* st, float* out, hipStream_t s) {
  NormArgs a{x, out, B, H, N, D, {st[0], st[1], st[2], st[3]}};
  const dim3 grid(static_cast<unsigned>((B * H * N + 255) / 256));
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
