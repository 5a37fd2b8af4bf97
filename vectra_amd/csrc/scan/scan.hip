// Distance scans of the engine's vector search on gfx950: the C ABI of
// include/vectra_scan.h and its kernels (libvectra_scan.so).
//
// Every output equals, bit for bit, what the reference function returns for
// the same inputs (engine/src/index/simd_distance.cc, pq_codec.cc), because
// each kernel performs the reference's floating-point operations in the
// reference's order:
//
// * Row distances (L2SquaredDistance :36-51, InnerProduct :53-62,
//   SquaredNorm :64-66).  The reference keeps sixteen accumulators: element
//   i + j of every full 16-element step is added to accumulator j, then the
//   accumulators are folded pairwise (ReduceLanes :27-32, widths 8, 4, 2, 1)
//   and the last dimension % 16 elements are added one at a time.  Here the
//   sixteen accumulators are sixteen lanes: a group of 16 lanes computes one
//   distance, lane j loading element i + j of each step (one 64-byte segment
//   per row and step, so a wave reads four rows' segments per load), the fold
//   is a shuffle tree over the group with the same pairs, and the tail terms,
//   computed in parallel by lanes 0 .. tail - 1, are added in order.  A group
//   keeps up to four queries' accumulators, so a row is read once for four
//   queries.
// * ADC distances (PqAdcDistance :68-81): one lane per code, four chains over
//   sub-spaces s .. s + 3, combined as (l0 + l1) + (l2 + l3), then the
//   remaining sub-spaces; the query's table sits in LDS when it fits, and
//   codes of up to 32 bytes on 16-byte boundaries arrive in 16-byte loads,
//   the next codes requested before the current ones are summed.
// * ADC tables (ProductQuantizer::ComputeDistanceTable, pq_codec.cc:208-217):
//   one lane per (query, sub-space, centroid), the L2 reduction above written
//   out sequentially in one lane.
//
// No multiply is fused into an add (this file is compiled with
// -ffp-contract=off, and the pragma below says the same), matching the
// reference's ISO C++ build.  The scans are bound by HBM reads of the rows or
// codes; nothing here is reshaped into a matrix product, which would change
// the order of the sums.
#pragma clang fp contract(off)

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <type_traits>

#include "vectra_scan.h"

namespace vectra_scan {
namespace {

constexpr int kLanes = 16;                       // accumulators of one distance
constexpr int kThreads = 256;                    // per workgroup
constexpr int kGroupsPerBlock = kThreads / kLanes;
constexpr int kUnroll = 8;                       // 16-element steps loaded together
constexpr int kQueryBlock = 4;                   // queries sharing one read of a row
constexpr int64_t kMaxBlocksX = 1 << 20;         // grid-stride beyond this
// Scans run on at most this many workgroups (8 per compute unit of an
// MI355X), each looping over candidates: per-workgroup set-up (query
// registers, an ADC table in LDS) is paid once for many candidates.
constexpr int64_t kScanBlocks = 2048;
constexpr int64_t kMaxBlocksY = 65535;
constexpr int kMaxLdsTableSubspaces = 64;        // 64 KiB of LDS per table

struct RowScan {
  const float* queries;
  const float* rows;
  const uint32_t* ids;
  float* out;
  int64_t query_stride, row_stride, out_stride;
  int64_t num_rows, num_cand;
  int32_t dim, num_queries;
};

// The term one element adds to an accumulator.
template <int kMetric>
__device__ __forceinline__ float term(float query, float row) {
  if constexpr (kMetric == VECTRA_SCAN_L2_SQUARED) {
    const float d = query - row;
    return d * d;
  } else {
    return query * row;  // inner product; the squared norm passes the row twice
  }
}

// ReduceLanes over a 16-lane group (one DPP row): lane i < w adds lane i + w,
// for w = 8, 4, 2, 1, and lane 0 ends with the reference's sum.  Each step is
// a row shift (lane i reads lane i + w of its row, zero past the row's end)
// and an add; lanes >= w add values no lane below w reads later.  The group
// must be wholly active, as it is wherever this is called.
__device__ __forceinline__ float reduce_lanes(float sum) {
  const auto shl = [](float x, auto w_tag) {
    constexpr int kW = decltype(w_tag)::value;
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), 0x100 + kW, 0xf, 0xf, true));
  };
  sum = sum + shl(sum, std::integral_constant<int, 8>{});
  sum = sum + shl(sum, std::integral_constant<int, 4>{});
  sum = sum + shl(sum, std::integral_constant<int, 2>{});
  sum = sum + shl(sum, std::integral_constant<int, 1>{});
  return sum;
}
static_assert(kLanes == 16, "one DPP row per distance");

template <int kMetric, int kQB, bool kIds>
__global__ __launch_bounds__(kThreads) void scan_rows_kernel(RowScan p) {
  constexpr bool kNorm = kMetric == VECTRA_SCAN_SQUARED_NORM;
  const int lane = static_cast<int>(threadIdx.x) & (kLanes - 1);
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / kLanes;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kGroupsPerBlock;
  const int q0 = static_cast<int>(blockIdx.y) * kQB;
  const int nq = min(kQB, p.num_queries - q0);  // >= 1: the grid has no empty query blocks
  const int full = p.dim - p.dim % kLanes;
  const int tail = p.dim - full;
  // Lane `lane`'s element of query q0 + j is at qlane + j * query_stride.
  const float* qlane = kNorm ? nullptr : p.queries + static_cast<int64_t>(q0) * p.query_stride + lane;
  // Element i + lane of query q0 + j (the queries stay in the caches).
  auto query = [&](int j, int i) -> float { return qlane[static_cast<int64_t>(j) * p.query_stride + i]; };

  for (int64_t cand = first; cand < p.num_cand; cand += step) {
    int64_t row = cand;
    bool valid = true;
    if constexpr (kIds) {
      const uint32_t id = p.ids[cand];
      valid = static_cast<int64_t>(id) < p.num_rows;
      row = valid ? id : 0;
    }
    const float* rlane = p.rows + row * p.row_stride + lane;
    float acc[kQB];
#pragma unroll
    for (int j = 0; j < kQB; ++j) acc[j] = 0.f;
    if (valid) {
      int i = 0;
      for (; i + kLanes * kUnroll <= full; i += kLanes * kUnroll) {
        float rv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) rv[u] = rlane[i + kLanes * u];
#pragma unroll
        for (int j = 0; j < kQB; ++j) {
          if (j < nq) {
            float qv[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) qv[u] = kNorm ? rv[u] : query(j, i + kLanes * u);
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) acc[j] = acc[j] + term<kMetric>(qv[u], rv[u]);
          }
        }
      }
      for (; i < full; i += kLanes) {
        const float r = rlane[i];
#pragma unroll
        for (int j = 0; j < kQB; ++j) {
          if (j < nq) acc[j] = acc[j] + term<kMetric>(kNorm ? r : query(j, i), r);
        }
      }
    }
    const float rtail = valid && lane < tail ? rlane[full] : 0.f;
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      if (j >= nq) break;
      // ReduceLanes: lane i < width adds lane i + width, widths 8, 4, 2, 1
      // (through LDS permutes: measured 1.3% faster here than the DPP form,
      // which the multi-query and top-k scans use).
      float sum = acc[j];
#pragma unroll
      for (int width = kLanes / 2; width > 0; width /= 2) {
        const float other = __shfl_down(sum, width, kLanes);
        if (lane < width) sum = sum + other;
      }
      // The tail, element by element in order (lane k holds element full + k).
      float t = 0.f;
      if (valid && lane < tail) t = term<kMetric>(kNorm ? rtail : query(j, full), rtail);
      for (int k = 0; k < tail; ++k) sum = sum + __shfl(t, k, kLanes);
      if (lane == 0) p.out[static_cast<int64_t>(q0 + j) * p.out_stride + cand] = valid ? sum : NAN;
    }
  }
}

// The same scan for rows of kDim (a multiple of 16 up to 128: the engine's
// 128) floats, on a capped grid: each 16-lane group keeps the kQB queries'
// elements lane + 16u in registers for all its candidates, and two register
// sets of rows, the next candidate's requested before the current one is
// summed.  Every load is issued (a candidate past the end re-reads the last
// one, an id past the rows reads row 0, and both are masked), so the compiler
// waits for exactly the older set; with the query loads or row loads behind a
// branch it would wait for every load in flight.  Each distance's operations
// are scan_rows_kernel's, in its order.  Requires num_rows >= 1.
template <int kMetric, int kQB, bool kIds, int kDim>
__global__ __launch_bounds__(kThreads) void scan_rows_pipe_kernel(RowScan p) {
  static_assert(kDim % kLanes == 0 && kDim <= kLanes * kUnroll, "one unrolled pass per row");
  constexpr bool kNorm = kMetric == VECTRA_SCAN_SQUARED_NORM;
  constexpr int kPer = kDim / kLanes;
  const int lane = static_cast<int>(threadIdx.x) & (kLanes - 1);
  const int64_t first = (static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x) / kLanes;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kGroupsPerBlock;
  const int q0 = static_cast<int>(blockIdx.y) * kQB;
  const int nq = min(kQB, p.num_queries - q0);
  const int64_t last = p.num_cand - 1;
  float qv[kQB][kPer];
#pragma unroll
  for (int j = 0; j < kQB; ++j)
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      qv[j][u] = kNorm ? 0.f : p.queries[static_cast<int64_t>(q0 + (j < nq ? j : 0)) * p.query_stride + lane + kLanes * u];
  struct Rows {
    float v[kPer];
    bool ok;
  };
  auto load = [&](int64_t cand, Rows& r) {
    const int64_t c = cand < last ? cand : last;
    int64_t row = c;
    r.ok = cand <= last;
    if constexpr (kIds) {
      const uint32_t id = p.ids[c];
      r.ok = r.ok && static_cast<int64_t>(id) < p.num_rows;
      row = r.ok ? id : 0;
    }
    const float* rl = p.rows + row * p.row_stride + lane;
#pragma unroll
    for (int u = 0; u < kPer; ++u) r.v[u] = rl[kLanes * u];
  };
  auto emit = [&](int64_t cand, const Rows& r) {
#pragma unroll
    for (int j = 0; j < kQB; ++j) {
      if (j >= nq) break;
      float sum = 0.f;
#pragma unroll
      for (int u = 0; u < kPer; ++u) sum = sum + term<kMetric>(kNorm ? r.v[u] : qv[j][u], r.v[u]);
      sum = reduce_lanes(sum);  // ReduceLanes
      if (lane == 0 && cand <= last) p.out[static_cast<int64_t>(q0 + j) * p.out_stride + cand] = r.ok ? sum : NAN;
    }
  };
  Rows a, b;
  int64_t cand = first;
  load(cand, a);
  for (; cand <= last; cand += 2 * step) {
    load(cand + step, b);
    emit(cand, a);
    load(cand + 2 * step, a);
    emit(cand + step, b);
  }
}

struct PqTable {
  const float* queries;
  const float* codebooks;
  float* tables;
  int64_t query_stride, table_stride, total;  // total = num_queries * subspaces * 256
  int32_t subspaces, dsub;
  int32_t num_queries;
};

// L2SquaredDistance(sub-vector, centroid, dsub) with the reference's sixteen
// accumulators held in registers.  kDsub is the sub-vector length when known
// at compile time, 0 for `dsub`: with a constant length every load of the
// operands is issued before the first term, where a loop of unknown length
// waits for each load in turn.
template <int kDsub>
__device__ __forceinline__ float table_entry(const float* sub, const float* centroid, int dsub_rt) {
  const int dsub = kDsub > 0 ? kDsub : dsub_rt;
  float lanes[kLanes];
#pragma unroll
  for (int j = 0; j < kLanes; ++j) lanes[j] = 0.f;
  const int full = dsub - dsub % kLanes;
  for (int i = 0; i < full; i += kLanes) {
#pragma unroll
    for (int j = 0; j < kLanes; ++j) lanes[j] = lanes[j] + term<VECTRA_SCAN_L2_SQUARED>(sub[i + j], centroid[i + j]);
  }
#pragma unroll
  for (int width = kLanes / 2; width > 0; width /= 2) {
#pragma unroll
    for (int j = 0; j < width; ++j) lanes[j] = lanes[j] + lanes[j + width];
  }
  float sum = lanes[0];
  for (int i = full; i < dsub; ++i) sum = sum + term<VECTRA_SCAN_L2_SQUARED>(sub[i], centroid[i]);
  return sum;
}

// One lane per table entry, any sub-vector length.
__global__ __launch_bounds__(kThreads) void pq_table_kernel(PqTable p) {
  // total < 2^31 (checked on the host): 32-bit index arithmetic.
  for (uint32_t t = blockIdx.x * kThreads + threadIdx.x; t < static_cast<uint32_t>(p.total); t += gridDim.x * kThreads) {
    const int c = static_cast<int>(t % VECTRA_PQ_CENTROIDS);
    const uint32_t qs = t / VECTRA_PQ_CENTROIDS;
    const int s = static_cast<int>(qs % static_cast<uint32_t>(p.subspaces));
    const int64_t q = qs / static_cast<uint32_t>(p.subspaces);
    const float* sub = p.queries + q * p.query_stride + static_cast<int64_t>(s) * p.dsub;
    const float* centroid = p.codebooks + (static_cast<int64_t>(s) * VECTRA_PQ_CENTROIDS + c) * p.dsub;
    p.tables[q * p.table_stride + static_cast<int64_t>(s) * VECTRA_PQ_CENTROIDS + c] = table_entry<0>(sub, centroid, p.dsub);
  }
}

// Sub-vectors of a known length up to 32: a workgroup of 256 lanes per
// (block of kTableQueries queries, sub-space), lane c holding centroid c of
// the sub-space in registers for every query of the block, the queries'
// sub-vectors staged in LDS.  Each centroid is read once per block instead
// of once per query, and the tables, written once, bypass the caches
// (blocks of 8 queries measured fastest: 4.5 us at 1,024 queries, against
// 4.7 with 16 and 5.3 with 4; cached stores 6.4 with 16).
constexpr int kTableQueries = 8;

template <int kDsub>
__global__ __launch_bounds__(VECTRA_PQ_CENTROIDS) void pq_table_sub_kernel(PqTable p) {
  static_assert(kDsub > 0 && kDsub <= 32, "sub-vectors held in registers");
  __shared__ float subs[kTableQueries][kDsub];
  const int s = static_cast<int>(blockIdx.y);
  const int c = static_cast<int>(threadIdx.x);
  const int64_t q0 = static_cast<int64_t>(blockIdx.x) * kTableQueries;
  const int nq = static_cast<int>(p.num_queries - q0 < kTableQueries ? p.num_queries - q0 : kTableQueries);
  for (int i = c; i < nq * kDsub; i += VECTRA_PQ_CENTROIDS)
    subs[i / kDsub][i % kDsub] = p.queries[(q0 + i / kDsub) * p.query_stride + static_cast<int64_t>(s) * kDsub + i % kDsub];
  float centroid[kDsub];
  const float* cp = p.codebooks + (static_cast<int64_t>(s) * VECTRA_PQ_CENTROIDS + c) * kDsub;
#pragma unroll
  for (int d = 0; d < kDsub; ++d) centroid[d] = cp[d];
  __syncthreads();
  for (int qq = 0; qq < nq; ++qq)
    __builtin_nontemporal_store(table_entry<kDsub>(subs[qq], centroid, kDsub),
                                &p.tables[(q0 + qq) * p.table_stride + static_cast<int64_t>(s) * VECTRA_PQ_CENTROIDS + c]);
}

struct PqAdc {
  const float* tables;
  const uint8_t* codes;
  const uint32_t* ids;
  float* out;
  int64_t table_stride, code_stride, out_stride;
  int64_t num_codes, num_cand;
  int32_t subspaces;
  int32_t words;    // codes may be read as 32-bit words (4-byte aligned base and stride)
  int32_t words16;  // table rows may be read as 16-byte words (16-byte aligned base and stride)
};

// PqAdcDistance for one code; `entry(s, c)` reads table[s * 256 + c].
template <typename Entry>
__device__ __forceinline__ float adc_sum(const uint8_t* code, int m, bool words, Entry entry) {
  float l0 = 0.f, l1 = 0.f, l2 = 0.f, l3 = 0.f;
  int s = 0;
  if (words) {
    for (; s + 4 <= m; s += 4) {
      const uint32_t w = *reinterpret_cast<const uint32_t*>(code + s);
      l0 = l0 + entry(s, w & 0xffu);
      l1 = l1 + entry(s + 1, (w >> 8) & 0xffu);
      l2 = l2 + entry(s + 2, (w >> 16) & 0xffu);
      l3 = l3 + entry(s + 3, w >> 24);
    }
  } else {
    for (; s + 4 <= m; s += 4) {
      l0 = l0 + entry(s, code[s]);
      l1 = l1 + entry(s + 1, code[s + 1]);
      l2 = l2 + entry(s + 2, code[s + 2]);
      l3 = l3 + entry(s + 3, code[s + 3]);
    }
  }
  float sum = (l0 + l1) + (l2 + l3);
  for (; s < m; ++s) sum = sum + entry(s, code[s]);
  return sum;
}

template <bool kLdsTable>
__global__ __launch_bounds__(kThreads) void pq_adc_kernel(PqAdc p) {
  extern __shared__ float table_lds[];  // subspaces * 256 floats when kLdsTable
  const int64_t q = blockIdx.y;
  const float* table = p.tables + q * p.table_stride;
  const int m = p.subspaces;
  if constexpr (kLdsTable) {
    for (int i = static_cast<int>(threadIdx.x); i < m * VECTRA_PQ_CENTROIDS; i += kThreads) table_lds[i] = table[i];
    __syncthreads();
  }
  for (int64_t cand = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x; cand < p.num_cand;
       cand += static_cast<int64_t>(gridDim.x) * kThreads) {
    int64_t index = cand;
    bool valid = true;
    if (p.ids != nullptr) {
      const uint32_t id = p.ids[cand];
      valid = static_cast<int64_t>(id) < p.num_codes;
      index = id;
    }
    float sum = NAN;
    if (valid) {
      const uint8_t* code = p.codes + index * p.code_stride;
      if constexpr (kLdsTable) {
        sum = adc_sum(code, m, p.words != 0,
                      [&](int s, uint32_t c) { return table_lds[s * VECTRA_PQ_CENTROIDS + static_cast<int>(c)]; });
      } else {
        sum = adc_sum(code, m, p.words != 0,
                      [&](int s, uint32_t c) { return table[s * VECTRA_PQ_CENTROIDS + static_cast<int>(c)]; });
      }
    }
    p.out[q * p.out_stride + cand] = sum;
  }
}

// The ADC scan for codes of at most 32 bytes laid out on 16-byte boundaries
// (base and stride): a code arrives in kChunks 16-byte loads, and the table
// sits in LDS.  The sums are adc_sum's, on the code's words.

template <int kChunks, typename Entry>
__device__ __forceinline__ float adc_sum_words(const uint4 (&chunk)[kChunks], int m, Entry entry) {
  constexpr int kWords = 4 * kChunks;
  uint32_t words[kWords];
#pragma unroll
  for (int c = 0; c < kChunks; ++c) {
    words[4 * c] = chunk[c].x;
    words[4 * c + 1] = chunk[c].y;
    words[4 * c + 2] = chunk[c].z;
    words[4 * c + 3] = chunk[c].w;
  }
  float l0 = 0.f, l1 = 0.f, l2 = 0.f, l3 = 0.f;
#pragma unroll
  for (int k = 0; k < kWords; ++k) {
    if (4 * k + 4 <= m) {
      const uint32_t w = words[k];
      l0 = l0 + entry(4 * k, w & 0xffu);
      l1 = l1 + entry(4 * k + 1, (w >> 8) & 0xffu);
      l2 = l2 + entry(4 * k + 2, (w >> 16) & 0xffu);
      l3 = l3 + entry(4 * k + 3, w >> 24);
    }
  }
  float sum = (l0 + l1) + (l2 + l3);
  const int full = m & ~3;
  uint32_t last = 0;
#pragma unroll
  for (int k = 0; k < kWords; ++k)
    if (k == full / 4) last = words[k];
#pragma unroll
  for (int r = 0; r < 3; ++r)
    if (full + r < m) sum = sum + entry(full + r, (last >> (8 * r)) & 0xffu);
  return sum;
}

// Workgroups of the 16-byte ADC scan: 512 threads, four per compute unit
// (kAdcBlocks over the 256 CUs of an MI355X), so the table is staged 1024
// times per launch instead of once per 256 codes.
constexpr int kAdcThreads = 512;
constexpr int64_t kAdcBlocks = 1024;

// Each lane sums one code per step and holds two steps' codes in two register
// sets: the next step's code is requested before the current one is summed.
// Every load is issued unconditionally (a candidate past the end re-reads the
// last one, an id past the codes reads code 0, and both are masked after),
// so the compiler can wait for exactly the older set with a counted
// s_waitcnt; loads behind a branch, or a copy of one set into the other,
// make it wait for every load in flight, the next step's included.  Codes are
// read once and the distances written once: both bypass the caches
// (non-temporal), and the table is staged with 16-byte loads where its rows
// allow.  kM is the sub-space count when known at compile time (the engine's
// 16: the lookups of a code are issued together), 0 for p.subspaces.  The
// launch requires num_codes >= 1.
template <int kChunks, int kM, bool kIds>
__global__ __launch_bounds__(kAdcThreads) void pq_adc_vec_kernel(PqAdc p) {
  extern __shared__ float table_lds[];  // subspaces * 256 floats
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  const int64_t q = blockIdx.y;
  const float* table = p.tables + q * p.table_stride;
  const int m = kM > 0 ? kM : p.subspaces;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kAdcThreads;
  const int64_t last = p.num_cand - 1;
  // Candidate `cand`'s code into `chunk`; `valid` says whether it exists.
  auto load = [&](int64_t cand, bool& valid, uint4 (&chunk)[kChunks]) {
    const int64_t c = cand < last ? cand : last;
    int64_t index = c;
    valid = cand <= last;
    if constexpr (kIds) {
      const uint32_t id = p.ids[c];
      valid = valid && static_cast<int64_t>(id) < p.num_codes;
      index = valid ? static_cast<int64_t>(id) : 0;
    }
#pragma unroll
    for (int k = 0; k < kChunks; ++k) {
      const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.codes + index * p.code_stride + 16 * k));
      chunk[k] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  };
  // The first code is requested before the table is staged.
  int64_t cand = static_cast<int64_t>(blockIdx.x) * kAdcThreads + threadIdx.x;
  bool valid_a, valid_b;
  uint4 chunk_a[kChunks], chunk_b[kChunks];
  load(cand, valid_a, chunk_a);
  if (p.words16 != 0) {
    const uint4* t4 = reinterpret_cast<const uint4*>(table);
    uint4* l4 = reinterpret_cast<uint4*>(table_lds);
    for (int i = static_cast<int>(threadIdx.x); i < m * VECTRA_PQ_CENTROIDS / 4; i += kAdcThreads) l4[i] = t4[i];
  } else {
    for (int i = static_cast<int>(threadIdx.x); i < m * VECTRA_PQ_CENTROIDS; i += kAdcThreads) table_lds[i] = table[i];
  }
  __syncthreads();
  auto entry = [&](int s, uint32_t c) { return table_lds[s * VECTRA_PQ_CENTROIDS + static_cast<int>(c)]; };
  auto emit = [&](int64_t at, bool valid, const uint4 (&chunk)[kChunks]) {
    const float d = valid ? adc_sum_words(chunk, m, entry) : NAN;
    if (at <= last) __builtin_nontemporal_store(d, &p.out[q * p.out_stride + at]);
  };
  if constexpr (kIds) {
    // A code's load waits for its id: the ids are requested a step ahead of
    // their codes, in two more registers, so that the wait for step t + 1's
    // id leaves step t's code in flight.  Issue order: id(t + 2), code(t + 1),
    // id(t + 3), code(t + 2), ...; each wait is for the older of two loads.
    uint32_t id_a = p.ids[cand + 2 * stride < last ? cand + 2 * stride : last];
    uint32_t id_b = p.ids[cand + stride < last ? cand + stride : last];
    auto code = [&](int64_t at, uint32_t id, bool& valid, uint4 (&chunk)[kChunks]) {
      valid = at <= last && static_cast<int64_t>(id) < p.num_codes;
      const int64_t index = valid ? static_cast<int64_t>(id) : 0;
#pragma unroll
      for (int k = 0; k < kChunks; ++k) {
        const u32x4 x =
            __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p.codes + index * p.code_stride + 16 * k));
        chunk[k] = make_uint4(x[0], x[1], x[2], x[3]);
      }
    };
    for (; cand <= last; cand += 2 * stride) {
      code(cand + stride, id_b, valid_b, chunk_b);
      const int64_t n3 = cand + 3 * stride;
      id_b = p.ids[n3 < last ? n3 : last];
      emit(cand, valid_a, chunk_a);
      code(cand + 2 * stride, id_a, valid_a, chunk_a);
      const int64_t n4 = cand + 4 * stride;
      id_a = p.ids[n4 < last ? n4 : last];
      emit(cand + stride, valid_b, chunk_b);
    }
  } else {
    for (; cand <= last; cand += 2 * stride) {
      load(cand + stride, valid_b, chunk_b);
      emit(cand, valid_a, chunk_a);
      load(cand + 2 * stride, valid_a, chunk_a);
      emit(cand + stride, valid_b, chunk_b);
    }
  }
}

unsigned blocks_for(int64_t items, int per_block, int64_t cap = kMaxBlocksX) {
  int64_t blocks = (items + per_block - 1) / per_block;
  if (blocks > cap) blocks = cap;
  return static_cast<unsigned>(blocks < 1 ? 1 : blocks);
}

int launched(hipError_t e) { return e == hipSuccess ? VECTRA_SCAN_OK : VECTRA_SCAN_LAUNCH_FAILED; }

template <int kMetric, bool kIds>
int launch_rows_ids(RowScan& p, hipStream_t stream) {
  void* args[] = {&p};
  // One pass of the grid covers every candidate: a wave's row loads are then
  // never queued behind its previous candidate's fold.
  const unsigned bx = blocks_for(p.num_cand, kGroupsPerBlock);
  if (p.num_queries == 1 || kMetric == VECTRA_SCAN_SQUARED_NORM) {
    return launched(hipLaunchKernel(reinterpret_cast<const void*>(&scan_rows_kernel<kMetric, 1, kIds>), dim3(bx, 1),
                                    dim3(kThreads), args, 0, stream));
  }
  const unsigned by = static_cast<unsigned>((p.num_queries + kQueryBlock - 1) / kQueryBlock);
  // Several queries over 128-dimensional rows: the queries held in registers
  // on a capped grid (4 queries over 4M rows: 534 -> 483 us; one query keeps
  // the one-pass grid, 314 us against 419 capped).
  if (p.dim == 128 && p.num_rows >= 1)
    return launched(hipLaunchKernel(reinterpret_cast<const void*>(&scan_rows_pipe_kernel<kMetric, kQueryBlock, kIds, 128>),
                                    dim3(blocks_for(p.num_cand, kGroupsPerBlock, kScanBlocks), by), dim3(kThreads), args,
                                    0, stream));
  return launched(hipLaunchKernel(reinterpret_cast<const void*>(&scan_rows_kernel<kMetric, kQueryBlock, kIds>),
                                  dim3(bx, by), dim3(kThreads), args, 0, stream));
}

template <int kMetric>
int launch_rows(RowScan& p, hipStream_t stream) {
  return p.ids != nullptr ? launch_rows_ids<kMetric, true>(p, stream) : launch_rows_ids<kMetric, false>(p, stream);
}


// ---------------------------------------------------------------- top k

// Exhaustive k-nearest search (ShardIndex::ExhaustiveSearch,
// shard_index.cc:236-264): one workgroup per query scans every candidate
// with the row scan's L2 arithmetic (the same operations in the same order,
// so the distances are bit-identical) and keeps the k nearest.  The order is
// CloserFirst's (search_scratch.h: distance ascending, ties by node id),
// which a 64-bit key turns into integer order: the distance's bits mapped so
// that unsigned order follows float order, above the node id.  The workgroup
// holds the k best keys and the candidates that beat the k-th since the last
// merge in LDS; when those could overflow the buffer, and at the end, the
// keys are sorted (bitonic) and the first k kept.
//
// Split form (few queries): a query's candidates are cut into `splits`
// contiguous ranges, one workgroup each; a workgroup writes the k best keys
// of its range to device memory and counts itself in the query's arrival
// counter, and the workgroup that arrives last gathers the splits * k keys
// (at most the LDS buffer), sorts them and writes the result.  The k nearest
// of the whole list are among the union of every range's k nearest, and
// keys are unique per (distance, node, position), so the result is the one
// workgroup form's, bit for bit.  The last workgroup puts the counter back to
// zero, so the counters are zero between calls.
struct TopK {
  const float* queries;
  const float* rows;
  const uint32_t* ids;
  float* distances;
  uint32_t* nodes;
  int64_t query_stride, row_stride, out_stride;
  int64_t num_rows, num_cand;
  int32_t dim, k;
  int32_t splits;     // workgroups per query (1: no split)
  int64_t split_len;  // candidates per split (the last one may have fewer)
  uint64_t* partial;  // [queries][splits][k] keys of each split's k best
  uint32_t* arrived;  // [queries] splits done; zero between calls
};

constexpr int kTopKKeys = 2048;        // LDS keys: the k best, then the new candidates
constexpr uint64_t kNoKey = ~uint64_t{0};  // an empty slot (above every real key)
// Workgroups of 4 waves when there are queries enough to fill the device
// with them; otherwise 16, so that one query's candidates are loaded 4
// times as wide and its sorts run on 4 times the threads.
constexpr int64_t kTopKWideBelow = 1024;  // queries

// Candidates ranked by (distance, node).  -0 ranks as +0 (CloserFirst
// compares values), and every NaN as one quiet NaN above +inf.
__device__ __forceinline__ uint64_t nearest_key(float d, uint32_t node) {
  uint32_t b = __float_as_uint(d);
  if (d != d) b = 0x7fc00000u;
  else if (b == 0x80000000u) b = 0u;
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return (static_cast<uint64_t>(ord) << 32) | node;
}
__device__ __forceinline__ float key_distance(uint64_t key) {
  const uint32_t ord = static_cast<uint32_t>(key >> 32);
  return __uint_as_float((ord & 0x80000000u) ? (ord & 0x7fffffffu) : ~ord);
}

// Wave-wide operations on one 64-bit key per lane, with no LDS buffer and
// no barrier: the partner exchanges are DPP moves and permlane swaps, which
// stay in the vector unit (an LDS permute, ds_bpermute, is a round trip
// through the LDS pipeline for every 32-bit half of every stage).
constexpr int kWaveLanes = 64;

// The value of lane `lane ^ kStride` (kStride a power of two below 64).
template <int kStride>
__device__ __forceinline__ uint32_t lane_xor(uint32_t x, int lane) {
  static_assert(kStride >= 1 && kStride <= 32 && (kStride & (kStride - 1)) == 0, "a lane bit");
  if constexpr (kStride == 1) {
    return __builtin_amdgcn_mov_dpp(x, 0xB1, 0xf, 0xf, false);  // quad_perm [1, 0, 3, 2]
  } else if constexpr (kStride == 2) {
    return __builtin_amdgcn_mov_dpp(x, 0x4E, 0xf, 0xf, false);  // quad_perm [2, 3, 0, 1]
  } else if constexpr (kStride == 4 || kStride == 8) {
    // Within a row of 16: row_shl:s gives lane i lane i + s, row_shr:s lane i - s.
    const uint32_t up = __builtin_amdgcn_mov_dpp(x, 0x100 + kStride, 0xf, 0xf, false);
    const uint32_t down = __builtin_amdgcn_mov_dpp(x, 0x110 + kStride, 0xf, 0xf, false);
    return (lane & kStride) ? down : up;
  } else if constexpr (kStride == 16) {
    // v_permlane16_swap(x, x): the first result holds rows 0, 0, 2, 2 of x,
    // the second rows 1, 1, 3, 3.
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane & 16) ? r[0] : r[1];
  } else {
    // v_permlane32_swap(x, x): the first result holds x's low half twice,
    // the second its high half twice.
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane & 32) ? r[0] : r[1];
  }
}
template <int kStride>
__device__ __forceinline__ uint64_t lane_xor(uint64_t key, int lane) {
  const uint32_t lo = lane_xor<kStride>(static_cast<uint32_t>(key), lane);
  const uint32_t hi = lane_xor<kStride>(static_cast<uint32_t>(key >> 32), lane);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// One compare-exchange stage of the bitonic network.
template <int kSize, int kStride>
__device__ __forceinline__ uint64_t bitonic_stage(uint64_t key, int lane) {
  const uint64_t other = lane_xor<kStride>(key, lane);
  const bool keep_min = ((lane & kStride) == 0) == ((lane & kSize) == 0);
  const uint64_t lo = key < other ? key : other, hi = key < other ? other : key;
  return keep_min ? lo : hi;
}
template <int kSize, int kStride>
__device__ __forceinline__ uint64_t bitonic_merge(uint64_t key, int lane) {
  key = bitonic_stage<kSize, kStride>(key, lane);
  if constexpr (kStride > 1) key = bitonic_merge<kSize, kStride / 2>(key, lane);
  return key;
}
template <int kSize>
__device__ __forceinline__ uint64_t bitonic_sort(uint64_t key, int lane) {
  if constexpr (kSize > 2) key = bitonic_sort<kSize / 2>(key, lane);
  return bitonic_merge<kSize, kSize / 2>(key, lane);
}

// Bitonic sort across the wave: lane i ends with the i-th smallest key (one
// query over 2,048 rows, the split form: 11.3 -> 9.5 us against the same
// network on LDS permutes; 1,024 queries: unchanged, 59.2-59.7 us both).
__device__ __forceinline__ uint64_t wave_sort(uint64_t key, int lane) {
  return bitonic_sort<kWaveLanes>(key, lane);
}

// The smallest key of the wave, in every lane (the split form's merge).
__device__ __forceinline__ uint64_t wave_min(uint64_t key) {
  const int lane = static_cast<int>(threadIdx.x) & (kWaveLanes - 1);
  auto step = [&](auto s_tag) {
    const uint64_t other = lane_xor<decltype(s_tag)::value>(key, lane);
    key = other < key ? other : key;
  };
  step(std::integral_constant<int, 32>{});
  step(std::integral_constant<int, 16>{});
  step(std::integral_constant<int, 8>{});
  step(std::integral_constant<int, 4>{});
  step(std::integral_constant<int, 2>{});
  step(std::integral_constant<int, 1>{});
  return key;
}

// kTopKThreads threads; a 16-lane group loads kTopKCands candidates at once,
// kSteps times per round of candidates between merge checks.  kDim is the
// row dimension when known at compile time (a multiple of 16 up to 128: the
// engine's 128), 0 for p.dim.
template <bool kIds, int kTopKThreads, int kTopKCands, int kSteps, int kDim = 0>
__global__ __launch_bounds__(kTopKThreads) void scan_top_k_kernel(TopK p) {
  static_assert(kDim % 16 == 0 && kDim <= 128, "whole 16-element steps, one unrolled pass");
  constexpr int kTopKGroups = kTopKThreads / kLanes;
  constexpr int kTopKRound = kTopKGroups * kTopKCands * kSteps;
  static_assert(kTopKKeys - VECTRA_SCAN_MAX_K >= kTopKRound, "room for a round of candidates");
  __shared__ uint64_t keys[kTopKKeys];
  __shared__ uint32_t fill;  // candidates in keys[k ..] since the last merge
  __shared__ uint32_t last;  // split form: this workgroup is the query's last
  const int tid = static_cast<int>(threadIdx.x);
  const int lane = tid & (kLanes - 1);
  const int group = tid / kLanes;
  const int64_t q = blockIdx.x / p.splits;
  const int split = static_cast<int>(blockIdx.x - q * p.splits);
  const int64_t cand_begin = split * p.split_len;
  const int64_t cand_end = cand_begin + p.split_len < p.num_cand ? cand_begin + p.split_len : p.num_cand;
  const int k = p.k;
  const int full = p.dim - p.dim % kLanes;
  const int tail = p.dim - full;
  const float* qlane = p.queries + q * p.query_stride + lane;

  for (int i = tid; i < kTopKKeys; i += kTopKThreads) keys[i] = kNoKey;
  if (tid == 0) fill = 0;
  __syncthreads();

  // Sorts keys[0 .. k + n) ascending (padded with empty slots to a power of
  // two), leaving the k best in keys[0 .. k); every thread takes part.
  auto merge = [&](int n) {
    int size = 2;
    while (size < k + n) size <<= 1;
    for (int i = k + n + tid; i < size; i += kTopKThreads) keys[i] = kNoKey;
    __syncthreads();
    for (int span = 2; span <= size; span <<= 1) {
      for (int stride = span >> 1; stride > 0; stride >>= 1) {
        for (int t = tid; t < size / 2; t += kTopKThreads) {
          const int i = 2 * t - (t & (stride - 1));
          const int j = i + stride;
          const uint64_t a = keys[i], b = keys[j];
          if ((a > b) == ((i & span) == 0)) {
            keys[i] = b;
            keys[j] = a;
          }
        }
        __syncthreads();
      }
    }
  };

  // The first selection of a workgroup whose rounds hold at most a wave's
  // worth of candidates: nothing has been selected yet, so keys[0 .. k) are
  // still empty (not merely short of k keys), and the n <= 64
  // candidates sit at keys[k ..]; one wave sorts them in its lanes (a
  // bitonic network over lane shuffles, where the LDS sort takes a barrier
  // per stage), and the sorted keys, empty slots included, fill keys[0 ..).
  auto first_select = [&](int n) {
    if (tid < kWaveLanes) {
      uint64_t key = tid < n ? keys[k + tid] : kNoKey;
      key = wave_sort(key, tid);
      if (tid < k) keys[tid] = key;
    }
    __syncthreads();
  };
  // Selections small enough for wave sorts, which take no barrier per stage
  // (the LDS sort takes one for each of its log2(size) (log2(size) + 1) / 2
  // stages, 45 for a round of 256 candidates):
  //  * k + n <= 64: one wave sorts the k kept keys (empty slots before the
  //    first selection) and the n candidates;
  //  * a first selection of at most one candidate per thread, with k at most
  //    64 / waves: each wave sorts 64 of the candidates and keeps its k best,
  //    and one wave sorts the waves' k-best lists.
  // Either leaves the k smallest keys of the same set in keys[0 .. k), in
  // order, as the LDS sort does.
  constexpr int kTopKWaves = kTopKThreads / kWaveLanes;
  auto wave_select = [&](bool first, int n) {
    if (k + n <= kWaveLanes) {
      if (tid < kWaveLanes) {
        uint64_t key = tid < k + n ? keys[tid] : kNoKey;
        key = wave_sort(key, tid);
        if (tid < k) keys[tid] = key;
      }
      __syncthreads();
      return true;
    }
    if (first && n <= kTopKThreads && kTopKWaves * k <= kWaveLanes) {
      const int lane = tid & (kWaveLanes - 1);
      uint64_t key = tid < n ? keys[k + tid] : kNoKey;
      key = wave_sort(key, lane);
      __syncthreads();  // every candidate read before the k-best lists overwrite them
      if (lane < k) keys[(tid / kWaveLanes) * k + lane] = key;
      __syncthreads();
      if (tid < kWaveLanes) {
        uint64_t best = tid < kTopKWaves * k ? keys[tid] : kNoKey;
        best = wave_sort(best, tid);
        if (tid < k) keys[tid] = best;
      }
      __syncthreads();
      return true;
    }
    return false;
  };
  auto select = [&](bool first, int n) {
    if constexpr (kTopKRound <= kWaveLanes) {
      if (first && n <= kWaveLanes) {
        first_select(n);
        return;
      }
    }
    // (Not in the split form's kernel, whose rounds fit one wave: there the
    // extra code measured 1.4 us slower on a lone query, 12.7 against 11.3.)
    if constexpr (kTopKRound > kWaveLanes) {
      if (wave_select(first, n)) return;
    }
    merge(n);
  };

  uint64_t worst = kNoKey;  // the k-th best key so far; empty while fewer than k
  // Its distance (NaN while empty): a candidate whose distance is above it
  // cannot beat it, and its key is not formed.  NaN distances, and every
  // candidate while `worst` is empty, fail `sum > worst_d` and go on to the
  // key comparison, so the filter drops only candidates the keys would.
  float worst_d = key_distance(kNoKey);
  // Whether keys[0 .. k) hold a selection.  An overflow merge can keep fewer
  // than k keys (ids past the rows are skipped), which leaves `worst` empty
  // with keys in the buffer, so `worst` cannot tell an empty buffer.
  bool selected = false;
  // End of a round: merge once k candidates are in hand (the threshold then
  // discards most of the rest), and whenever the next round might not fit.
  auto round_end = [&]() {
    __syncthreads();
    const int n = static_cast<int>(fill);
    if ((worst == kNoKey && n >= k) || n > kTopKKeys - k - kTopKRound) {
      select(!selected, n);
      selected = true;
      if (tid == 0) fill = 0;
      worst = keys[k - 1];
      worst_d = key_distance(worst);
      __syncthreads();
    }
  };
  if constexpr (kDim > 0) {
    // Steps of kTopKCands candidates per group, in two register sets: the
    // next step's rows are requested before the current step is summed, and
    // the next round's first step before a round's merge.  Every load is
    // issued (a candidate past the range re-reads the range's first, an id
    // past the rows reads row 0, and both are masked), so the compiler waits
    // for exactly the older set.  The query's kDim / 16 elements of this
    // lane stay in registers.  Each candidate's operations are the row
    // scan's, in its order.
    constexpr int kPer = kDim / kLanes;
    struct Step {
      float v[kTopKCands][kPer];
      uint32_t row[kTopKCands];
      bool ok[kTopKCands];
    };
    float qv[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) qv[u] = qlane[kLanes * u];
    const int64_t len = cand_end - cand_begin;
    const int64_t steps = p.num_rows > 0 && len > 0 ? (len + kTopKRound - 1) / kTopKRound * kSteps : 0;
    auto load = [&](int64_t t, Step& st) {
      const int64_t first = cand_begin + (t / kSteps) * kTopKRound + (t % kSteps) * (kTopKCands * kTopKGroups);
#pragma unroll
      for (int c = 0; c < kTopKCands; ++c) {
        const int64_t cand = first + c * kTopKGroups + group;
        bool ok = cand < cand_end;
        int64_t row = ok ? cand : cand_begin;
        if constexpr (kIds) {
          const uint32_t id = p.ids[row];
          ok = ok && static_cast<int64_t>(id) < p.num_rows;
          row = ok ? id : 0;
        }
        st.ok[c] = ok;
        st.row[c] = static_cast<uint32_t>(row);
        const float* r = p.rows + row * p.row_stride + lane;
#pragma unroll
        for (int u = 0; u < kPer; ++u) st.v[c][u] = r[kLanes * u];
      }
    };
    auto consume = [&](const Step& st) {
#pragma unroll
      for (int c = 0; c < kTopKCands; ++c) {
        float sum = 0.f;
#pragma unroll
        for (int u = 0; u < kPer; ++u) sum = sum + term<VECTRA_SCAN_L2_SQUARED>(qv[u], st.v[c][u]);
        sum = reduce_lanes(sum);
        if (st.ok[c] && lane == 0 && !(sum > worst_d)) {
          const uint64_t key = nearest_key(sum, st.row[c]);
          if (key < worst) keys[k + atomicAdd(&fill, 1u)] = key;
        }
      }
    };
    Step a, b;
    if (steps > 0) load(0, a);
    for (int64_t t = 0; t < steps; t += 2) {
      load(t + 1 < steps ? t + 1 : t, b);
      consume(a);
      if ((t + 1) % kSteps == 0) round_end();
      load(t + 2 < steps ? t + 2 : t, a);
      if (t + 1 < steps) {
        consume(b);
        if ((t + 2) % kSteps == 0) round_end();
      }
    }
  } else {
    for (int64_t base = cand_begin; base < cand_end; base += kTopKRound) {
      // A round: kSteps steps of kTopKCands candidates per 16-lane group, a
      // step's loads issued before any of its sums (each candidate's own
      // operations keep the row scan's order).
      for (int s = 0; s < kSteps; ++s) {
        bool valid[kTopKCands];
        const float* rlane[kTopKCands];
        int64_t row[kTopKCands];
#pragma unroll
        for (int c = 0; c < kTopKCands; ++c) {
          const int64_t cand = base + static_cast<int64_t>(s * kTopKCands + c) * kTopKGroups + group;
          valid[c] = cand < cand_end;
          row[c] = valid[c] ? cand : 0;
          if constexpr (kIds) {
            const uint32_t id = valid[c] ? p.ids[cand] : 0u;
            valid[c] = valid[c] && static_cast<int64_t>(id) < p.num_rows;
            row[c] = valid[c] ? id : 0;
          }
          rlane[c] = p.rows + row[c] * p.row_stride + lane;
        }
        float acc[kTopKCands];
#pragma unroll
        for (int c = 0; c < kTopKCands; ++c) acc[c] = 0.f;
        int i = 0;
        for (; i + kLanes * kUnroll <= full; i += kLanes * kUnroll) {
          float rv[kTopKCands][kUnroll], qv[kUnroll];
#pragma unroll
          for (int c = 0; c < kTopKCands; ++c)
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) rv[c][u] = valid[c] ? rlane[c][i + kLanes * u] : 0.f;
#pragma unroll
          for (int u = 0; u < kUnroll; ++u) qv[u] = qlane[i + kLanes * u];
#pragma unroll
          for (int c = 0; c < kTopKCands; ++c)
#pragma unroll
            for (int u = 0; u < kUnroll; ++u) acc[c] = acc[c] + term<VECTRA_SCAN_L2_SQUARED>(qv[u], rv[c][u]);
        }
        for (; i < full; i += kLanes) {
          const float qi = qlane[i];
#pragma unroll
          for (int c = 0; c < kTopKCands; ++c)
            acc[c] = acc[c] + term<VECTRA_SCAN_L2_SQUARED>(qi, valid[c] ? rlane[c][i] : 0.f);
        }
#pragma unroll
        for (int c = 0; c < kTopKCands; ++c) {
          float sum = reduce_lanes(acc[c]);
          float t = 0.f;
          if (valid[c] && lane < tail) t = term<VECTRA_SCAN_L2_SQUARED>(qlane[full], rlane[c][full]);
          for (int e = 0; e < tail; ++e) sum = sum + __shfl(t, e, kLanes);
          if (valid[c] && lane == 0 && !(sum > worst_d)) {
            const uint64_t key = nearest_key(sum, static_cast<uint32_t>(row[c]));
            if (key < worst) keys[k + atomicAdd(&fill, 1u)] = key;
          }
        }
      }
      round_end();
    }
  }
  const int n = static_cast<int>(fill);
  if (n > 0) select(!selected, n);
  if (p.splits > 1) {
    // This range's k best to device memory, visible device-wide before the
    // arrival is counted: the barrier completes every wave's stores to this
    // XCD's L2, and one release at agent scope writes them back (the
    // workgroup that reads them may sit on another XCD, behind another L2).
    uint64_t* part = p.partial + (q * p.splits + split) * k;
    for (int r = tid; r < k; r += kTopKThreads) part[r] = keys[r];
    __syncthreads();
    if (tid == 0) {
      __threadfence();
      last = atomicAdd(&p.arrived[q], 1u) == static_cast<uint32_t>(p.splits - 1);
    }
    __syncthreads();
    if (!last) return;
    __threadfence();  // acquire: the other ranges' keys
    const int all = p.splits * k;
    const uint64_t* parts = p.partial + q * p.splits * k;
    for (int i = tid; i < all; i += kTopKThreads) keys[i] = parts[i];
    if (k <= kWaveLanes && p.splits <= kWaveLanes) {
      // The ranges' lists are sorted: one wave merges them, lane i holding
      // the head of range i; k times the smallest head is taken (the lowest
      // lane on a tie) and its range advances.
      __syncthreads();
      if (tid < kWaveLanes) {
        int pos = 0;
        uint64_t head = tid < p.splits ? keys[tid * k] : kNoKey;
        uint64_t mine = kNoKey;
        for (int r = 0; r < k; ++r) {
          const uint64_t m = wave_min(head);
          const int win = __ffsll(static_cast<unsigned long long>(__ballot(head == m))) - 1;
          if (tid == r) mine = m;
          if (tid == win) {
            ++pos;
            head = tid < p.splits && pos < k ? keys[tid * k + pos] : kNoKey;
          }
        }
        if (tid < k) keys[tid] = mine;
      }
      __syncthreads();
    } else {
      merge(all - k);
    }
    if (tid == 0) p.arrived[q] = 0u;
  }
  for (int r = tid; r < k; r += kTopKThreads) {
    const uint64_t key = keys[r];
    const int64_t off = q * p.out_stride + r;
    p.distances[off] = key == kNoKey ? INFINITY : key_distance(key);
    p.nodes[off] = key == kNoKey ? VECTRA_SCAN_NO_NODE : static_cast<uint32_t>(key);
  }
}

}  // namespace
}  // namespace vectra_scan

using namespace vectra_scan;

extern "C" int vectra_scan_rows(const vectra_scan_args* a, hipStream_t stream) {
  if (a == nullptr) return VECTRA_SCAN_INVALID_ARGUMENT;
  const bool norm = a->metric == VECTRA_SCAN_SQUARED_NORM;
  if (a->metric < VECTRA_SCAN_L2_SQUARED || a->metric > VECTRA_SCAN_SQUARED_NORM) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->dimension < 0 || a->num_queries < 0 || a->num_rows < 0 || (a->ids != nullptr && a->num_ids < 0))
    return VECTRA_SCAN_INVALID_ARGUMENT;
  if (norm && a->num_queries != 1) return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t cand = a->ids != nullptr ? a->num_ids : a->num_rows;
  if (a->row_stride < a->dimension || a->out_stride < cand) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (!norm && a->query_stride < a->dimension) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->num_queries == 0 || cand == 0) return VECTRA_SCAN_OK;
  // Vectors of zero floats are never read (their distances are 0).
  const bool reads = a->dimension > 0;
  if (a->out == nullptr || (reads && a->num_rows > 0 && a->rows == nullptr) || (reads && !norm && a->queries == nullptr))
    return VECTRA_SCAN_INVALID_ARGUMENT;
  if ((a->num_queries + kQueryBlock - 1) / kQueryBlock > kMaxBlocksY) return VECTRA_SCAN_TOO_LARGE;
  // Element offsets stay below 2^62.
  const int64_t lim = int64_t{1} << 62;
  if ((a->num_rows > 0 && a->row_stride > lim / a->num_rows) || a->out_stride > lim / a->num_queries ||
      (!norm && a->query_stride > lim / a->num_queries))
    return VECTRA_SCAN_TOO_LARGE;
  RowScan p;
  p.queries = a->queries;
  p.rows = a->rows;
  p.ids = a->ids;
  p.out = a->out;
  p.query_stride = a->query_stride;
  p.row_stride = a->row_stride;
  p.out_stride = a->out_stride;
  p.num_rows = a->num_rows;
  p.num_cand = cand;
  p.dim = a->dimension;
  p.num_queries = static_cast<int32_t>(a->num_queries);
  switch (a->metric) {
    case VECTRA_SCAN_L2_SQUARED: return launch_rows<VECTRA_SCAN_L2_SQUARED>(p, stream);
    case VECTRA_SCAN_INNER_PRODUCT: return launch_rows<VECTRA_SCAN_INNER_PRODUCT>(p, stream);
    default: return launch_rows<VECTRA_SCAN_SQUARED_NORM>(p, stream);
  }
}

extern "C" int vectra_pq_distance_tables(const vectra_pq_table_args* a, hipStream_t stream) {
  if (a == nullptr) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->subspaces <= 0 || a->dimension <= 0 || a->dimension % a->subspaces != 0 || a->num_queries < 0)
    return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t entries = static_cast<int64_t>(a->subspaces) * VECTRA_PQ_CENTROIDS;
  if (a->query_stride < a->dimension || a->table_stride < entries) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->num_queries == 0) return VECTRA_SCAN_OK;
  if (a->queries == nullptr || a->codebooks == nullptr || a->tables == nullptr) return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t lim = int64_t{1} << 62;
  if (a->table_stride > lim / a->num_queries || a->query_stride > lim / a->num_queries) return VECTRA_SCAN_TOO_LARGE;
  if (a->num_queries > (int64_t{1} << 31) / entries - 1) return VECTRA_SCAN_TOO_LARGE;  // entries in total < 2^31
  PqTable p;
  p.queries = a->queries;
  p.codebooks = a->codebooks;
  p.tables = a->tables;
  p.query_stride = a->query_stride;
  p.table_stride = a->table_stride;
  p.total = a->num_queries * entries;
  p.subspaces = a->subspaces;
  p.dsub = a->dimension / a->subspaces;
  p.num_queries = static_cast<int32_t>(a->num_queries);
  void* args[] = {&p};
  const void* sub_kernel = p.dsub == 8    ? reinterpret_cast<const void*>(&pq_table_sub_kernel<8>)
                           : p.dsub == 4  ? reinterpret_cast<const void*>(&pq_table_sub_kernel<4>)
                           : p.dsub == 16 ? reinterpret_cast<const void*>(&pq_table_sub_kernel<16>)
                           : p.dsub == 32 ? reinterpret_cast<const void*>(&pq_table_sub_kernel<32>)
                                          : nullptr;
  if (sub_kernel != nullptr && p.subspaces <= kMaxBlocksY) {
    const dim3 grid(static_cast<unsigned>((a->num_queries + kTableQueries - 1) / kTableQueries),
                    static_cast<unsigned>(p.subspaces));
    return launched(hipLaunchKernel(sub_kernel, grid, dim3(VECTRA_PQ_CENTROIDS), args, 0, stream));
  }
  return launched(hipLaunchKernel(reinterpret_cast<const void*>(&pq_table_kernel), dim3(blocks_for(p.total, kThreads)),
                                  dim3(kThreads), args, 0, stream));
}

extern "C" int vectra_scan_pq_adc(const vectra_pq_adc_args* a, hipStream_t stream) {
  if (a == nullptr) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->subspaces < 1 || a->subspaces > VECTRA_PQ_CENTROIDS || a->num_queries < 0 || a->num_codes < 0 ||
      (a->ids != nullptr && a->num_ids < 0))
    return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t cand = a->ids != nullptr ? a->num_ids : a->num_codes;
  const int64_t entries = static_cast<int64_t>(a->subspaces) * VECTRA_PQ_CENTROIDS;
  if (a->table_stride < entries || a->code_stride < a->subspaces || a->out_stride < cand)
    return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->num_queries == 0 || cand == 0) return VECTRA_SCAN_OK;
  if (a->tables == nullptr || a->out == nullptr || (a->num_codes > 0 && a->codes == nullptr))
    return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->num_queries > kMaxBlocksY) return VECTRA_SCAN_TOO_LARGE;
  const int64_t lim = int64_t{1} << 62;
  if ((a->num_codes > 0 && a->code_stride > lim / a->num_codes) || a->out_stride > lim / a->num_queries ||
      a->table_stride > lim / a->num_queries)
    return VECTRA_SCAN_TOO_LARGE;
  PqAdc p;
  p.tables = a->tables;
  p.codes = a->codes;
  p.ids = a->ids;
  p.out = a->out;
  p.table_stride = a->table_stride;
  p.code_stride = a->code_stride;
  p.out_stride = a->out_stride;
  p.num_codes = a->num_codes;
  p.num_cand = cand;
  p.subspaces = a->subspaces;
  p.words = (a->code_stride % 4 == 0 && reinterpret_cast<uintptr_t>(a->codes) % 4 == 0) ? 1 : 0;
  p.words16 = (a->table_stride % 4 == 0 && reinterpret_cast<uintptr_t>(a->tables) % 16 == 0) ? 1 : 0;
  void* args[] = {&p};
  const dim3 grid(blocks_for(cand, kThreads, kScanBlocks), static_cast<unsigned>(a->num_queries));
  const bool vec16 = a->code_stride % 16 == 0 && reinterpret_cast<uintptr_t>(a->codes) % 16 == 0;
  if (vec16 && a->subspaces <= 32 && a->num_codes > 0) {
    const size_t lds = static_cast<size_t>(entries) * sizeof(float);
    const bool ids = a->ids != nullptr;
    const void* kernel =
        a->subspaces == 16 ? (ids ? reinterpret_cast<const void*>(&pq_adc_vec_kernel<1, 16, true>)
                                  : reinterpret_cast<const void*>(&pq_adc_vec_kernel<1, 16, false>))
        : a->subspaces < 16 ? (ids ? reinterpret_cast<const void*>(&pq_adc_vec_kernel<1, 0, true>)
                                   : reinterpret_cast<const void*>(&pq_adc_vec_kernel<1, 0, false>))
                            : (ids ? reinterpret_cast<const void*>(&pq_adc_vec_kernel<2, 0, true>)
                                   : reinterpret_cast<const void*>(&pq_adc_vec_kernel<2, 0, false>));
    const dim3 vgrid(blocks_for(cand, kAdcThreads, kAdcBlocks), static_cast<unsigned>(a->num_queries));
    return launched(hipLaunchKernel(kernel, vgrid, dim3(kAdcThreads), args, lds, stream));
  }
  if (a->subspaces <= kMaxLdsTableSubspaces) {
    const size_t lds = static_cast<size_t>(entries) * sizeof(float);
    return launched(hipLaunchKernel(reinterpret_cast<const void*>(&pq_adc_kernel<true>), grid, dim3(kThreads), args,
                                    lds, stream));
  }
  return launched(
      hipLaunchKernel(reinterpret_cast<const void*>(&pq_adc_kernel<false>), grid, dim3(kThreads), args, 0, stream));
}

// The scratch of vectra_scan_top_k_no_alloc: room for the largest workspace
// of the split form (fewer than kSplitBelow queries of at most kTopKKeys
// keys each, after the counter block), one copy per GPU for the life of the
// process.  Zero when the library is loaded; every call leaves its counters
// zero again.
constexpr int64_t kNoAllocScratchBytes = 256 + 64 * 2048 * 8;
static __device__ __align__(256) uint8_t scratch[kNoAllocScratchBytes];

namespace {

// Split form: below kSplitBelow queries, a query's candidates are cut into
// ranges of at least kSplitCands (one step of the 4-wave kernel) over at
// most kSplitMax workgroups, and splits * k keys must fit the LDS buffer of
// the workgroup that merges them.
constexpr int64_t kSplitBelow = 64;
constexpr int64_t kSplitCands = 64;
constexpr int64_t kSplitMax = 64;
constexpr int64_t kCounterBytes = 256;  // the arrival counters' block (kSplitBelow of them)
static_assert(kSplitBelow * 4 <= kCounterBytes, "counters of every query of the split form");
static_assert(kNoAllocScratchBytes == kCounterBytes + kSplitBelow * kTopKKeys * 8, "the scratch's size");

// Validates the arguments and fills the kernel parameters (splits = 1).
int top_k_params(const vectra_scan_top_k_args* a, TopK& p) {
  if (a == nullptr) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->dimension < 0 || a->num_queries < 0 || a->num_rows < 0 || (a->ids != nullptr && a->num_ids < 0))
    return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->k < 1 || a->k > VECTRA_SCAN_MAX_K) return VECTRA_SCAN_INVALID_ARGUMENT;
  if (a->row_stride < a->dimension || a->query_stride < a->dimension || a->out_stride < a->k)
    return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t cand = a->ids != nullptr ? a->num_ids : a->num_rows;
  if (a->num_queries > 0) {
    const bool reads = a->dimension > 0 && cand > 0;
    if (a->distances == nullptr || a->nodes == nullptr || (reads && (a->queries == nullptr || a->rows == nullptr)))
      return VECTRA_SCAN_INVALID_ARGUMENT;
    // Node ids are 32-bit, below VECTRA_SCAN_NO_NODE; one workgroup per query.
    if (a->num_rows > int64_t{VECTRA_SCAN_NO_NODE} || a->num_queries > 0x7fffffffLL) return VECTRA_SCAN_TOO_LARGE;
    const int64_t lim = int64_t{1} << 62;
    if ((a->num_rows > 0 && a->row_stride > lim / a->num_rows) || a->out_stride > lim / a->num_queries ||
        a->query_stride > lim / a->num_queries)
      return VECTRA_SCAN_TOO_LARGE;
  }
  p.queries = a->queries;
  p.rows = a->rows;
  p.ids = a->ids;
  p.distances = a->distances;
  p.nodes = a->nodes;
  p.query_stride = a->query_stride;
  p.row_stride = a->row_stride;
  p.out_stride = a->out_stride;
  p.num_rows = a->num_rows;
  p.num_cand = cand;
  p.dim = a->dimension;
  p.k = a->k;
  p.splits = 1;
  p.split_len = cand;
  p.partial = nullptr;
  p.arrived = nullptr;
  return VECTRA_SCAN_OK;
}

// Workgroups per query of the split form for valid parameters (1: none).
int64_t top_k_splits(int64_t queries, const TopK& p) {
  if (queries < 1 || queries >= kSplitBelow) return 1;
  int64_t kp = 1;
  while (kp < p.k) kp <<= 1;
  int64_t s = kTopKKeys / kp;
  if (s > kSplitMax) s = kSplitMax;
  const int64_t by_cands = (p.num_cand + kSplitCands - 1) / kSplitCands;
  if (s > by_cands) s = by_cands;
  return s >= 2 ? s : 1;
}

// Workspace bytes of the split form: the counter block, then the keys.
int64_t top_k_workspace(int64_t queries, int64_t splits, int k) {
  return splits > 1 ? kCounterBytes + queries * splits * k * int64_t{8} : 0;
}

// The kernel of a launch form, for ids or none.
template <int kThreadsT, int kCands, int kSteps, int kDim>
const void* top_k_kernel(bool ids) {
  return ids ? reinterpret_cast<const void*>(&scan_top_k_kernel<true, kThreadsT, kCands, kSteps, kDim>)
             : reinterpret_cast<const void*>(&scan_top_k_kernel<false, kThreadsT, kCands, kSteps, kDim>);
}

// The engine's 128 dimensions take the pipelined kernels.  (Six candidates
// per group in the wide form's generic kernel; four in its pipelined one,
// whose two register sets hold six only with spills.)
int launch_top_k(int64_t queries, TopK& p, hipStream_t stream) {
  void* args[] = {&p};
  const bool ids = p.ids != nullptr;
  const bool d128 = p.dim == 128;
  if (p.splits > 1)
    return launched(hipLaunchKernel(d128 ? top_k_kernel<256, 4, 1, 128>(ids) : top_k_kernel<256, 4, 1, 0>(ids),
                                    dim3(static_cast<unsigned>(queries * p.splits)), dim3(256), args, 0, stream));
  const bool wide = queries < kTopKWideBelow;
  const void* kernel = wide ? (d128 ? top_k_kernel<1024, 4, 1, 128>(ids) : top_k_kernel<1024, 6, 1, 0>(ids))
                            : (d128 ? top_k_kernel<256, 4, 4, 128>(ids) : top_k_kernel<256, 4, 4, 0>(ids));
  return launched(hipLaunchKernel(kernel, dim3(static_cast<unsigned>(queries)), dim3(wide ? 1024 : 256), args, 0,
                                  stream));
}

// Points the split form at a workspace: counters first, keys after.
void use_workspace(TopK& p, int64_t splits, void* base) {
  p.splits = static_cast<int32_t>(splits);
  p.split_len = (p.num_cand + splits - 1) / splits;
  p.arrived = static_cast<uint32_t*>(base);
  p.partial = reinterpret_cast<uint64_t*>(static_cast<char*>(base) + kCounterBytes);
}

// Device address of `scratch` on each device, resolved on the entry point's
// first call there (the array's host-side name is not a device address).
constexpr int kMaxDevices = 64;
std::atomic<void*> scratch_ptr[kMaxDevices];

int scratch_address(void** out) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return VECTRA_SCAN_LAUNCH_FAILED;
  void* ptr = scratch_ptr[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || ptr == nullptr)
      return VECTRA_SCAN_LAUNCH_FAILED;
    scratch_ptr[dev].store(ptr, std::memory_order_release);
  }
  *out = ptr;
  return VECTRA_SCAN_OK;
}

}  // namespace

extern "C" int vectra_scan_top_k(const vectra_scan_top_k_args* a, hipStream_t stream) {
  TopK p;
  const int st = top_k_params(a, p);
  if (st != VECTRA_SCAN_OK || a->num_queries == 0) return st;
  return launch_top_k(a->num_queries, p, stream);
}

extern "C" int64_t vectra_scan_top_k_workspace_bytes(const vectra_scan_top_k_args* a) {
  TopK p;
  if (top_k_params(a, p) != VECTRA_SCAN_OK) return 0;
  return top_k_workspace(a->num_queries, top_k_splits(a->num_queries, p), p.k);
}

extern "C" int vectra_scan_top_k_ws(const vectra_scan_top_k_args* a, void* workspace, int64_t workspace_bytes,
                                    hipStream_t stream) {
  TopK p;
  const int st = top_k_params(a, p);
  if (st != VECTRA_SCAN_OK || a->num_queries == 0) return st;
  if (workspace != nullptr && (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
    return VECTRA_SCAN_INVALID_ARGUMENT;
  const int64_t splits = top_k_splits(a->num_queries, p);
  if (splits > 1 && workspace != nullptr && workspace_bytes >= top_k_workspace(a->num_queries, splits, p.k))
    use_workspace(p, splits, workspace);
  return launch_top_k(a->num_queries, p, stream);
}

extern "C" int vectra_scan_top_k_no_alloc(const vectra_scan_top_k_args* a, hipStream_t stream) {
  TopK p;
  const int st = top_k_params(a, p);
  if (st != VECTRA_SCAN_OK || a->num_queries == 0) return st;
  const int64_t splits = top_k_splits(a->num_queries, p);
  if (splits > 1) {
    if (top_k_workspace(a->num_queries, splits, p.k) > kNoAllocScratchBytes) return VECTRA_SCAN_TOO_LARGE;
    void* base = nullptr;
    const int sa = scratch_address(&base);
    if (sa != VECTRA_SCAN_OK) return sa;
    use_workspace(p, splits, base);
  }
  return launch_top_k(a->num_queries, p, stream);
}

extern "C" const char* vectra_scan_status_string(int status) {
  switch (status) {
    case VECTRA_SCAN_OK: return "ok";
    case VECTRA_SCAN_INVALID_ARGUMENT: return "invalid argument";
    case VECTRA_SCAN_TOO_LARGE: return "problem too large for the scan kernels";
    case VECTRA_SCAN_LAUNCH_FAILED: return "kernel launch failed";
    default: return "unknown status";
  }
}

extern "C" int vectra_scan_abi_version(void) { return VECTRA_SCAN_ABI_VERSION; }
