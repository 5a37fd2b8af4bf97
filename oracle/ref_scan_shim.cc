// C entry points over the reference engine's distance kernels, so the tests
// can call them through ctypes.  Compiled by oracle/Makefile together with
// the reference's own sources (engine/src/index/simd_distance.cc and
// pq_codec.cc, read in place under /root/reference) into
// oracle/_ref/libref_scan.so.  Test infrastructure only: the product never
// loads it.
#include <algorithm>
#include <cstdint>
#include <optional>
#include <string>
#include <vector>

#include "vectra/index/pq_codec.h"
#include "vectra/index/search_scratch.h"
#include "vectra/index/simd_distance.h"

namespace vi = vectra::index;

extern "C" {

// metric 0: L2SquaredDistance; 1: InnerProduct; 2: SquaredNorm of each row.
// out[i] for rows i = 0 .. n - 1 laid out `stride` floats apart.
void ref_scan_rows(int metric, const float* query, const float* rows, int64_t n, int64_t stride, int dim,
                   float* out) {
  for (int64_t i = 0; i < n; ++i) {
    const float* row = rows + i * stride;
    out[i] = metric == 0   ? vi::L2SquaredDistance(query, row, dim)
             : metric == 1 ? vi::InnerProduct(query, row, dim)
                           : vi::SquaredNorm(row, dim);
  }
}

// The double-precision references of the SIMD parity tests.
double ref_l2_squared_fp64(const float* a, const float* b, int dim) {
  return vi::L2SquaredDistanceReference(a, b, dim);
}
double ref_inner_product_fp64(const float* a, const float* b, int dim) {
  return vi::InnerProductReference(a, b, dim);
}

// PqAdcDistance for codes i = 0 .. n - 1 laid out `stride` bytes apart.
void ref_pq_adc_rows(const float* table, const uint8_t* codes, int64_t n, int64_t stride, int subspaces,
                     float* out) {
  for (int64_t i = 0; i < n; ++i) out[i] = vi::PqAdcDistance(table, codes + i * stride, subspaces);
}

// ProductQuantizer::FromCodebooks + ComputeDistanceTable; -1 when the
// reference rejects the geometry.
int ref_pq_distance_table(int dim, int subspaces, const float* codebooks, const float* query, float* table) {
  std::string error;
  std::optional<vi::ProductQuantizer> pq = vi::ProductQuantizer::FromCodebooks(
      dim, subspaces, std::vector<float>(codebooks, codebooks + static_cast<size_t>(dim) * vi::kPqCentroids),
      &error);
  if (!pq.has_value()) return -1;
  pq->ComputeDistanceTable(query, table);
  return 0;
}

// The k nearest of candidates (distance[i], node[i]) under the reference's
// own comparator, CloserFirst (search_scratch.h: distance ascending, ties by
// node id), the order ExhaustiveSearch returns (shard_index.cc:264).  Writes
// min(k, n) results and returns that count.  Finite distances only: the
// comparator is not a strict weak order over NaN.
int64_t ref_nearest(const float* distance, const uint32_t* node, int64_t n, int64_t k, float* out_distance,
                    uint32_t* out_node) {
  std::vector<vi::Neighbor> all(static_cast<size_t>(n));
  for (int64_t i = 0; i < n; ++i) all[static_cast<size_t>(i)] = {distance[i], node[i]};
  const int64_t m = std::min(k, n);
  std::partial_sort(all.begin(), all.begin() + m, all.end(), vi::CloserFirst());
  for (int64_t i = 0; i < m; ++i) {
    out_distance[i] = all[static_cast<size_t>(i)].distance;
    out_node[i] = all[static_cast<size_t>(i)].node;
  }
  return m;
}

}  // extern "C"
