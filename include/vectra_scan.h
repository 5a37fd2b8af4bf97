/*
 * vectra_scan.h -- C ABI of the MI355X (gfx950) distance scans,
 * libvectra_scan.so.
 *
 * The reference engine computes the distances of its vector search one pair
 * at a time on the CPU (engine/src/index/simd_distance.cc): the exhaustive
 * scan of a shard's rows (ShardIndex::ExhaustiveSearch,
 * engine/src/index/shard_index.cc:236-264), the exact re-rank of PQ-ranked
 * candidates (HnswSearcher, engine/src/index/hnsw_searcher.cc:145-158), the
 * product-quantisation distance table (ProductQuantizer::
 * ComputeDistanceTable, engine/src/index/pq_codec.cc:208-217) and the ADC
 * distance of every code (PqAdcDistance, include/vectra/index/
 * hnsw_searcher.h:74; engine/tests/tools/index_study.cc:81-83).  Each entry
 * point below computes a whole batch of those calls in one launch, with the
 * reference's order of floating-point operations, so every output is
 * bit-identical to the reference function's return value for the same
 * inputs (the reference built as ISO C++20, where no multiply-add is
 * contracted).
 *
 * Contract shared by every entry point:
 *  - all pointers are device pointers the caller owns; the library allocates
 *    nothing and keeps no state between calls (vectra_scan_top_k_no_alloc
 *    keeps a static scratch array per GPU, zero between calls);
 *  - work is queued on `stream`, asynchronously; nothing is synchronised;
 *  - sizes and strides are in elements (floats, or bytes for codes);
 *  - zero counts are valid and launch nothing;
 *  - a candidate id that is not below the row (code) count gives a NaN
 *    distance and reads nothing;
 *  - the return value is a vectra_scan_status; no error crosses the ABI as
 *    an exception.
 */
#ifndef VECTRA_SCAN_H_
#define VECTRA_SCAN_H_

#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define VECTRA_SCAN_ABI_VERSION 3

/* Entries of a PQ sub-space's codebook (kPqCentroids,
 * include/vectra/index/simd_distance.h). */
#define VECTRA_PQ_CENTROIDS 256

typedef enum vectra_scan_status {
  VECTRA_SCAN_OK = 0,
  VECTRA_SCAN_INVALID_ARGUMENT = 1,
  VECTRA_SCAN_TOO_LARGE = 2,
  VECTRA_SCAN_LAUNCH_FAILED = 3
} vectra_scan_status;

typedef enum vectra_scan_metric {
  /* L2SquaredDistance(query, row, dimension), simd_distance.cc:36-51 */
  VECTRA_SCAN_L2_SQUARED = 0,
  /* InnerProduct(query, row, dimension), simd_distance.cc:53-62 */
  VECTRA_SCAN_INNER_PRODUCT = 1,
  /* SquaredNorm(row, dimension), simd_distance.cc:64-66 (no queries) */
  VECTRA_SCAN_SQUARED_NORM = 2
} vectra_scan_metric;

/*
 * Row scan: out[q * out_stride + i] = metric(query q, row ids[i]) for every
 * query q < num_queries and candidate i < num_ids, or of row i for
 * i < num_rows when ids is NULL.  (In every entry point here a NULL `ids`
 * means every row whatever num_ids is; an empty candidate list is a
 * non-NULL `ids` with num_ids 0, of which nothing is read.  A zero-size
 * allocation may come back NULL: pass any valid pointer for it.)  Query q is `dimension` floats at
 * queries + q * query_stride; row r at rows + r * row_stride.  For
 * VECTRA_SCAN_SQUARED_NORM, `queries` is unused and num_queries must be 1.
 * With dimension 0 every output is 0 and `queries` and `rows` may be NULL.
 *
 * Replaces the per-node distance loops of ShardIndex::ExhaustiveSearch
 * (shard_index.cc:244-264) and the re-rank in hnsw_searcher.cc:145-158, and
 * FlatVectorStore's norm computation (flat_store.cc:46).
 */
typedef struct vectra_scan_args {
  int32_t metric;            /* vectra_scan_metric */
  int32_t dimension;         /* >= 0 floats per vector */
  const float* queries;      /* [num_queries][query_stride] */
  int64_t num_queries;
  int64_t query_stride;      /* >= dimension */
  const float* rows;         /* [num_rows][row_stride] */
  int64_t num_rows;
  int64_t row_stride;        /* >= dimension */
  const uint32_t* ids;       /* [num_ids] candidate rows, or NULL for every row in order */
  int64_t num_ids;
  float* out;                /* [num_queries][out_stride] */
  int64_t out_stride;        /* >= the candidate count */
} vectra_scan_args;

int vectra_scan_rows(const vectra_scan_args* args, hipStream_t stream);

/*
 * ADC distance tables: tables[q * table_stride + s * 256 + c] =
 * L2SquaredDistance(sub-vector s of query q, centroid c of sub-space s,
 * dimension / subspaces), as ProductQuantizer::ComputeDistanceTable
 * (pq_codec.cc:208-217).  `codebooks` is laid out as
 * ProductQuantizer::codebooks() (pq_codec.h): [subspaces][256][dimension /
 * subspaces].  dimension must be a positive multiple of subspaces
 * (ProductQuantizer::FromCodebooks, pq_codec.cc).
 */
typedef struct vectra_pq_table_args {
  int32_t dimension;
  int32_t subspaces;
  const float* queries;      /* [num_queries][query_stride] */
  int64_t num_queries;
  int64_t query_stride;      /* >= dimension */
  const float* codebooks;    /* [subspaces][256][dimension / subspaces] */
  float* tables;             /* [num_queries][table_stride] */
  int64_t table_stride;      /* >= subspaces * 256 */
} vectra_pq_table_args;

int vectra_pq_distance_tables(const vectra_pq_table_args* args, hipStream_t stream);

/*
 * ADC scan: out[q * out_stride + i] = PqAdcDistance(table q, code ids[i],
 * subspaces) (simd_distance.cc:68-81) for every query table q and candidate
 * i, or of code i when ids is NULL.  Table q is subspaces * 256 floats at
 * tables + q * table_stride; code r is `subspaces` bytes at
 * codes + r * code_stride.  subspaces is 1 .. 256.
 */
typedef struct vectra_pq_adc_args {
  int32_t subspaces;
  const float* tables;       /* [num_queries][table_stride] */
  int64_t num_queries;
  int64_t table_stride;      /* >= subspaces * 256 */
  const uint8_t* codes;      /* [num_codes][code_stride] */
  int64_t num_codes;
  int64_t code_stride;       /* >= subspaces */
  const uint32_t* ids;       /* [num_ids] candidate codes, or NULL for every code in order */
  int64_t num_ids;
  float* out;                /* [num_queries][out_stride] */
  int64_t out_stride;        /* >= the candidate count */
} vectra_pq_adc_args;

int vectra_scan_pq_adc(const vectra_pq_adc_args* args, hipStream_t stream);

/* Largest k of vectra_scan_top_k (SearchLimits::max_top_k,
 * include/vectra/service/search_handler.h:28) and the node of an empty
 * result slot. */
#define VECTRA_SCAN_MAX_K 1024
#define VECTRA_SCAN_NO_NODE 0xFFFFFFFFu

/*
 * Exhaustive k-nearest search: for every query q, the k candidates nearest
 * by L2SquaredDistance, as ShardIndex::ExhaustiveSearch returns them
 * (shard_index.cc:236-264): candidates are the rows ids[0 .. num_ids) (ids
 * not below num_rows are skipped, :245; duplicates are kept), or every row
 * when ids is NULL; at most k are kept (PushBounded, :111-120) and they are
 * ordered by CloserFirst (include/vectra/index/search_scratch.h: distance
 * ascending, ties by node id ascending).  Result r of query q is
 * distances[q * out_stride + r] and nodes[q * out_stride + r] (the row
 * index); slots past the number of candidates hold +inf and
 * VECTRA_SCAN_NO_NODE.  Distances are bit-identical to vectra_scan_rows'
 * (NaN distances, which CloserFirst cannot order, rank after every number,
 * ties by node, and come out as the quiet NaN 0x7fc00000).  k is
 * 1 .. VECTRA_SCAN_MAX_K; num_rows is below VECTRA_SCAN_NO_NODE.  With
 * dimension 0 every distance is 0 and `queries` and `rows` may be NULL.
 */
typedef struct vectra_scan_top_k_args {
  int32_t dimension;         /* >= 0 floats per vector */
  int32_t k;                 /* 1 .. VECTRA_SCAN_MAX_K */
  const float* queries;      /* [num_queries][query_stride] */
  int64_t num_queries;
  int64_t query_stride;      /* >= dimension */
  const float* rows;         /* [num_rows][row_stride] */
  int64_t num_rows;
  int64_t row_stride;        /* >= dimension */
  const uint32_t* ids;       /* [num_ids] candidate rows, or NULL for every row */
  int64_t num_ids;
  float* distances;          /* [num_queries][out_stride] */
  uint32_t* nodes;           /* [num_queries][out_stride] */
  int64_t out_stride;        /* >= k */
} vectra_scan_top_k_args;

int vectra_scan_top_k(const vectra_scan_top_k_args* args, hipStream_t stream);

/*
 * vectra_scan_top_k with a device workspace: below 64 queries the
 * candidates of a query are cut into ranges, one workgroup each (at least 64
 * candidates per range, at most 64 ranges, ranges * k <= 2048), and the
 * workgroup that finishes last merges the ranges' k best; the results are
 * the same bits as vectra_scan_top_k's.  The workspace is `workspace_bytes`
 * of device memory, 256-byte aligned, whose first 256 bytes (arrival
 * counters) are zero before the first call on it; every call leaves them
 * zero.  With a NULL or smaller workspace than
 * vectra_scan_top_k_workspace_bytes(args), or 64 queries or more, this is
 * vectra_scan_top_k.  Calls that share a workspace must not overlap.
 * Replaces the same reference loop as vectra_scan_top_k
 * (shard_index.cc:236-264), for requests of one or a few queries.
 */
int vectra_scan_top_k_ws(const vectra_scan_top_k_args* args, void* workspace, int64_t workspace_bytes,
                         hipStream_t stream);

/* Workspace bytes vectra_scan_top_k_ws uses for these arguments (0: none;
 * also 0 for arguments vectra_scan_top_k would reject). */
int64_t vectra_scan_top_k_workspace_bytes(const vectra_scan_top_k_args* args);

/*
 * vectra_scan_top_k_ws with the library's own scratch instead of a
 * workspace: it allocates nothing, for callers that cannot allocate (code
 * under HIP graph capture, serving loops that forbid allocation).  No
 * counterpart in the reference.  The scratch is a static device array of
 * 1,048,832 bytes on each GPU the library runs on, held until the process
 * ends; a call whose split form would need more returns
 * VECTRA_SCAN_TOO_LARGE (none does within the limits above).  Every call on
 * one GPU shares that GPU's scratch: calls that overlap on one GPU race.
 */
int vectra_scan_top_k_no_alloc(const vectra_scan_top_k_args* args, hipStream_t stream);

const char* vectra_scan_status_string(int status);
int vectra_scan_abi_version(void);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif  /* VECTRA_SCAN_H_ */
