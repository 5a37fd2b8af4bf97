/*
 * vectra_rbf.h -- C ABI of the MI355X (gfx950) fused RBF-attention library.
 *
 *   out[b,h,i,:] = sum_j softmax_j( -scale[b,h] * max(|q_i|^2 + |k_j|^2 - 2 q_i.k_j, 0)
 *                                   + key_bias[b,h,j] ) * v[b,h,j,:]
 *
 * This header is the drop-in boundary for the device implementation of the
 * operator `vectra::rbf_attention`.  It replaces the reference's GPU entry
 *   kernels/vectra_kernels/spatial_rbf_attention.py:177-281 (rbf_attention_forward,
 *   the Triton launch) and
 *   kernels/vectra_kernels/norm_precompute.py:67-86 (squared_norms),
 * which the reference binds to the operator at
 *   kernels/vectra_kernels/custom_ops.py:75-85 (the 'cuda' kernel registration).
 *
 * Contract:
 *  - Plain pointers, sizes and element strides; no torch types cross the ABI.
 *  - Every buffer is owned by the caller.  The library allocates nothing on
 *    the device or the host.  Its only global state is three write-once
 *    caches of facts that never change within a process: the compute-unit
 *    count of each device (an atomic per device id), the environment
 *    override VECTRA_STREAM_WAVES_PER_CU (read once), and per kernel
 *    instantiation the number of its workgroups resident on one compute
 *    unit (an atomic, asked of the HIP runtime on first launch).  Two threads
 *    that fill one cache at once store the same value, so calls are
 *    reentrant and may be captured into a HIP graph.
 *  - Work is enqueued on `stream` and the call returns without synchronising.
 *  - Errors are returned as a status code (never thrown); see
 *    vectra_rbf_status_string().
 */
#ifndef VECTRA_RBF_H_
#define VECTRA_RBF_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* vectra_stream_t;

/* Element types.  q, k and v share one of F32/F16/BF16; scale and key_bias
 * may be any of the four (they are converted to fp32 on load, as the
 * reference does with `.to(torch.float32)` at spatial_rbf_attention.py:208-213
 * and :221). */
typedef enum vectra_dtype {
  VECTRA_F32 = 0,
  VECTRA_F16 = 1,
  VECTRA_BF16 = 2,
  VECTRA_F64 = 3
} vectra_dtype;

/* Status codes. */
enum {
  VECTRA_OK = 0,
  VECTRA_ERR_NULL_ARGUMENT = 1,    /* a required pointer is NULL            */
  VECTRA_ERR_BAD_DTYPE = 2,        /* unsupported dtype combination         */
  VECTRA_ERR_BAD_SHAPE = 3,        /* negative or inconsistent sizes        */
  VECTRA_ERR_BAD_STRUCT = 4,       /* struct_size does not match this build */
  VECTRA_ERR_TOO_LARGE = 5,        /* a size exceeds the kernels' index range */
  VECTRA_ERR_LAUNCH = 6,           /* the HIP launch itself failed          */
  VECTRA_ERR_BAD_VARIANT = 7,      /* forced kernel variant cannot run this problem */
  VECTRA_ERR_BAD_FLAGS = 8         /* flags has bits this build does not know */
};

/* Kernel variants (for benchmarks and tests; VECTRA_VARIANT_AUTO in production). */
enum {
  VECTRA_VARIANT_AUTO = 0,
  VECTRA_VARIANT_GENERIC = 1,  /* any strides / dims / dtypes               */
  VECTRA_VARIANT_STREAM = 2,   /* few query rows: HBM-scheduled, 128-bit loads */
  VECTRA_VARIANT_MFMA = 3,     /* query tiles of 16+ rows on MFMA (bf16/fp16/fp32) */
  VECTRA_VARIANT_PLANE = 4,    /* whole (b, h) planes of <= 80 rows per wave on MFMA (bf16/fp16) */
  VECTRA_VARIANT_TILE = 5      /* key tiles streamed through LDS, 32 query rows per wave (bf16/fp16) */
};

/*
 * Problem description.  All strides are in ELEMENTS of the tensor they
 * describe and may be zero (broadcast) or arbitrary (head-transposed views,
 * spatial_rbf_attention.py:31-32; negative ones too, which the generic
 * kernel serves: the faster kernels address rows by unsigned offsets).
 *
 *   q   [B, H, Nq, D]    k [B, H, Nk, D]    v [B, H, Nk, Dv]
 *   out [B, H, Nq, Dv]   written in out_dtype (the operator passes v.dtype;
 *                        parity harnesses ask for F32)
 *   scale    broadcast to [B, H]: element (b,h) at scale[b*scale_stride_b + h*scale_stride_h]
 *   key_bias optional (NULL = none), broadcast to [B, H, Nk]: element (b,h,j) at
 *            key_bias[b*bias_stride_b + h*bias_stride_h + j*bias_stride_n].
 *            A per-query bias is not expressible (spatial_rbf_attention.py:224-225).
 *            Without a bias every key < Nk takes part.
 */
typedef struct vectra_rbf_args {
  int64_t struct_size; /* sizeof(vectra_rbf_args) as compiled by the caller */

  const void* q;
  const void* k;
  const void* v;
  void* out;
  const void* scale;
  const void* key_bias;

  int32_t in_dtype;    /* dtype of q, k, v: F32, F16 or BF16 */
  int32_t out_dtype;   /* F32, F16 or BF16 */
  int32_t scale_dtype; /* any vectra_dtype */
  int32_t bias_dtype;  /* any vectra_dtype (ignored when key_bias == NULL) */

  int64_t batch, heads, n_q, n_k, head_dim, value_dim;

  int64_t q_stride[4];   /* (b, h, n, d) */
  int64_t k_stride[4];
  int64_t v_stride[4];
  int64_t out_stride[4];
  int64_t scale_stride_b, scale_stride_h;
  int64_t bias_stride_b, bias_stride_h, bias_stride_n;

  int32_t variant;  /* VECTRA_VARIANT_*; 0 picks automatically */
  int32_t flags;    /* VECTRA_FLAG_* bits; 0 by default (other bits are rejected) */
} vectra_rbf_args;

/*
 * VECTRA_FLAG_SPLIT_WEIGHTS: the tile kernel keeps every weight as a 16-bit
 * hi + lo pair (2^-17 of it).  By default, on key axes of 1024 keys or more
 * with no bias and scale >= 0, it first rounds each weight once to fp16 (2^-11
 * of it, one product instead of two).  The rounding errors of independent
 * weights add up like a random walk; the kernel bounds the walk's deviation
 * per output from the weights' sums (sum w, sum w^2) and the largest |v|, and
 * keeps the fp16 result for a work item only if four such deviations fit
 * rtol 1e-3 / atol 1e-4 at every output and every weight sum is at least 256;
 * otherwise (large values, weights held by few keys) the item runs the split.
 * A pass whose bound misses twice over after an eighth of the keys stops
 * there.  Other kernels ignore the flag.  (No counterpart in the reference:
 * its kernel rounds the weights to the input dtype,
 * spatial_rbf_attention.py:163.)
 */
enum { VECTRA_FLAG_SPLIT_WEIGHTS = 1 };

/*
 * Enqueues the fused forward pass on `stream`.
 * Replaces spatial_rbf_attention.py:177-281 (host launch) and :47-174 (kernel).
 * Returns VECTRA_OK or an error code; on error nothing was enqueued.
 * Zero-sized problems (B*H*Nq == 0 or Dv == 0) are a successful no-op;
 * Nk == 0 with Nq > 0 writes rows of zeros, as the reference's default
 * implementation does (reference.py:79-99: softmax over an empty axis times
 * an empty v is an empty sum, 0).
 */
int vectra_rbf_attention_fwd(const vectra_rbf_args* args, vectra_stream_t stream);

/*
 * Row norms |x_j|^2 in fp32: out[(b*H + h)*N + j] (contiguous [B, H, N]).
 * Replaces norm_precompute.py:67-86 (squared_norms); x is [B, H, N, D] with
 * element strides x_stride and dtype F32/F16/BF16.
 */
int vectra_rbf_squared_norms(const void* x, int32_t dtype, int64_t batch, int64_t heads,
                             int64_t rows, int64_t cols, const int64_t x_stride[4],
                             float* out, vectra_stream_t stream);

/*
 * The variant vectra_rbf_attention_fwd() would run for `args` (VECTRA_VARIANT_*),
 * or a negative status if the arguments are invalid.  Host-only; no GPU call.
 * Replaces the reference's tile heuristic tile_configs.py:114-133 (select).
 */
int vectra_rbf_select_variant(const vectra_rbf_args* args);

/* Human-readable text for a status code (static storage, never NULL). */
const char* vectra_rbf_status_string(int status);

/* Library ABI version: (major << 16) | minor.  Host-only. */
int vectra_rbf_abi_version(void);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* VECTRA_RBF_H_ */
