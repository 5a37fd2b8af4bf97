// The C ABI of libvectra_rbf.so: argument validation, kernel selection and
// launch.  Declared in include/vectra_rbf.h.
//
// Replaces the reference's host launch (kernels/vectra_kernels/
// spatial_rbf_attention.py:177-281) and tile heuristic (tile_configs.py:114-133).
// Differences by design:
//  * no device allocation: scale and key_bias are read in place through their
//    dtype and strides (the reference materialises an fp32 [B*H] scale copy and
//    an fp32 bias copy, :208-213 and :221);
//  * the output dtype is a parameter, so a parity harness can read the fp32
//    result of the same kernel the operator runs in v.dtype.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>

#include "rbf_common.h"
#include "rbf_kernels.h"
#include "vectra_rbf.h"

namespace vectra {

void make_fast_div(int64_t d, uint32_t* mul, uint32_t* shift) {
  uint32_t l = 0;
  while ((int64_t{1} << l) < d) ++l;  // l = ceil(log2 d)
  if ((int64_t{1} << l) == d) {
    *mul = 0;
    *shift = l;
    return;
  }
  *mul = static_cast<uint32_t>(((uint64_t{1} << (31 + l)) + static_cast<uint64_t>(d) - 1) /
                               static_cast<uint64_t>(d));
  *shift = l - 1;
}

}  // namespace vectra

namespace {

using vectra::make_fast_div;
using vectra::Problem;

constexpr int kAbiMajor = 1;
constexpr int kAbiMinor = 3;

bool is_io_dtype(int32_t d) { return d == VECTRA_F32 || d == VECTRA_F16 || d == VECTRA_BF16; }
bool is_any_dtype(int32_t d) { return is_io_dtype(d) || d == VECTRA_F64; }
int elem_size(int32_t d) { return d == VECTRA_F32 ? 4 : (d == VECTRA_F64 ? 8 : 2); }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device.  Cached per device: a device property
// never changes, so the cache is the only state the library keeps.
int device_compute_units() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 256;
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Waves per CU the stream kernel is sized for: 32 (8 per SIMD) by default,
// which at the serving shape gives one row per wave with every wave resident
// at once (measured fastest on MI355X); VECTRA_STREAM_WAVES_PER_CU (1..32)
// overrides it for tuning sweeps.
int stream_waves_per_cu() {
  static const int value = [] {
    const char* env = getenv("VECTRA_STREAM_WAVES_PER_CU");
    const int v = env ? atoi(env) : 0;
    return (v >= 1 && v <= 32) ? v : 32;
  }();
  return value;
}

int validate(const vectra_rbf_args* a) {
  if (a == nullptr) return VECTRA_ERR_NULL_ARGUMENT;
  if (a->struct_size != static_cast<int64_t>(sizeof(vectra_rbf_args))) return VECTRA_ERR_BAD_STRUCT;
  if (!is_io_dtype(a->in_dtype) || !is_io_dtype(a->out_dtype) || !is_any_dtype(a->scale_dtype))
    return VECTRA_ERR_BAD_DTYPE;
  if (a->key_bias != nullptr && !is_any_dtype(a->bias_dtype)) return VECTRA_ERR_BAD_DTYPE;
  if (a->batch < 0 || a->heads < 0 || a->n_q < 0 || a->n_k < 0 || a->head_dim < 0 ||
      a->value_dim < 0)
    return VECTRA_ERR_BAD_SHAPE;
  if (a->variant < VECTRA_VARIANT_AUTO || a->variant > VECTRA_VARIANT_TILE)
    return VECTRA_ERR_BAD_VARIANT;
  if ((a->flags & ~VECTRA_FLAG_SPLIT_WEIGHTS) != 0) return VECTRA_ERR_BAD_FLAGS;
  // Each size below 2^31 keeps every product of two or three of them in int64.
  constexpr int64_t kMaxDim = 0x7fffffffLL;
  if (a->batch > kMaxDim || a->heads > kMaxDim || a->n_q > kMaxDim || a->n_k > kMaxDim ||
      a->head_dim > kMaxDim || a->value_dim > kMaxDim)
    return VECTRA_ERR_TOO_LARGE;
  const int64_t rows = a->batch * a->heads * a->n_q;
  if (rows == 0 || a->value_dim == 0) return VECTRA_OK;  // nothing to read or write
  // Buffers with no elements may be NULL (torch gives empty tensors no storage).
  if (a->out == nullptr || a->scale == nullptr || (a->head_dim > 0 && a->q == nullptr) ||
      (a->n_k > 0 && a->head_dim > 0 && a->k == nullptr) || (a->n_k > 0 && a->v == nullptr))
    return VECTRA_ERR_NULL_ARGUMENT;
  // Kernels index query rows with 32-bit wave ids.
  if (rows > 0x7fffffffLL) return VECTRA_ERR_TOO_LARGE;
  // The generic kernel's grid has one row of workgroups per 256 value columns.
  if ((a->value_dim + 255) / 256 > vectra::kMaxGenericSlices) return VECTRA_ERR_TOO_LARGE;
  return VECTRA_OK;
}

Problem make_problem(const vectra_rbf_args* a) {
  Problem p{};
  p.q = a->q;
  p.k = a->k;
  p.v = a->v;
  p.out = a->out;
  p.scale = a->scale;
  p.bias = a->key_bias;
  p.scale_dtype = a->scale_dtype;
  p.bias_dtype = a->bias_dtype;
  p.B = a->batch;
  p.H = a->heads;
  p.Nq = a->n_q;
  p.Nk = a->n_k;
  p.D = a->head_dim;
  p.Dv = a->value_dim;
  for (int i = 0; i < 4; ++i) {
    p.sq[i] = a->q_stride[i];
    p.sk[i] = a->k_stride[i];
    p.sv[i] = a->v_stride[i];
    p.so[i] = a->out_stride[i];
  }
  p.ssb = a->scale_stride_b;
  p.ssh = a->scale_stride_h;
  p.sbb = a->bias_stride_b;
  p.sbh = a->bias_stride_h;
  p.sbn = a->bias_stride_n;
  p.total_rows = a->batch * a->heads * a->n_q;
  p.flags = a->flags;
  make_fast_div(a->n_q > 0 ? a->n_q : 1, &p.nq_mul, &p.nq_shift);
  make_fast_div(a->heads > 0 ? a->heads : 1, &p.h_mul, &p.h_shift);
  return p;
}

// Number of 16-byte chunks per row if the stream kernel can run `a`, else 0.
int stream_chunks(const vectra_rbf_args* a) {
  // Stream kernels write the input dtype or fp32.
  if (a->out_dtype != a->in_dtype && a->out_dtype != VECTRA_F32) return 0;
  // The stream kernels decode 2- and 4-byte coefficient and bias elements.
  if (a->scale_dtype == VECTRA_F64 || (a->key_bias != nullptr && a->bias_dtype == VECTRA_F64))
    return 0;
  const int in_sz = elem_size(a->in_dtype);
  const int vec = 16 / in_sz;
  if (a->head_dim != a->value_dim || a->head_dim == 0 || a->head_dim % vec != 0) return 0;
  const int64_t chunks = a->head_dim / vec;
  if (chunks != 2 && chunks != 4 && chunks != 8 && chunks != 16) return 0;
  // 8- and 16-chunk rows run one key tile per row only (more would spill
  // registers in the looping variant).
  if (chunks >= 8 && a->n_k > 64) return 0;
  // Per-lane key offsets inside a (b, h) plane are unsigned 32-bit: key row
  // strides (K, V and the bias) must be non-negative and the last row's
  // bytes within 2^31.
  if (a->k_stride[2] < 0 || a->v_stride[2] < 0 || (a->key_bias != nullptr && a->bias_stride_n < 0)) return 0;
  const int64_t limit = int64_t{1} << 31;
  const int64_t last_key = a->n_k > 0 ? a->n_k - 1 : 0;
  if (last_key * a->k_stride[2] * in_sz + 16 * chunks >= limit ||
      last_key * a->v_stride[2] * in_sz + 16 * chunks >= limit)
    return 0;
  if (a->key_bias != nullptr && last_key * a->bias_stride_n * elem_size(a->bias_dtype) + 4 >= limit)
    return 0;
  const int64_t* strides[3] = {a->q_stride, a->k_stride, a->v_stride};
  const void* ptrs[3] = {a->q, a->k, a->v};
  for (int t = 0; t < 3; ++t) {
    if (strides[t][3] != 1 || !aligned16(ptrs[t])) return 0;
    for (int d = 0; d < 3; ++d)
      if (strides[t][d] % vec != 0) return 0;
  }
  // Output: each lane writes vec contiguous elements of out_dtype (8, 16 or
  // 32 bytes) with 16-byte stores, or 8-byte stores for an 8-byte chunk.
  // Strides that are multiples of vec keep every chunk as aligned as the base.
  const int out_chunk_bytes = vec * elem_size(a->out_dtype);
  const uintptr_t need = out_chunk_bytes >= 16 ? 16 : 8;
  if (a->out_stride[3] != 1 || (reinterpret_cast<uintptr_t>(a->out) & (need - 1)) != 0) return 0;
  for (int d = 0; d < 3; ++d)
    if (a->out_stride[d] % vec != 0) return 0;
  return static_cast<int>(chunks);
}

// Query tiles of this many rows or more go to the MFMA kernel.
constexpr int64_t kMfmaMinQueries = 16;

int select_variant(const vectra_rbf_args* a) {
  const Problem p = make_problem(a);
  const bool mfma = vectra::mfma_supports(p, a->in_dtype, a->out_dtype);
  const bool plane = vectra::plane_supports(p, a->in_dtype, a->out_dtype);
  const bool tile = vectra::tile_supports(p, a->in_dtype, a->out_dtype);
  switch (a->variant) {
    case VECTRA_VARIANT_GENERIC: return VECTRA_VARIANT_GENERIC;
    case VECTRA_VARIANT_STREAM: return stream_chunks(a) ? VECTRA_VARIANT_STREAM : -VECTRA_ERR_BAD_VARIANT;
    case VECTRA_VARIANT_MFMA: return mfma ? VECTRA_VARIANT_MFMA : -VECTRA_ERR_BAD_VARIANT;
    case VECTRA_VARIANT_PLANE: return plane ? VECTRA_VARIANT_PLANE : -VECTRA_ERR_BAD_VARIANT;
    case VECTRA_VARIANT_TILE: return tile ? VECTRA_VARIANT_TILE : -VECTRA_ERR_BAD_VARIANT;
    default: break;
  }
  if (a->n_q >= kMfmaMinQueries) {
    if (plane) return VECTRA_VARIANT_PLANE;
    if (tile) return VECTRA_VARIANT_TILE;
    if (mfma) return VECTRA_VARIANT_MFMA;
  }
  return stream_chunks(a) ? VECTRA_VARIANT_STREAM : VECTRA_VARIANT_GENERIC;
}

}  // namespace

extern "C" {

int vectra_rbf_attention_fwd(const vectra_rbf_args* a, vectra_stream_t stream) {
  const int status = validate(a);
  if (status != VECTRA_OK) return status;
  if (a->batch * a->heads * a->n_q == 0 || a->value_dim == 0) return VECTRA_OK;
  const int variant = select_variant(a);
  if (variant < 0) return -variant;
  Problem p = make_problem(a);
  // Wave budget for the persistent stream kernel (it sizes its own grid).
  p.compute_units = device_compute_units();
  p.grid_waves = p.compute_units * stream_waves_per_cu();
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipError_t err = hipErrorInvalidValue;
  switch (variant) {
    case VECTRA_VARIANT_STREAM:
      err = vectra::launch_stream(p, a->in_dtype, a->out_dtype, stream_chunks(a), s);
      break;
    case VECTRA_VARIANT_MFMA:
      err = vectra::launch_mfma(p, a->in_dtype, a->out_dtype, s);
      break;
    case VECTRA_VARIANT_PLANE:
      err = vectra::launch_plane(p, a->in_dtype, a->out_dtype, s);
      break;
    case VECTRA_VARIANT_TILE:
      err = vectra::launch_tile(p, a->in_dtype, a->out_dtype, s);
      break;
    default:
      err = vectra::launch_generic(p, a->in_dtype, a->out_dtype, s);
      break;
  }
  return err == hipSuccess ? VECTRA_OK : VECTRA_ERR_LAUNCH;
}

int vectra_rbf_squared_norms(const void* x, int32_t dtype, int64_t batch, int64_t heads,
                             int64_t rows, int64_t cols, const int64_t x_stride[4], float* out,
                             vectra_stream_t stream) {
  if (!is_io_dtype(dtype)) return VECTRA_ERR_BAD_DTYPE;
  if (batch < 0 || heads < 0 || rows < 0 || cols < 0) return VECTRA_ERR_BAD_SHAPE;
  if (batch == 0 || heads == 0 || rows == 0) return VECTRA_OK;
  if (x == nullptr || out == nullptr || x_stride == nullptr) return VECTRA_ERR_NULL_ARGUMENT;
  // The kernel loops over rows with a grid stride, so any row count fits its
  // grid; rows are 64-bit.  B*H*N must not overflow int64.
  if (rows > INT64_MAX / batch / heads) return VECTRA_ERR_TOO_LARGE;
  const hipError_t err = vectra::launch_squared_norms(x, dtype, batch, heads, rows, cols, x_stride,
                                                      out, reinterpret_cast<hipStream_t>(stream));
  return err == hipSuccess ? VECTRA_OK : VECTRA_ERR_LAUNCH;
}

int vectra_rbf_select_variant(const vectra_rbf_args* a) {
  const int status = validate(a);
  if (status != VECTRA_OK) return -status;
  return select_variant(a);
}

const char* vectra_rbf_status_string(int status) {
  switch (status) {
    case VECTRA_OK: return "ok";
    case VECTRA_ERR_NULL_ARGUMENT: return "a required pointer is NULL";
    case VECTRA_ERR_BAD_DTYPE: return "unsupported dtype (q/k/v/out: f32, f16 or bf16; scale/bias: f32, f16, bf16 or f64)";
    case VECTRA_ERR_BAD_SHAPE: return "negative size";
    case VECTRA_ERR_BAD_STRUCT: return "vectra_rbf_args.struct_size does not match the library";
    case VECTRA_ERR_TOO_LARGE: return "problem exceeds the kernel grid limits";
    case VECTRA_ERR_LAUNCH: return "HIP kernel launch failed";
    case VECTRA_ERR_BAD_VARIANT: return "the requested kernel variant cannot run this problem";
    case VECTRA_ERR_BAD_FLAGS: return "unknown bits in flags";
    default: return "unknown status";
  }
}

int vectra_rbf_abi_version(void) { return (kAbiMajor << 16) | kAbiMinor; }

}  // extern "C"
