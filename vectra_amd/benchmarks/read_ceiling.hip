// Plain streaming read of a device buffer: the practical HBM read ceiling
// that the serving kernel (98 % K and V reads) is compared with; and a
// streaming read with writes mixed in, the ceiling of kernels that write a
// larger share of their bytes (the plane kernels write a quarter).
//
// Built into vectra_amd/lib/libvectra_bench.so; benchmark infrastructure,
// not part of the operator.  Each lane issues kUnroll independent 16-byte
// non-temporal loads per iteration of a grid-stride loop (the same load form
// the stream kernel uses for K and V) and folds them into one word, which is
// stored only if it equals a value the data never produces in practice, so
// the loads cannot be removed and almost nothing is written.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kUnroll = 4;

__global__ __launch_bounds__(kThreads) void read_stream_kernel(const u32x4* src, int64_t n16,
                                                               uint32_t* sink) {
  uint32_t acc = 0;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads * kUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kThreads * kUnroll + threadIdx.x; base < n16;
       base += step) {
    u32x4 x[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + u * kThreads;
      x[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= x[u].x ^ x[u].y ^ x[u].z ^ x[u].w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x * kThreads + threadIdx.x] = acc;
}

// Reads and writes interleaved as a kernel that produces one output word
// from kRatio input words does: unit i of the grid-stride loop reads word i
// of each of the kRatio input regions (each region n_write16 words, one
// coalesced load per region) and writes word i of the output with a
// non-temporal store.  Input words past kRatio * n_write16 are read in a
// tail loop.
template <int kRatio>
__global__ __launch_bounds__(kThreads) void read_write_stream_kernel(const u32x4* src, int64_t n_read16, u32x4* dst,
                                                                     int64_t n_write16, uint32_t* sink) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * kThreads;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
  for (int64_t i = first; i < n_write16; i += step) {
    u32x4 x[kRatio];
#pragma unroll
    for (int u = 0; u < kRatio; ++u) x[u] = __builtin_nontemporal_load(src + u * n_write16 + i);
    u32x4 acc = x[0];
#pragma unroll
    for (int u = 1; u < kRatio; ++u) acc ^= x[u];
    __builtin_nontemporal_store(acc, dst + i);
  }
  uint32_t tail = 0;
  for (int64_t i = kRatio * n_write16 + first; i < n_read16; i += step) {
    const u32x4 x = __builtin_nontemporal_load(src + i);
    tail ^= x.x ^ x.y ^ x.z ^ x.w;
  }
  if (tail == 0x9e3779b9u) sink[blockIdx.x * kThreads + threadIdx.x] = tail;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16, 16-byte-aligned `src`) once on `stream`
// with `blocks` workgroups of 256 threads.  `sink` must hold blocks * 256
// words.  Returns 0 on success, 1 on bad arguments, 2 on a launch error.
int vectra_bench_read_stream(const void* src, int64_t bytes, uint32_t* sink, int32_t blocks,
                             hipStream_t stream) {
  if (src == nullptr || sink == nullptr || bytes < 0 || bytes % 16 != 0 || blocks < 1 ||
      (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
    return 1;
  if (bytes == 0) return 0;
  hipLaunchKernelGGL(read_stream_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kThreads), 0, stream,
                     static_cast<const u32x4*>(src), bytes / 16, sink);
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

// Reads `read_bytes` from `src` and writes `write_bytes` to `dst` in one
// launch on `stream` (both multiples of 16, 16-byte-aligned buffers, and
// 1 <= read_bytes / write_bytes; reads go to floor(read / write) <= 8 input
// regions of write_bytes each, the rest in a tail).  `sink` must hold
// blocks * 256 words.  Returns 0 on success, 1 on bad arguments, 2 on a
// launch error.
int vectra_bench_read_write_stream(const void* src, int64_t read_bytes, void* dst, int64_t write_bytes,
                                   uint32_t* sink, int32_t blocks, hipStream_t stream) {
  if (src == nullptr || dst == nullptr || sink == nullptr || read_bytes % 16 != 0 || write_bytes % 16 != 0 ||
      write_bytes < 16 || read_bytes < write_bytes || blocks < 1 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0 ||
      (reinterpret_cast<uintptr_t>(dst) & 15u) != 0)
    return 1;
  const int64_t ratio = read_bytes / write_bytes;
  const auto* in = static_cast<const u32x4*>(src);
  auto* out = static_cast<u32x4*>(dst);
  const int64_t nr = read_bytes / 16, nw = write_bytes / 16;
  const dim3 grid(static_cast<unsigned>(blocks)), block(kThreads);
  switch (ratio) {
    case 1: hipLaunchKernelGGL(read_write_stream_kernel<1>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 2: hipLaunchKernelGGL(read_write_stream_kernel<2>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 3: hipLaunchKernelGGL(read_write_stream_kernel<3>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 4: hipLaunchKernelGGL(read_write_stream_kernel<4>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 5: hipLaunchKernelGGL(read_write_stream_kernel<5>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 6: hipLaunchKernelGGL(read_write_stream_kernel<6>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 7: hipLaunchKernelGGL(read_write_stream_kernel<7>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    case 8: hipLaunchKernelGGL(read_write_stream_kernel<8>, grid, block, 0, stream, in, nr, out, nw, sink); break;
    default: return 1;
  }
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

}  // extern "C"
