// How far matrix-core and vector instructions overlap on one gfx950 SIMD: the
// practical ceiling of a kernel that needs both, such as the long-key tile
// kernel (per score one FMA, one exp2 and half a conversion beside its
// matrix products).
//
// Built into vectra_amd/lib/libvectra_bench.so; benchmark infrastructure, not
// part of the operator.  Every wave runs a loop whose body issues a fixed mix
// of independent instructions: 16x16x32 (or 32x32x16) bf16 MFMAs on 8 (4)
// accumulator chains and fp32 FMAs, optionally every fourth one an exp2, on
// 16 chains, in a fixed interleave (one MFMA, then its share of the vector
// instructions; scheduling groups keep that order).  The chains are long
// enough that no instruction waits on its predecessor's result.  Each wave
// reads the shader clock (s_memtime) and the 100 MHz constant clock
// (s_memrealtime) around the loop; the host divides by the iteration count.  A dynamic LDS allocation per one-wave workgroup fixes
// how many waves share a SIMD (one or two: 4 or 8 workgroups per compute
// unit, one grid of 256 x 4 x waves_per_simd workgroups).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kIters = 2000;

// kMfma matrix instructions and kValu vector instructions per iteration;
// kExp: every fourth vector instruction is an exp2; kBig: 32x32x16 MFMAs.
template <int kMfma, int kValu, bool kExp, bool kBig>
__global__ __launch_bounds__(64) void coexec_kernel(uint64_t* ticks, float* sink) {
  extern __shared__ float lds_pad[];  // sized by the launch: sets the waves per SIMD
  const int lane = static_cast<int>(threadIdx.x);
  bf16x8 a, b;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(0.001f * static_cast<float>(lane + i));
    b[i] = static_cast<__bf16>(0.002f * static_cast<float>(lane - i));
  }
  f32x4 acc[8];
  f32x16 big[4];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) big[c][e] = 0.f;
  float v[16];
#pragma unroll
  for (int c = 0; c < 16; ++c) v[c] = 0.01f * static_cast<float>(lane + c);
  lds_pad[lane] = v[0];
  __syncthreads();
  constexpr int kPer = kMfma > 0 ? kValu / kMfma : kValu;
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  for (int it = 0; it < kIters; ++it) {
#pragma unroll
    for (int m = 0; m < (kMfma > 0 ? kMfma : 1); ++m) {
      if constexpr (kMfma > 0) {
        if constexpr (kBig)
          big[m % 4] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, big[m % 4], 0, 0, 0);
        else
          acc[m % 8] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc[m % 8], 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < kPer; ++j) {
        const int k = m * kPer + j;
        if (kExp && k % 4 == 0)
          v[k % 16] = __builtin_amdgcn_exp2f(v[k % 16]);
        else
          v[k % 16] = fmaf(v[k % 16], 0.999f, 1e-3f);
      }
      if constexpr (kMfma > 0) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);     // the MFMA
        if constexpr (kPer > 0) __builtin_amdgcn_sched_group_barrier(0x002, kPer, 0);  // then its VALU share
      }
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < 8; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int e = 0; e < 16; ++e) s += big[c][e];
#pragma unroll
  for (int c = 0; c < 16; ++c) s += v[c];
  sink[blockIdx.x * 64 + lane] = s + lds_pad[(lane + 1) & 63];
  if (lane == 0) {
    ticks[2 * blockIdx.x] = t1 - t0;
    ticks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

struct Variant {
  const void* fn;
  int mfma, valu, exp, big;
};

#define VECTRA_COEXEC(m, v, e, g) {reinterpret_cast<const void*>(&coexec_kernel<m, v, e, g>), m, v, e, g}
const Variant kVariants[] = {
    VECTRA_COEXEC(8, 0, false, false),   // 0: 16x16x32 MFMAs alone
    VECTRA_COEXEC(0, 32, false, false),  // 1: FMAs alone
    VECTRA_COEXEC(0, 32, true, false),   // 2: 8 exp2 + 24 FMAs
    VECTRA_COEXEC(8, 16, false, false),  // 3: 1 MFMA : 2 FMAs
    VECTRA_COEXEC(8, 32, false, false),  // 4: 1 MFMA : 4 FMAs
    VECTRA_COEXEC(8, 64, false, false),  // 5: 1 MFMA : 8 FMAs
    VECTRA_COEXEC(8, 32, true, false),   // 6: 1 MFMA : 1 exp2 + 3 FMAs
    VECTRA_COEXEC(4, 0, false, true),    // 7: 32x32x16 MFMAs alone
    VECTRA_COEXEC(4, 32, false, true),   // 8: one 32x32x16 : 8 FMAs
};
#undef VECTRA_COEXEC
constexpr int kNumVariants = static_cast<int>(sizeof(kVariants) / sizeof(kVariants[0]));

}  // namespace

extern "C" {

int vectra_bench_coexec_variants(void) { return kNumVariants; }

// Describes variant `i` (MFMAs, vector instructions, exp2 flag, 32x32 flag).
int vectra_bench_coexec_describe(int i, int* mfma, int* valu, int* exp2, int* big) {
  if (i < 0 || i >= kNumVariants || !mfma || !valu || !exp2 || !big) return 1;
  *mfma = kVariants[i].mfma;
  *valu = kVariants[i].valu;
  *exp2 = kVariants[i].exp;
  *big = kVariants[i].big;
  return 0;
}

// Runs variant `i` with `waves_per_simd` (1 or 2) waves sharing each SIMD of
// device 0 and writes the mean shader-clock ticks per loop iteration, the
// shader clock's ticks per 100 MHz tick, and the loop's iteration count.
// `ticks` and `sink` are caller-owned device buffers of at least 4096 words
// (8-byte) and 2048 * 64 floats.  Synchronous.
int vectra_bench_coexec(int i, int waves_per_simd, const void* dev_ticks, const void* dev_sink, double* ticks_per_iter,
                        double* ticks_per_realtime, int* iters) {
  if (i < 0 || i >= kNumVariants || (waves_per_simd != 1 && waves_per_simd != 2) || !dev_ticks || !dev_sink ||
      !ticks_per_iter || !ticks_per_realtime || !iters)
    return 1;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0) != hipSuccess || cus < 1) return 2;
  const int blocks = cus * 4 * waves_per_simd;
  if (blocks > 2048) return 1;
  // 36 KB or 18 KB of LDS per one-wave workgroup: 4 or 8 resident per compute unit.
  const size_t lds = waves_per_simd == 1 ? 36 * 1024 : 18 * 1024;
  uint64_t* ticks = static_cast<uint64_t*>(const_cast<void*>(dev_ticks));
  float* sink = static_cast<float*>(const_cast<void*>(dev_sink));
  void* args[] = {&ticks, &sink};
  for (int rep = 0; rep < 2; ++rep) {  // the first run warms the instruction cache and clocks
    if (hipLaunchKernel(kVariants[i].fn, dim3(blocks), dim3(64), args, lds, nullptr) != hipSuccess) return 3;
    if (hipDeviceSynchronize() != hipSuccess) return 3;
  }
  std::vector<uint64_t> host(2 * static_cast<size_t>(blocks));
  if (hipMemcpy(host.data(), ticks, sizeof(uint64_t) * 2 * blocks, hipMemcpyDeviceToHost) != hipSuccess) return 3;
  double sum = 0.0, real = 0.0;
  for (int b = 0; b < blocks; ++b) {
    sum += static_cast<double>(host[2 * b]);
    real += static_cast<double>(host[2 * b + 1]);
  }
  *ticks_per_iter = sum / blocks / kIters;
  *ticks_per_realtime = real > 0.0 ? sum / real : 0.0;
  *iters = kIters;
  return 0;
}

}  // extern "C"
