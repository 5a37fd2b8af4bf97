// Host-side launchers of the RBF-attention kernels (internal to the library).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace vectra {

struct Problem;

// Multiplier and shift for fast_div (division of 31-bit values by d >= 1).
void make_fast_div(int64_t d, uint32_t* mul, uint32_t* shift);

// Stream kernel: requires unit element stride in d for q, k, v and out,
// 16-byte-aligned rows, D == Dv == chunks * (16 / sizeof(input element)),
// chunks in {2, 4, 8, 16}.
hipError_t launch_stream(Problem& p, int in_dtype, int out_dtype, int chunks, hipStream_t s);

// Generic kernel: any strides and sizes.  Its grid has one row of
// workgroups per 256-column slice of Dv, at most this many.
constexpr int64_t kMaxGenericSlices = 65535;
hipError_t launch_generic(Problem& p, int in_dtype, int out_dtype, hipStream_t s);

// MFMA kernel: bf16/fp16/fp32 inputs, output in the input dtype or fp32,
// D == Dv in {16, 32, 64, 128}, unit d stride, 16-byte rows, Nk >= 1.
bool mfma_supports(const Problem& p, int in_dtype, int out_dtype);
hipError_t launch_mfma(Problem& p, int in_dtype, int out_dtype, hipStream_t s);

// Plane kernel (one workgroup per (b, h) plane): bf16/fp16/fp32 inputs, output
// in the input dtype or fp32, D == Dv in {16, 32}, Nq and Nk both <= 80
// (<= 128 for 16-dim heads), unit d stride, 16-byte-aligned rows, K and V
// rows that do not overlap.
bool plane_supports(const Problem& p, int in_dtype, int out_dtype);
hipError_t launch_plane(Problem& p, int in_dtype, int out_dtype, hipStream_t s);

// Tile kernel (key tiles streamed through LDS, 32 query rows per wave):
// bf16/fp16 inputs, output in the input dtype or fp32, D == Dv in
// {32, 64, 128}, unit d stride, 16-byte-aligned rows.
bool tile_supports(const Problem& p, int in_dtype, int out_dtype);
hipError_t launch_tile(Problem& p, int in_dtype, int out_dtype, hipStream_t s);

hipError_t launch_squared_norms(const void* x, int dtype, int64_t B, int64_t H, int64_t N,
                                int64_t D, const int64_t* strides, float* out, hipStream_t s);

}  // namespace vectra
