// Plane kernels for __bf16 inputs and float outputs (see rbf_plane_impl.h).
#include "rbf_plane_impl.h"

namespace vectra {

hipError_t launch_plane_bf16_f32(Problem& p, hipStream_t s) { return launch_plane_t<__bf16, float>(p, s); }

}  // namespace vectra
