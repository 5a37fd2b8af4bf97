// Plane kernels for __bf16 inputs and __bf16 outputs (see rbf_plane_impl.h).
#include "rbf_plane_impl.h"

namespace vectra {

hipError_t launch_plane_bf16_bf16(Problem& p, hipStream_t s) { return launch_plane_t<__bf16, __bf16>(p, s); }

}  // namespace vectra
