// Plane kernels for _Float16 inputs and float outputs (see rbf_plane_impl.h).
#include "rbf_plane_impl.h"

namespace vectra {

hipError_t launch_plane_f16_f32(Problem& p, hipStream_t s) { return launch_plane_t<_Float16, float>(p, s); }

}  // namespace vectra
