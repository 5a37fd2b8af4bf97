// Plane kernels for fp32 inputs and outputs (see rbf_plane32_impl.h).
#include "rbf_plane32_impl.h"

namespace vectra {

hipError_t launch_plane_f32_f32(Problem& p, hipStream_t s) {
  switch (p.D) {
    case 16: return launch_plane32_d<16>(p, s);
    case 32: return launch_plane32_d<32>(p, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace vectra
