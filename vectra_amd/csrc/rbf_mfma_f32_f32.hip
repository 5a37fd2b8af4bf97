// MFMA kernels for float inputs and float outputs (see rbf_mfma_impl.h).
#include "rbf_mfma_impl.h"

namespace vectra {

hipError_t launch_mfma_f32_f32(Problem& p, hipStream_t s) { return launch_mfma_t<float, float>(p, s); }

}  // namespace vectra
