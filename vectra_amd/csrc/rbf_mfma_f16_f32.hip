// MFMA kernels for _Float16 inputs and float outputs (see rbf_mfma_impl.h).
#include "rbf_mfma_impl.h"

namespace vectra {

hipError_t launch_mfma_f16_f32(Problem& p, hipStream_t s) { return launch_mfma_t<_Float16, float>(p, s); }

}  // namespace vectra
