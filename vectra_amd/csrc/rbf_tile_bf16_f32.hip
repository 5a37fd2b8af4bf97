// Tile kernels for __bf16 inputs and float outputs (see rbf_tile_impl.h).
#include "rbf_tile_impl.h"

namespace vectra {

hipError_t launch_tile_bf16_f32(Problem& p, hipStream_t s) { return launch_tile_t<__bf16, float>(p, s); }

}  // namespace vectra
