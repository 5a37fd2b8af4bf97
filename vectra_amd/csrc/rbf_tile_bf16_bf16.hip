// Tile kernels for __bf16 inputs and __bf16 outputs (see rbf_tile_impl.h).
#include "rbf_tile_impl.h"

namespace vectra {

hipError_t launch_tile_bf16_bf16(Problem& p, hipStream_t s) { return launch_tile_t<__bf16, __bf16>(p, s); }

}  // namespace vectra
