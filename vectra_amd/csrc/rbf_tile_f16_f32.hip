// Tile kernels for _Float16 inputs and float outputs (see rbf_tile_impl.h).
#include "rbf_tile_impl.h"

namespace vectra {

hipError_t launch_tile_f16_f32(Problem& p, hipStream_t s) { return launch_tile_t<_Float16, float>(p, s); }

}  // namespace vectra
