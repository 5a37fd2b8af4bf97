// Tile kernels for _Float16 inputs and _Float16 outputs (see rbf_tile_impl.h).
#include "rbf_tile_impl.h"

namespace vectra {

hipError_t launch_tile_f16_f16(Problem& p, hipStream_t s) { return launch_tile_t<_Float16, _Float16>(p, s); }

}  // namespace vectra
