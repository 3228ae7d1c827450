// Kernel instantiations for element type __bf16 (channels per lane 8 or 12).
#include "fda_kernels.h"

namespace ops3d_fda {

hipError_t launch_bf16(int which, int cpl, int lpu, const Args &a, unsigned grid, size_t lds,
                     hipStream_t st) {
  switch (cpl) {
    case 8: return launch_cpl<__bf16, 8>(which, lpu, a, grid, lds, st);
    case 12: return launch_cpl<__bf16, 12>(which, lpu, a, grid, lds, st);
    default: return hipErrorInvalidValue;
  }
}

// Resident blocks per CU of the tile-major backward's tile kernel (the f16 instance has the same
// resources).
int fused_tile_blocks_per_cu() {
  int occ = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, fda_bwd_fused_tile_kernel<__bf16, false>, kFusedThreads,
                                                   fused_tile_lds_bytes()) != hipSuccess)
    return 0;
  return occ;
}

}  // namespace ops3d_fda
