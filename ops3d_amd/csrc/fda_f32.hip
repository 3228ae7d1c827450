// Kernel instantiations for element type float (channels per lane 4 or 6).
#include "fda_kernels.h"

namespace ops3d_fda {

hipError_t launch_f32(int which, int cpl, int lpu, const Args &a, unsigned grid, size_t lds,
                     hipStream_t st) {
  switch (cpl) {
    case 4: return launch_cpl<float, 4>(which, lpu, a, grid, lds, st);
    case 6: return launch_cpl<float, 6>(which, lpu, a, grid, lds, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace ops3d_fda
