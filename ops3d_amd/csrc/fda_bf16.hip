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

}  // namespace ops3d_fda
