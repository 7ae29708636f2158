// Residual-stack kernel, bf16 weights: the tiled form and the sweep form (long rows).
#include "residual_stack.h"

namespace omni_stack {

template <>
int launch_stack96<false>(const StackParams& p, int grid, bool sweep, hipStream_t stream) {
  if (sweep) {
    auto k = residual_stack_kernel<96, 1, 8, 3, false, true>;
    static const bool raised = omni_conv::raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(Stack96Sweep::NT), Stack96Sweep::lds_bytes(),
                       stream, p);
  } else {
    auto k = residual_stack_kernel<96, 1, 8, 3, false, false>;
    static const bool raised = omni_conv::raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(Stack96Dma::NT), Stack96Dma::lds_bytes(),
                       stream, p);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace omni_stack
