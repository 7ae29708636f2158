// Residual-stack kernel, fp8 (E4M3) weights: the tiled form and the sweep form (long rows), both
// with the weights' bytes staged by LDS DMA and widened to bf16 when read.
#include "residual_stack.h"

namespace omni_stack {

template <>
int launch_stack96<true>(const StackParams& p, int grid, bool sweep, hipStream_t stream) {
  if (sweep) {
    auto k = residual_stack_kernel<96, 1, 8, 3, true, true>;
    static const bool raised = omni_conv::raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(Stack96Sweep8::NT), Stack96Sweep8::lds_bytes(),
                       stream, p);
  } else {
    auto k = residual_stack_kernel<96, 1, 8, 3, true, false>;
    static const bool raised = omni_conv::raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(Stack96Dma8::NT), Stack96Dma8::lds_bytes(),
                       stream, p);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace omni_stack
