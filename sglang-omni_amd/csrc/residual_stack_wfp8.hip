// Residual-stack kernel, fp8 weights.
#include "residual_stack.h"

namespace omni_stack {

template <>
int launch_stack96<true>(const StackParams& p, int grid, bool sweep, hipStream_t stream) {
  if (sweep) return OMNI_ERR_UNSUPPORTED;  // the sweep runs the LDS-DMA (bf16) form only
  auto k = residual_stack_kernel<96, 1, 8, 2, true, false, false>;
  static const bool raised = omni_conv::raise_lds_limit((const void*)k);
  (void)raised;
  hipLaunchKernelGGL(k, dim3((unsigned)grid), dim3(Stack96::NT), Stack96::lds_bytes(), stream, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace omni_stack
