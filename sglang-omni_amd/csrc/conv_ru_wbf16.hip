// Fused residual-unit kernels (conv k <= 7 -> activation -> conv k = 1) for 96 and 192 channels,
// bf16 weights.
#include "conv_dma_fused.h"

namespace omni_conv {

template <>
int launch_fused<false>(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream) {
  if (p.n_cols == 96)
    return launch_fused_list<false, void, ResidualUnit96, ResidualUnit96Short>(p, in_mode, ch, stream);
  if (p.n_cols == 192)
    return launch_fused_list<false, FusedDmaConfig, ResidualUnit192, ResidualUnit192Short>(
        p, in_mode, ch, stream);
  return OMNI_ERR_UNSUPPORTED;
}

}  // namespace omni_conv
