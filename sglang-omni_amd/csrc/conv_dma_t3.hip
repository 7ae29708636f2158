// LDS-DMA convolution kernels for k = 3 convs of narrow layers (HiFiGAN's multi-receptive-
// field ResBlocks at 64 and 32 channels; bf16 operand and weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps3(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  // 64 or 32 columns x 512 positions
  if (fp8 || p.k_splits > 1 || p.n_cols > 64) return OMNI_ERR_UNSUPPORTED;
  return launch_first_fit<DmaConfig<1, 8, 4, 4, 640, 3, 1>,
                          DmaConfig<1, 8, 2, 4, 640, 3, 1>>(p, ch, stream);
}

}  // namespace omni_conv
