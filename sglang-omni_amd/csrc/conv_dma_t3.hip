// LDS-DMA convolution kernels for k = 3 convs of narrow layers (HiFiGAN's multi-receptive-
// field ResBlocks at 128, 64 and 32 channels; bf16 operand and weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps3(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  if (fp8 || p.k_splits > 1 || (p.n_cols > 64 && p.n_cols != 128)) return OMNI_ERR_UNSUPPORTED;
  if (p.n_cols == 128)  // 128 columns x 192 positions, 8 waves of 64 x 48
    return launch_first_fit<DmaConfig<2, 4, 4, 3, 320, 3, 1>>(p, ch, stream);
  // Layers of one stage first, two workgroups per CU on a one-buffer ring: 32 columns x 512
  // positions (c_in 32), 64 x 256 (c_in 64, both chunks in the stage); then 64 or 32 columns x
  // 512 positions on the two-buffer ring
  return launch_first_fit<DmaConfig<1, 8, 2, 4, 640, 3, 1, false, false, true>,
                          DmaConfig<1, 8, 4, 2, 384, 3, 2, false, false, true>,
                          DmaConfig<1, 8, 4, 4, 640, 3, 1>,
                          DmaConfig<1, 8, 2, 4, 640, 3, 1>>(p, ch, stream);
}

}  // namespace omni_conv
