// LDS-DMA convolution kernels for k = 3 convs of narrow layers (HiFiGAN's multi-receptive-
// field ResBlocks at 256, 128, 64 and 32 channels; bf16 operand and weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps3(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  if (fp8 || p.k_splits > 1 || (p.n_cols > 64 && p.n_cols % 128 != 0 && p.n_cols % 96 != 0))
    return OMNI_ERR_UNSUPPORTED;
  // HiFiGAN's 256- and 128-channel stages and its k = 3 transposed convs: 128 columns x 384
  // positions (16 waves of 64 x 48) or x 192 (8 waves) (the 128-channel convs 107 -> 104 us and
  // the 2 500-workgroup transposed conv 233 -> 195 us with 16 waves first)
  if (p.n_cols > 64 && p.n_cols % 128 == 0)
    return launch_first_fit<DmaConfig<2, 8, 4, 3, 496, 3, 1>,
                            DmaConfig<2, 4, 4, 3, 320, 3, 1>>(p, ch, stream);
  // other multiples of 96 columns (the 128 -> 64 transposed conv's three phases: 192 columns):
  // 96 x 384 (16 waves of 48 x 48) or 96 x 192 (8 waves)
  if (p.n_cols > 64)
    return launch_first_fit<DmaConfig<2, 8, 3, 3, 496, 3, 1>,
                            DmaConfig<2, 4, 3, 3, 368, 3, 1>>(p, ch, stream);
  // Layers of one stage first, on a one-buffer ring: 32 columns x 256 positions (c_in 32; 4
  // waves, four workgroups per CU: 151 / 274 us for the 32-channel stage's conv without / with
  // the residual stream, 158 / 286 with 8 waves of 32 x 512 and two per CU), 64 x 256 (c_in 64,
  // both chunks in the stage, 8 waves, two per CU); then 64 or 32 columns x 512 positions on the
  // two-buffer ring
  return launch_first_fit<DmaConfig<1, 4, 2, 4, 384, 3, 1, false, false, 4>,
                          DmaConfig<1, 8, 4, 2, 384, 3, 2, false, false, 2>,
                          DmaConfig<1, 8, 4, 4, 640, 3, 1>,
                          DmaConfig<1, 8, 2, 4, 640, 3, 1>>(p, ch, stream);
}

}  // namespace omni_conv
