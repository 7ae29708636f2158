// LDS-DMA convolution kernels for k = 11 convs of narrow layers (HiFiGAN's multi-receptive-
// field ResBlocks at 128, 64 and 32 channels; bf16 operand and weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps11(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  // (HiFiGAN's 256-channel stage stays on the register-staged kernel: 128.6 against 133.8 us on
  // these tiles, 334 workgroups of 16 waves)
  if (fp8 || p.k_splits > 1 || (p.n_cols > 64 && p.n_cols != 128)) return OMNI_ERR_UNSUPPORTED;
  // HiFiGAN's 128-channel stage in 64-column tiles (an 11-tap weight stage of 128 columns would
  // take 92 KB, twice over in the ring): 64 x 384 (16 waves of 32 x 48) or 64 x 256 (8 waves)
  if (p.n_cols == 128)
    return launch_first_fit<DmaConfig<2, 8, 2, 3, 496, 11, 1>,
                            DmaConfig<1, 8, 4, 2, 384, 11, 1>>(p, ch, stream);
  // 32 columns x 256 positions for a layer of one stage (c_in 32; 4 waves on a one-buffer ring,
  // three workgroups per CU: 202 / 286 us without / with the residual stream, 206 / 308 with
  // 8 waves of 32 x 512 and two per CU); 64 columns x 256 positions or 32 x 512 (an 11-tap
  // weight stage of 64 columns takes 46 KB)
  return launch_first_fit<DmaConfig<1, 4, 2, 4, 384, 11, 1, false, false, 3>,
                          DmaConfig<1, 8, 4, 2, 384, 11, 1>,
                          DmaConfig<1, 8, 2, 4, 640, 11, 1>>(p, ch, stream);
}

}  // namespace omni_conv
