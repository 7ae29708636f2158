// LDS-DMA convolution kernels for two-tap convs: the polyphase form of a ConvTranspose1d with
// kernel 2 * stride (bf16 operand; bf16 or E4M3 weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps2(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  // 192 columns x 192 positions, 16 waves of 48 x 48 (four per SIMD) or 8 of 96 x 48; 96 x 192,
  // 8 waves of 48 x 48 with two
  // chunks per stage; 96 x 384, 8 waves of 96 x 48 (up to 17 short rows of one halo row each)
  // (the same tiles for E4M3 weights)
  if (fp8)
    return launch_first_fit<DmaConfig<4, 4, 3, 3, 224, 2, 1, true>,
                            DmaConfig<2, 4, 6, 3, 224, 2, 1, true>,
                            DmaConfig<2, 4, 3, 3, 224, 2, 2, true>,
                            DmaConfig<1, 8, 6, 3, 432, 2, 1, true>>(p, ch, stream);
  return launch_first_fit<DmaConfig<4, 4, 3, 3, 224, 2, 1>,
                            DmaConfig<2, 4, 6, 3, 224, 2, 1>,
                            DmaConfig<2, 4, 3, 3, 224, 2, 2>,
                            DmaConfig<1, 8, 6, 3, 432, 2, 1>>(p, ch, stream);
}

}  // namespace omni_conv
