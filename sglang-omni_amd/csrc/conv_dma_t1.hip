// LDS-DMA convolution kernels for k = 1 convs (bf16 operand; bf16 or E4M3 weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps1(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  // 192 columns x 192 positions, 16 waves of 48 x 48 (four per SIMD) or 8 of 96 x 48, with two
  // chunks per stage (16 waves with the transposed convs': DAC step 0.985x); 96 x 192, 8 waves
  // of 48 x 48 with three chunks per stage; 96 x 256, 8 waves of 96 x 32
  // (the same tiles for E4M3 weights)
  if (fp8)
    return launch_first_fit<DmaConfig<4, 4, 3, 3, 192, 1, 2, true>,
                            DmaConfig<2, 4, 6, 3, 192, 1, 2, true>,
                            DmaConfig<2, 4, 3, 3, 192, 1, 3, true>,
                            DmaConfig<1, 8, 6, 2, 256, 1, 2, true>>(p, ch, stream);
  if (p.k_splits > 1)  // split-K (bf16 weights): the same tiles, each a K slice of a tile
    return launch_first_fit<DmaConfig<4, 4, 3, 3, 192, 1, 2, false, true>,
                            DmaConfig<2, 4, 6, 3, 192, 1, 2, false, true>,
                            DmaConfig<2, 4, 3, 3, 192, 1, 3, false, true>,
                            DmaConfig<1, 8, 6, 2, 256, 1, 2, false, true>>(p, ch, stream);
  return launch_first_fit<DmaConfig<4, 4, 3, 3, 192, 1, 2>,
                            DmaConfig<2, 4, 6, 3, 192, 1, 2>,
                            DmaConfig<2, 4, 3, 3, 192, 1, 3>,
                            DmaConfig<1, 8, 6, 2, 256, 1, 2>>(p, ch, stream);
}

}  // namespace omni_conv
