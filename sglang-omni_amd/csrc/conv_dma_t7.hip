// LDS-DMA convolution kernels for k = 7 convs (bf16 operand; bf16 or E4M3 weights).
#include "conv_dma.h"

namespace omni_conv {

int launch_dma_taps7(const ConvParams& p, bool fp8, Choice& ch, hipStream_t stream) {
  // 96 columns x 384 positions, 16 waves of 48 x 48 (four per SIMD: 0.97x the step time of 8
  // waves of 96 x 48 on the 24 kHz decoder, while one wave per SIMD of 96 x 96 took 1.07x), or
  // 8 waves of 96 x 48; 96 x 192, 8 waves of 48 x 48;
  // 96 x 192, 4 waves of 96 x 48 (staged rows: positions plus a halo of up to 54 per segment)
  // (the same tiles for E4M3 weights)
  if (fp8)
    return launch_first_fit<DmaConfig<2, 8, 3, 3, 496, 7, 1, true>,
                            DmaConfig<1, 8, 6, 3, 496, 7, 1, true>,
                            DmaConfig<2, 4, 3, 3, 368, 7, 1, true>,
                            DmaConfig<1, 4, 6, 3, 368, 7, 1, true>>(p, ch, stream);
  // narrow layers (HiFiGAN's 64- and 32-channel stages): 64 or 32 columns x 512 positions
  // (64 first: 13.99 against 14.18 ms per HiFiGAN call with 32 first, 14.48 on the
  // register-staged kernel)
  // (a layer of one stage, c_in 32, first: 32 columns x 256 positions, 4 waves, on a one-buffer
  // ring with four workgroups per CU)
  if (p.n_cols <= 64 && p.k_splits == 1 && !fp8)
    return launch_first_fit<DmaConfig<1, 4, 2, 4, 384, 7, 1, false, false, 4>,
                            DmaConfig<1, 8, 4, 4, 640, 7, 1>,
                            DmaConfig<1, 8, 2, 4, 640, 7, 1>>(p, ch, stream);
  // HiFiGAN's 128-channel stage: 128 columns x 192 positions, 8 waves of 64 x 48 (the ring fills
  // the 160 KiB)
  if (p.n_cols == 128 && p.k_splits == 1 && !fp8)
    return launch_first_fit<DmaConfig<2, 4, 4, 3, 288, 7, 1>>(p, ch, stream);
  if (p.k_splits > 1)  // split-K (bf16 weights): K slices of the 96 x 192 tiles (8 / 4 waves)
    return launch_first_fit<DmaConfig<2, 4, 3, 3, 368, 7, 1, false, true>,
                            DmaConfig<1, 4, 6, 3, 368, 7, 1, false, true>>(p, ch, stream);
  return launch_first_fit<DmaConfig<2, 8, 3, 3, 496, 7, 1>,
                            DmaConfig<1, 8, 6, 3, 496, 7, 1>,
                            DmaConfig<2, 4, 3, 3, 368, 7, 1>,
                            DmaConfig<1, 4, 6, 3, 368, 7, 1>>(p, ch, stream);
}

}  // namespace omni_conv
