// Convolution kernels for up to 11 taps (the HiFiGAN k = 11 resblocks), bf16 input (as is or
// activated while staged) and bf16 weights.
#include "conv_kernel.h"

namespace omni_conv {

int launch_taps11(const ConvParams& p, int in_mode, Choice& ch, hipStream_t stream) {
  if (in_mode == IN_RAW) return Configs<11>::launch<IN_RAW, false>(p, ch, stream);
  if (in_mode == IN_ACT) return Configs<11>::launch<IN_ACT, false>(p, ch, stream);
  return OMNI_ERR_UNSUPPORTED;
}

}  // namespace omni_conv
