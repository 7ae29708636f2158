// Convolution kernels for up to 7 taps, bf16 input used as is, fp8-e4m3 weights.
#include "conv_kernel.h"

namespace omni_conv {

template <>
int launch_taps7<IN_RAW, true>(const ConvParams& p, Choice& ch, hipStream_t stream) {
  return Configs<7>::launch<IN_RAW, true>(p, ch, stream);
}

}  // namespace omni_conv
