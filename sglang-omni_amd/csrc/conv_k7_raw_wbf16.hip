// Convolution kernels for up to 7 taps, bf16 input used as is, bf16 weights.
#include "conv_kernel.h"

namespace omni_conv {

template <>
int launch_taps7<IN_RAW, false>(const ConvParams& p, Choice& ch, hipStream_t stream) {
  return Configs<7>::launch<IN_RAW, false>(p, ch, stream);
}

}  // namespace omni_conv
