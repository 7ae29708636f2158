// Convolution kernels for up to 7 taps, input activated while staged (bf16 or float32 input),
// bf16 weights.
#include "conv_kernel.h"

namespace omni_conv {

template <>
int launch_taps7<IN_ACT, false>(const ConvParams& p, Choice& ch, hipStream_t stream) {
  return Configs<7>::launch<IN_ACT, false>(p, ch, stream);
}

template <>
int launch_taps7<IN_F32, false>(const ConvParams& p, Choice& ch, hipStream_t stream) {
  return Configs<7>::launch<IN_F32, false>(p, ch, stream);
}

}  // namespace omni_conv
