// Fused residual-unit kernels (conv k <= 7 -> activation -> conv k = 1) for 96 and 192 channels,
// fp8-e4m3 weights.
#include "conv_kernel.h"

namespace omni_conv {

namespace {
template <typename Cfg>
int launch_mode(const ConvParams& p, int in_mode, hipStream_t stream) {
  if (in_mode == IN_RAW) return Cfg::template launch<IN_RAW, true, true>(p, stream);
  if (in_mode == IN_ACT) return Cfg::template launch<IN_ACT, true, true>(p, stream);
  return Cfg::template launch<IN_F32, true, true>(p, stream);
}
}  // namespace

template <>
int launch_fused<true>(const ConvParams& p, int in_mode, hipStream_t stream) {
  if (p.n_cols == 96) {
    if (ResidualUnit96::fits(p, true)) return launch_mode<ResidualUnit96>(p, in_mode, stream);
    if (ResidualUnit96Short::fits(p, true))
      return launch_mode<ResidualUnit96Short>(p, in_mode, stream);
  }
  if (p.n_cols == 192) {
    if (ResidualUnit192::fits(p, true)) return launch_mode<ResidualUnit192>(p, in_mode, stream);
    if (ResidualUnit192Short::fits(p, true))
      return launch_mode<ResidualUnit192Short>(p, in_mode, stream);
  }
  return OMNI_ERR_UNSUPPORTED;
}

}  // namespace omni_conv
