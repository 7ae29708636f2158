// General Conv1d / ConvTranspose1d of channels-last activations: the shapes and dtypes of the
// reference's channels-last conv API that the MFMA kernels do not take (channel counts that are
// not multiples of 8 / 16, grouped and depthwise convs, any stride, dilation and zero padding,
// float32 / fp16 activations). One thread per output element, float32 accumulation in a fixed
// order (taps ascending, then the group's input channels ascending), rounded once.
//
// The thread's output channel is the fastest index, so a wave's threads read one input sample's
// channels (broadcast or contiguous) and one weight column per tap; weights are read in the
// reference's own layout through explicit strides ([C_out, C_in / g, k] for a conv, [C_in,
// C_out / g, k] for a transposed conv), so callers pass the module's weight as it is.
#include <type_traits>

#include "common.h"

namespace {

struct GeneralParams {
  const void* x;
  int64_t x_sb, x_st, x_sc;
  int64_t batch, length_in, c_in;
  const void* w;
  int64_t w_s0, w_s1, w_s2, taps;
  const void* bias;
  int64_t c_out, groups, stride, dilation, pad_left;
  void* y;
  int64_t y_sb, y_st, y_sc, length_out;
};

template <typename T>
__device__ __forceinline__ float load_as_float(const void* base, int64_t i) {
  if constexpr (std::is_same<T, float>::value) {
    return reinterpret_cast<const float*>(base)[i];
  } else if constexpr (std::is_same<T, __bf16>::value) {
    return bits_to_float_bf16(reinterpret_cast<const u16*>(base)[i]);
  } else {
    return bits_to_float_f16(reinterpret_cast<const u16*>(base)[i]);
  }
}

template <typename T>
__device__ __forceinline__ void store_from_float(void* base, int64_t i, float v) {
  if constexpr (std::is_same<T, float>::value) {
    reinterpret_cast<float*>(base)[i] = v;
  } else if constexpr (std::is_same<T, __bf16>::value) {
    reinterpret_cast<u16*>(base)[i] = float_to_bits_bf16(v);
  } else {
    reinterpret_cast<u16*>(base)[i] = float_to_bits_f16(v);
  }
}

template <typename T, bool TRANSPOSED>
__global__ void __launch_bounds__(256) conv_general_kernel(const GeneralParams p) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= p.batch * p.length_out * p.c_out) return;
  const int64_t co = idx % p.c_out;
  const int64_t rest = idx / p.c_out;
  const int64_t i = rest % p.length_out;
  const int64_t b = rest / p.length_out;
  const int64_t cout_g = p.c_out / p.groups;
  const int64_t cin_g = p.c_in / p.groups;
  const int64_t g = co / cout_g;
  const int64_t ci0 = g * cin_g;
  const int64_t col = co - g * cout_g;  // the output channel within its group
  float acc = p.bias ? load_as_float<T>(p.bias, co) : 0.f;
  const int64_t xb = b * p.x_sb;
  for (int64_t j = 0; j < p.taps; ++j) {
    int64_t pos;
    if constexpr (TRANSPOSED) {
      // output i gathers the inputs q with q * stride + j * dilation = i + pad_left
      const int64_t num = i + p.pad_left - j * p.dilation;
      if (num < 0 || num % p.stride != 0) continue;
      pos = num / p.stride;
    } else {
      pos = i * p.stride + j * p.dilation - p.pad_left;
    }
    if (pos < 0 || pos >= p.length_in) continue;
    const int64_t xo = xb + pos * p.x_st + ci0 * p.x_sc;
    for (int64_t c = 0; c < cin_g; ++c) {
      const int64_t wo = TRANSPOSED ? (ci0 + c) * p.w_s0 + col * p.w_s1 + j * p.w_s2
                                    : co * p.w_s0 + c * p.w_s1 + j * p.w_s2;
      acc = fmaf(load_as_float<T>(p.w, wo), load_as_float<T>(p.x, xo + c * p.x_sc), acc);
    }
  }
  store_from_float<T>(p.y, b * p.y_sb + i * p.y_st + co * p.y_sc, acc);
}

template <typename T>
int launch_general(const GeneralParams& p, bool transposed, hipStream_t stream) {
  const int64_t total = p.batch * p.length_out * p.c_out;
  const int64_t blocks = (total + 255) / 256;
  if (blocks > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  if (transposed)
    hipLaunchKernelGGL((conv_general_kernel<T, true>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, p);
  else
    hipLaunchKernelGGL((conv_general_kernel<T, false>), dim3((unsigned)blocks), dim3(256), 0,
                       stream, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_conv1d_general(const void* x, int dtype, int64_t batch, int64_t length_in,
                                   int64_t c_in, int64_t x_stride_b, int64_t x_stride_t,
                                   int64_t x_stride_c, const void* weight, int64_t taps,
                                   int64_t weight_stride0, int64_t weight_stride1,
                                   int64_t weight_stride2, const void* bias, int64_t c_out,
                                   int64_t groups, int64_t stride, int64_t dilation,
                                   int64_t pad_left, int transposed, void* y, int64_t length_out,
                                   int64_t y_stride_b, int64_t y_stride_t, int64_t y_stride_c,
                                   omni_stream_t stream) {
  if (!x || !weight || !y) return OMNI_ERR_INVALID_ARG;
  if (dtype != OMNI_DTYPE_F32 && dtype != OMNI_DTYPE_BF16 && dtype != OMNI_DTYPE_F16)
    return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || length_in < 0 || length_out < 0 || c_in < 1 || c_out < 1 || taps < 1 ||
      groups < 1 || stride < 1 || dilation < 1 || pad_left < 0)
    return OMNI_ERR_INVALID_ARG;
  if (c_in % groups || c_out % groups) return OMNI_ERR_INVALID_ARG;
  if (x_stride_b < 0 || x_stride_t < 0 || x_stride_c < 0 || y_stride_b < 0 || y_stride_t < 0 ||
      y_stride_c < 0 || weight_stride0 < 0 || weight_stride1 < 0 || weight_stride2 < 0)
    return OMNI_ERR_INVALID_ARG;
  if (batch == 0 || length_out == 0) return OMNI_OK;
  GeneralParams p{x, x_stride_b, x_stride_t, x_stride_c, batch, length_in, c_in,
                  weight, weight_stride0, weight_stride1, weight_stride2, taps, bias,
                  c_out, groups, stride, dilation, pad_left, y, y_stride_b, y_stride_t,
                  y_stride_c, length_out};
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_F32) return launch_general<float>(p, transposed != 0, s);
  if (dtype == OMNI_DTYPE_BF16) return launch_general<__bf16>(p, transposed != 0, s);
  return launch_general<_Float16>(p, transposed != 0, s);
}
