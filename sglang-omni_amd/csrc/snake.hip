// Elementwise Snake family kernels with the reference's rounding conventions:
//   * bias_snake_beta: SnakeBeta(conv + bias [+ residual]) rounding after every op, the eager
//     bf16/fp16 op chain the reference's fused kernel reproduces;
//   * snake: Snake1d / SnakeBeta in float32, rounded once (round_intermediates = 0), or the
//     eager chain (round_intermediates = 1).
// Both are HBM-bound and use the device library's sinf, whose float32 result the rounding to
// bf16/fp16 then absorbs.
#include "common.h"

// The eager op chain rounds after every op: no multiply-add contraction in this file.
#pragma clang fp contract(off)

namespace {

template <int DT>
__device__ __forceinline__ float ld(const void* p, int64_t i) {
  if constexpr (DT == OMNI_DTYPE_F32) return reinterpret_cast<const float*>(p)[i];
  else if constexpr (DT == OMNI_DTYPE_BF16)
    return bits_to_float_bf16(reinterpret_cast<const u16*>(p)[i]);
  else return bits_to_float_f16(reinterpret_cast<const u16*>(p)[i]);
}
template <int DT>
__device__ __forceinline__ void st(void* p, int64_t i, float v) {
  if constexpr (DT == OMNI_DTYPE_F32) reinterpret_cast<float*>(p)[i] = v;
  else if constexpr (DT == OMNI_DTYPE_BF16) reinterpret_cast<u16*>(p)[i] = float_to_bits_bf16(v);
  else reinterpret_cast<u16*>(p)[i] = float_to_bits_f16(v);
}
template <int DT>
__device__ __forceinline__ float rnd(float v) {
  if constexpr (DT == OMNI_DTYPE_F32) return v;
  else if constexpr (DT == OMNI_DTYPE_BF16) return bits_to_float_bf16(float_to_bits_bf16(v));
  else return bits_to_float_f16(float_to_bits_f16(v));
}

template <int DT, int PDT>
__global__ void bias_snake_beta_kernel(const void* conv, int64_t conv_sb, int64_t batch,
                                       int64_t length, int64_t channels, const void* bias,
                                       const void* alpha_scale, const void* inverse_beta,
                                       const void* residual, void* sum_out, void* out,
                                       int64_t out_sb) {
  const int64_t per_row = length * channels;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= batch * per_row) return;
  const int64_t b = idx / per_row;
  const int64_t off = idx - b * per_row;
  const int64_t c = off % channels;
  float total = rnd<DT>(ld<DT>(conv, b * conv_sb + off) + (bias ? ld<PDT>(bias, c) : 0.f));
  if (residual) total = rnd<DT>(total + ld<DT>(residual, idx));
  if (sum_out) st<DT>(sum_out, idx, total);
  const float phase = rnd<DT>(total * ld<PDT>(alpha_scale, c));
  const float sine = rnd<DT>(sinf(phase));
  const float sq = rnd<DT>(sine * sine);
  const float scaled = rnd<DT>(ld<PDT>(inverse_beta, c) * sq);
  st<DT>(out, b * out_sb + off, total + scaled);
}

template <int DT>
__global__ void snake_kernel(const void* x, void* y, int64_t n, int64_t channels, int64_t frames,
                             int channels_last, const float* a, const float* bcoef,
                             int round_intermediates) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int64_t c = channels_last ? idx % channels : (idx / frames) % channels;
  const float v = ld<DT>(x, idx);
  float out;
  if (round_intermediates) {
    const float phase = rnd<DT>(v * a[c]);
    const float sine = rnd<DT>(sinf(phase));
    const float sq = rnd<DT>(sine * sine);
    const float scaled = rnd<DT>(bcoef[c] * sq);
    out = v + scaled;
  } else {
    const float s = sinf(a[c] * v);
    out = v + bcoef[c] * (s * s);
  }
  st<DT>(y, idx, out);
}

// SnakeBeta from the module's raw log-scale parameters, read at every launch (a captured graph
// sees the parameters' current values), with the eager op chain's rounding in DT:
//   a = rnd(exp(alpha)), e = rnd(exp(beta)), t = rnd(e + eps), r = rnd(1 / t)
//   y = rnd(x + rnd(r * rnd(rnd(sin(rnd(x * a)))^2)))
// Layout: [B, C, T] contiguous, or (channels_last) its [B, T, C] transpose contiguous; y has
// x's layout. Each thread takes consecutive elements of one row, so loads and stores coalesce
// in both layouts.
template <int DT, int PDT>
__global__ void __launch_bounds__(256) snake_beta_params_kernel(
    const void* x, void* y, int64_t n, int64_t channels, int64_t frames, int channels_last,
    const void* alpha, const void* beta, float eps) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= n) return;
  const int64_t c = channels_last ? idx % channels : (idx / frames) % channels;
  const float a = rnd<DT>(expf(ld<PDT>(alpha, c)));
  const float e = rnd<DT>(expf(ld<PDT>(beta, c)));
  const float t = rnd<DT>(e + eps);
  const float r = rnd<DT>(1.0f / t);
  const float v = ld<DT>(x, idx);
  const float phase = rnd<DT>(v * a);
  const float sine = rnd<DT>(sinf(phase));
  const float sq = rnd<DT>(sine * sine);
  const float scaled = rnd<DT>(r * sq);
  st<DT>(y, idx, v + scaled);
}

bool half_like(int dt) { return dt == OMNI_DTYPE_BF16 || dt == OMNI_DTYPE_F16; }

template <int DT>
int launch_bsb(const void* conv, int64_t conv_sb, int64_t batch, int64_t length,
               int64_t channels, const void* bias, const void* alpha_scale,
               const void* inverse_beta, int param_dtype, const void* residual, void* sum_out,
               void* out, int64_t out_sb, hipStream_t s) {
  const int64_t n = batch * length * channels;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  if (param_dtype == OMNI_DTYPE_F32)
    hipLaunchKernelGGL((bias_snake_beta_kernel<DT, OMNI_DTYPE_F32>), grid, block, 0, s, conv,
                       conv_sb, batch, length, channels, bias, alpha_scale, inverse_beta, residual,
                       sum_out, out, out_sb);
  else if (param_dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL((bias_snake_beta_kernel<DT, OMNI_DTYPE_BF16>), grid, block, 0, s, conv,
                       conv_sb, batch, length, channels, bias, alpha_scale, inverse_beta, residual,
                       sum_out, out, out_sb);
  else
    hipLaunchKernelGGL((bias_snake_beta_kernel<DT, OMNI_DTYPE_F16>), grid, block, 0, s, conv,
                       conv_sb, batch, length, channels, bias, alpha_scale, inverse_beta, residual,
                       sum_out, out, out_sb);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_bias_snake_beta(const void* conv, int64_t conv_stride_b, int64_t batch,
                                    int64_t length, int64_t channels, const void* bias,
                                    const void* alpha_scale, const void* inverse_beta,
                                    int param_dtype, const void* residual, void* sum_out,
                                    void* out, int64_t out_stride_b, int dtype,
                                    omni_stream_t stream) {
  if (!conv || !alpha_scale || !inverse_beta || !out) return OMNI_ERR_INVALID_ARG;
  if (!half_like(dtype)) return OMNI_ERR_INVALID_ARG;
  if (param_dtype != OMNI_DTYPE_F32 && param_dtype != dtype) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || length < 0 || channels < 1) return OMNI_ERR_INVALID_ARG;
  if (conv_stride_b < length * channels || out_stride_b < length * channels)
    return OMNI_ERR_INVALID_ARG;
  if (batch * length == 0) return OMNI_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_BF16)
    return launch_bsb<OMNI_DTYPE_BF16>(conv, conv_stride_b, batch, length, channels, bias,
                                       alpha_scale, inverse_beta, param_dtype, residual, sum_out,
                                       out, out_stride_b, s);
  return launch_bsb<OMNI_DTYPE_F16>(conv, conv_stride_b, batch, length, channels, bias,
                                    alpha_scale, inverse_beta, param_dtype, residual, sum_out,
                                    out, out_stride_b, s);
}

extern "C" int omni_snake(const void* x, void* y, int dtype, int64_t batch, int64_t frames,
                          int64_t channels, int channels_last, const float* a, const float* b,
                          int round_intermediates, omni_stream_t stream) {
  if (!x || !y || !a || !b) return OMNI_ERR_INVALID_ARG;
  if (dtype != OMNI_DTYPE_F32 && !half_like(dtype)) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || frames < 0 || channels < 1) return OMNI_ERR_INVALID_ARG;
  const int64_t n = batch * frames * channels;
  if (n == 0) return OMNI_OK;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_F32)
    hipLaunchKernelGGL(snake_kernel<OMNI_DTYPE_F32>, grid, block, 0, s, x, y, n, channels, frames,
                       channels_last, a, b, round_intermediates);
  else if (dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL(snake_kernel<OMNI_DTYPE_BF16>, grid, block, 0, s, x, y, n, channels,
                       frames, channels_last, a, b, round_intermediates);
  else
    hipLaunchKernelGGL(snake_kernel<OMNI_DTYPE_F16>, grid, block, 0, s, x, y, n, channels, frames,
                       channels_last, a, b, round_intermediates);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

extern "C" int omni_snake_beta(const void* x, void* y, int dtype, int64_t batch, int64_t channels,
                               int64_t frames, int channels_last, const void* alpha,
                               const void* beta, int param_dtype, float eps,
                               omni_stream_t stream) {
  if (!x || !y || !alpha || !beta) return OMNI_ERR_INVALID_ARG;
  if (!half_like(dtype) || param_dtype != dtype) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || frames < 0 || channels < 1) return OMNI_ERR_INVALID_ARG;
  const int64_t n = batch * frames * channels;
  if (n == 0) return OMNI_OK;
  const int64_t blocks = (n + 255) / 256;
  if (blocks > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL((snake_beta_params_kernel<OMNI_DTYPE_BF16, OMNI_DTYPE_BF16>),
                       dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, channels, frames,
                       channels_last, alpha, beta, eps);
  else
    hipLaunchKernelGGL((snake_beta_params_kernel<OMNI_DTYPE_F16, OMNI_DTYPE_F16>),
                       dim3((unsigned)blocks), dim3(256), 0, s, x, y, n, channels, frames,
                       channels_last, alpha, beta, eps);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}
