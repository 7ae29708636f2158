/*
 * C restatement of the integer/index and direct-summation parts of the codec decode path.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ to pin the PyTorch oracle (codec_oracle.py); the
 * product never links or calls it. Compiled with -ffp-contract=off so every float32 add is a
 * separate IEEE add.
 *
 *   oracle_rvq_gather_sum   sum_k E_k[codes[b,k,t]] in float32, k = 0..K-1 from 0.0 (the
 *                           sequential order of TF/models/dac/modeling_dac.py:362-371 and
 *                           sglang_omni/models/personaplex/components/mimi.py:275-280); codes
 *                           clamped to V-1 as rvq.py:374-388 does.
 *   oracle_conv1d_f64       y[b,co,t] = bias[co] + sum_{ci,j} W[co,ci,j] x[b,ci,t + j*d - lpad]
 *                           by direct summation in double (zeros outside [0, L)).
 *   oracle_conv_transpose1d_f64
 *                           y[b,co,s*i + j - pad] += W[ci,co,j] x[b,ci,i] by scatter in double,
 *                           outputs in [0, L_out).
 */
#include <stdint.h>

void oracle_rvq_gather_sum(const int64_t* codes, int64_t batch, int64_t k, int64_t frames,
                           const float* tables, int64_t v, int64_t d, float* out, int clamp) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t t = 0; t < frames; ++t)
      for (int64_t e = 0; e < d; ++e) {
        float acc = 0.0f;
        for (int64_t q = 0; q < k; ++q) {
          int64_t c = codes[(b * k + q) * frames + t];
          if (clamp && c > v - 1) c = v - 1;
          acc = acc + tables[(q * v + c) * d + e];
        }
        out[(b * d + e) * frames + t] = acc;
      }
}

void oracle_conv1d_f64(const double* x, int64_t batch, int64_t c_in, int64_t length,
                       const double* w, const double* bias, int64_t c_out, int64_t taps,
                       int64_t dilation, int64_t left_pad, double* y) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t co = 0; co < c_out; ++co)
      for (int64_t t = 0; t < length; ++t) {
        double acc = bias ? bias[co] : 0.0;
        for (int64_t ci = 0; ci < c_in; ++ci)
          for (int64_t j = 0; j < taps; ++j) {
            const int64_t p = t + j * dilation - left_pad;
            if (p >= 0 && p < length)
              acc += w[(co * c_in + ci) * taps + j] * x[(b * c_in + ci) * length + p];
          }
        y[(b * c_out + co) * length + t] = acc;
      }
}

void oracle_conv_transpose1d_f64(const double* x, int64_t batch, int64_t c_in, int64_t length,
                                 const double* w, const double* bias, int64_t c_out, int64_t taps,
                                 int64_t stride, int64_t padding, int64_t out_length, double* y) {
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t co = 0; co < c_out; ++co)
      for (int64_t o = 0; o < out_length; ++o) y[(b * c_out + co) * out_length + o] = bias ? bias[co] : 0.0;
  for (int64_t b = 0; b < batch; ++b)
    for (int64_t ci = 0; ci < c_in; ++ci)
      for (int64_t i = 0; i < length; ++i)
        for (int64_t co = 0; co < c_out; ++co)
          for (int64_t j = 0; j < taps; ++j) {
            const int64_t o = stride * i + j - padding;
            if (o >= 0 && o < out_length)
              y[(b * c_out + co) * out_length + o] +=
                  w[(ci * c_out + co) * taps + j] * x[(b * c_in + ci) * length + i];
          }
}
