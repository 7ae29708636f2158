// Conv from channels-last activations to one output channel (the decoder's last layer), with
// tanh or clamp, accumulated in float32 in one fixed order per position.
//
// A workgroup owns 256 consecutive positions of one row. Per 32-channel chunk it stages the
// positions [i0 - (taps-1), i0 + 256) in LDS as float32 with a 33-float row pitch (so the 64 lanes
// of a wave, one position each, read 64 distinct banks), then every thread accumulates its own
// position: chunk by chunk, tap by tap, channel by channel. That order depends on nothing but
// the position, so any split of positions or rows gives identical bits. The weights are read
// wave-uniformly and land in scalar registers.
#include "common.h"

namespace {

constexpr int kPositions = 256;
constexpr int kChunk = 32;
constexpr int kPitch = kChunk + 1;
constexpr int kMaxTaps = 16;

template <int DT>
__device__ __forceinline__ float load_act(const void* base, int64_t idx) {
  if constexpr (DT == OMNI_DTYPE_F32) return reinterpret_cast<const float*>(base)[idx];
  else if constexpr (DT == OMNI_DTYPE_BF16)
    return bits_to_float_bf16(reinterpret_cast<const u16*>(base)[idx]);
  else return bits_to_float_f16(reinterpret_cast<const u16*>(base)[idx]);
}

template <int DT>
__device__ __forceinline__ void store_val(void* base, int64_t idx, float v) {
  if constexpr (DT == OMNI_DTYPE_F32) reinterpret_cast<float*>(base)[idx] = v;
  else if constexpr (DT == OMNI_DTYPE_BF16)
    reinterpret_cast<u16*>(base)[idx] = float_to_bits_bf16(v);
  else reinterpret_cast<u16*>(base)[idx] = float_to_bits_f16(v);
}

struct SocParams {
  const void* x;
  int64_t x_sb, x_st, batch, length, channels;
  int ctx_in_buffer;
  const float* weight;
  const float* bias;
  int64_t taps, lpad;
  const u16* hist;
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_slots;
  int64_t hist_slot_stride;
  int hist_cold;
  int act;
  void* out;
  int64_t o_sb;
};

template <int XDT, int ODT>
__global__ void __launch_bounds__(kPositions) single_output_conv_kernel(const SocParams p) {
  __shared__ float xs[(kPositions + kMaxTaps - 1) * kPitch];
  const int tid = threadIdx.x;
  const int64_t tiles = (p.length + kPositions - 1) / kPositions;
  const int64_t b = blockIdx.x / tiles;
  const int64_t i0 = (blockIdx.x - b * tiles) * kPositions;
  const int64_t ctx = p.lpad;        // positions read left of i
  const int64_t rows = kPositions + p.taps - 1;
  const int64_t L = p.length;
  const int64_t C = p.channels;

  const u16* hist_read = nullptr;
  u16* hist_write = nullptr;
  const int64_t slot = p.hist != nullptr ? p.slot_index[b] : -1;
  if (slot >= 0 && slot < p.hist_slots) {
    const int64_t parity = p.slot_parity[slot] & 1;
    const u16* base = p.hist + slot * p.hist_slot_stride;
    hist_read = p.hist_cold ? nullptr : base + parity * ctx * C;
    hist_write = const_cast<u16*>(base) + (1 - parity) * ctx * C;
  }

  float acc = 0.f;
  const int64_t i = i0 + tid;
  for (int64_t c0 = 0; c0 < C; c0 += kChunk) {
    __syncthreads();
    for (int64_t e = tid; e < rows * kChunk; e += kPositions) {
      const int64_t r = e / kChunk;
      const int64_t c = c0 + (e - r * kChunk);
      const int64_t pos = i0 - ctx + r;
      float v = 0.f;
      if (c < C) {
        if (pos >= 0 && pos < L) {
          v = load_act<XDT>(p.x, b * p.x_sb + pos * p.x_st + c);
        } else if (pos < 0) {
          if (p.ctx_in_buffer) v = load_act<XDT>(p.x, b * p.x_sb + pos * p.x_st + c);
          else if (hist_read) v = bits_to_float_bf16(hist_read[(ctx + pos) * C + c]);
        }
        // History (streaming only, where ctx = taps - 1): the last ctx samples of history ++ x.
        if (hist_write != nullptr && pos >= L - ctx && pos < L &&
            ((pos >= i0 && pos < i0 + kPositions) || (i0 == 0 && pos < 0)))
          hist_write[(pos - (L - ctx)) * C + c] = float_to_bits_bf16(v);
      }
      xs[r * kPitch + (e - r * kChunk)] = v;
    }
    __syncthreads();
    const int64_t cn = (C - c0) < kChunk ? (C - c0) : kChunk;
    for (int64_t j = 0; j < p.taps; ++j) {
      const float* wrow = p.weight + j * C + c0;
      const float* xrow = xs + (tid + j) * kPitch;
      for (int64_t c = 0; c < cn; ++c) acc = __builtin_fmaf(wrow[c], xrow[c], acc);
    }
  }
  if (i < L) {
    const float v = acc + (p.bias ? p.bias[0] : 0.f);
    store_val<ODT>(p.out, b * p.o_sb + i, apply_act(p.act, v, 0.f, 0.f, 0.f));
  }
}

template <int XDT>
int launch_soc_x(const SocParams& p, int out_dtype, hipStream_t s, dim3 grid) {
  if (out_dtype == OMNI_DTYPE_F32)
    hipLaunchKernelGGL((single_output_conv_kernel<XDT, OMNI_DTYPE_F32>), grid, dim3(kPositions),
                       0, s, p);
  else if (out_dtype == OMNI_DTYPE_BF16)
    hipLaunchKernelGGL((single_output_conv_kernel<XDT, OMNI_DTYPE_BF16>), grid, dim3(kPositions),
                       0, s, p);
  else
    hipLaunchKernelGGL((single_output_conv_kernel<XDT, OMNI_DTYPE_F16>), grid, dim3(kPositions),
                       0, s, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

bool float_like(int dt) {
  return dt == OMNI_DTYPE_F32 || dt == OMNI_DTYPE_BF16 || dt == OMNI_DTYPE_F16;
}

}  // namespace

extern "C" int omni_single_output_conv(const void* x, int x_dtype, int64_t x_stride_b,
                                       int64_t x_stride_t, int64_t batch, int64_t length,
                                       int64_t channels, int context_in_buffer,
                                       const float* weight, const float* bias, int64_t taps,
                                       int64_t left_pad, const void* hist_pool, const int64_t* slot_index,
                                       const int64_t* slot_parity, int64_t hist_num_slots,
                                       int64_t hist_slot_stride, int history_cold, int activation,
                                       void* out, int out_dtype,
                                       int64_t out_stride_b, omni_stream_t stream) {
  if (!x || !weight || !out) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || length < 0 || channels < 1 || taps < 1 || taps > kMaxTaps)
    return OMNI_ERR_INVALID_ARG;
  if (left_pad < 0 || left_pad > taps - 1) return OMNI_ERR_INVALID_ARG;
  if (!float_like(x_dtype) || !float_like(out_dtype)) return OMNI_ERR_INVALID_ARG;
  if (activation != OMNI_ACTIVATION_NONE && activation != OMNI_ACTIVATION_TANH &&
      activation != OMNI_ACTIVATION_CLAMP)
    return OMNI_ERR_INVALID_ARG;
  if (x_stride_t < channels) return OMNI_ERR_INVALID_ARG;
  if (hist_pool) {
    if (context_in_buffer || !slot_index || !slot_parity || left_pad != taps - 1)
      return OMNI_ERR_INVALID_ARG;
    if (hist_slot_stride < 2 * (taps - 1) * channels || hist_num_slots < 1)
      return OMNI_ERR_INVALID_ARG;
  }
  if (batch == 0 || length == 0) return OMNI_OK;
  SocParams p{};
  p.x = x;
  p.x_sb = x_stride_b;
  p.x_st = x_stride_t;
  p.batch = batch;
  p.length = length;
  p.channels = channels;
  p.ctx_in_buffer = context_in_buffer;
  p.weight = weight;
  p.bias = bias;
  p.taps = taps;
  p.lpad = left_pad;
  p.hist = reinterpret_cast<const u16*>(hist_pool);
  p.slot_index = slot_index;
  p.slot_parity = slot_parity;
  p.hist_slots = hist_num_slots;
  p.hist_slot_stride = hist_slot_stride;
  p.hist_cold = history_cold;
  p.act = activation;
  p.out = out;
  p.o_sb = out_stride_b;
  const int64_t tiles = (length + kPositions - 1) / kPositions;
  if (batch * tiles > 0x7fffffffLL) return OMNI_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)(batch * tiles));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (x_dtype == OMNI_DTYPE_F32) return launch_soc_x<OMNI_DTYPE_F32>(p, out_dtype, s, grid);
  if (x_dtype == OMNI_DTYPE_BF16) return launch_soc_x<OMNI_DTYPE_BF16>(p, out_dtype, s, grid);
  return launch_soc_x<OMNI_DTYPE_F16>(p, out_dtype, s, grid);
}
