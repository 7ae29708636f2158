// Waveform egress: a decode step's float32 waveform rows packed into one buffer for a single
// device-to-host copy, either as float32 (the relay payload's "audio_waveform" samples,
// utils/audio_payload.py:40-55) or as signed 16-bit PCM (the realtime output encoding,
// serve/realtime/session_bridge.py:86-88: clip to [-1, 1], times 32767 in float32, truncated
// toward zero). PCM halves the bytes that cross PCIe.
//
// One thread writes 8 consecutive samples of a row: two 16-byte loads and one 16-byte (PCM) or
// two 16-byte (float32) stores when the row and both strides keep 16-byte alignment, element
// loads and stores otherwise. Rows may stop early (row_samples); samples past a row's count are
// not written.
#include "common.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 8;

struct EgressParams {
  const float* wave;
  int64_t wave_stride;  // elements between rows
  int64_t samples;      // the longest row
  const int64_t* row_samples;  // per-row counts (nullable)
  void* out;
  int64_t out_stride;  // elements between rows
  int64_t chunks_per_row;
};

// numpy's float32 -> int16 conversion of a clipped sample: truncation toward zero; NaN (which
// np.clip passes through) converts to 0.
OMNI_DEVICE int16_t pcm16_sample(float v) {
  if (v != v) return 0;
  v = fminf(fmaxf(v, -1.f), 1.f);
  return (int16_t)(int)(v * 32767.f);
}

template <int FORMAT, bool VEC>
__global__ __launch_bounds__(kThreads) void waveform_egress_kernel(EgressParams p) {
  const int64_t chunk = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (chunk >= p.chunks_per_row) return;
  const int64_t row = blockIdx.y;
  int64_t n = p.samples;
  if (p.row_samples) n = min(n, max(p.row_samples[row], (int64_t)0));
  const int64_t s0 = chunk * kPerThread;
  if (s0 >= n) return;
  const float* src = p.wave + row * p.wave_stride + s0;
  float v[kPerThread];
  const bool whole = VEC && s0 + kPerThread <= n;
  if (whole) {
    const float4 a = *reinterpret_cast<const float4*>(src);
    const float4 b = *reinterpret_cast<const float4*>(src + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
    v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < kPerThread; ++i) v[i] = s0 + i < n ? src[i] : 0.f;
  }
  if (FORMAT == OMNI_EGRESS_PCM16) {
    int16_t* dst = static_cast<int16_t*>(p.out) + row * p.out_stride + s0;
    if (whole) {
      uint32_t w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = (uint32_t)(uint16_t)pcm16_sample(v[2 * i]) |
               ((uint32_t)(uint16_t)pcm16_sample(v[2 * i + 1]) << 16);
      *reinterpret_cast<uint4*>(dst) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
      for (int i = 0; i < kPerThread; ++i)
        if (s0 + i < n) dst[i] = pcm16_sample(v[i]);
    }
  } else {
    float* dst = static_cast<float*>(p.out) + row * p.out_stride + s0;
    if (whole) {
      *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
#pragma unroll
      for (int i = 0; i < kPerThread; ++i)
        if (s0 + i < n) dst[i] = v[i];
    }
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

extern "C" int omni_waveform_egress(const float* wave, int64_t rows, int64_t samples,
                                    int64_t wave_stride_row, const int64_t* row_samples,
                                    int format, void* out, int64_t out_stride_row,
                                    omni_stream_t stream) {
  if (!wave || !out) return OMNI_ERR_INVALID_ARG;
  if (format != OMNI_EGRESS_F32 && format != OMNI_EGRESS_PCM16) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || samples < 0 || wave_stride_row < samples || out_stride_row < samples)
    return OMNI_ERR_INVALID_ARG;
  if (rows == 0 || samples == 0) return OMNI_OK;
  if (rows > 65535) return OMNI_ERR_UNSUPPORTED;
  EgressParams p{};
  p.wave = wave;
  p.wave_stride = wave_stride_row;
  p.samples = samples;
  p.row_samples = row_samples;
  p.out = out;
  p.out_stride = out_stride_row;
  p.chunks_per_row = (samples + kPerThread - 1) / kPerThread;
  if (p.chunks_per_row > (int64_t)0x7fffffff * kThreads) return OMNI_ERR_UNSUPPORTED;
  const int elem_out = format == OMNI_EGRESS_PCM16 ? 2 : 4;
  // every row start stays 16-byte aligned: base pointers aligned, row strides multiples of 16 B
  const bool vec = aligned16(wave) && aligned16(out) && (wave_stride_row * 4) % 16 == 0 &&
                   (out_stride_row * elem_out) % 16 == 0;
  dim3 grid((unsigned)((p.chunks_per_row + kThreads - 1) / kThreads), (unsigned)rows);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (format == OMNI_EGRESS_PCM16) {
    if (vec)
      hipLaunchKernelGGL((waveform_egress_kernel<OMNI_EGRESS_PCM16, true>), grid, dim3(kThreads),
                         0, s, p);
    else
      hipLaunchKernelGGL((waveform_egress_kernel<OMNI_EGRESS_PCM16, false>), grid, dim3(kThreads),
                         0, s, p);
  } else {
    if (vec)
      hipLaunchKernelGGL((waveform_egress_kernel<OMNI_EGRESS_F32, true>), grid, dim3(kThreads), 0,
                         s, p);
    else
      hipLaunchKernelGGL((waveform_egress_kernel<OMNI_EGRESS_F32, false>), grid, dim3(kThreads),
                         0, s, p);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}
