// HiFT's short-time Fourier transform and its inverse (the iSTFT tail of the CosyVoice3 /
// MiniCPM-o vocoders), on gfx950. Both are HBM-bound: a 16-point transform does 16 MACs per
// output component, so the kernels read their input once, keep the small bases and the
// workgroup's window of frames in LDS, and give every output one fixed summation order (so a row's
// result does not depend on the batch or the tiling). HiFT's geometry (n_fft 16, hop 4) has its
// own instantiation with the loops unrolled; other sizes take the runtime-sized kernels.
//
//   short_time_spectrum: spectrum[r, c, f] = sum_{k < n_fft} x[r, f * hop + k - pad] * basis[c, k]
//     (c < bins the windowed cosines, c >= bins the windowed negative sines; pad = n_fft / 2 with
//     reflection when centring, else the caller's signal is already padded)
//   overlap_add_inverse: y[r, i] = (sum_{frames f over i} sum_{b < bins} re[r, b, f] *
//     ibasis[b, t] + im[r, b, f] * ibasis[bins + b, t]) / (sum_f window[t]^2), t = i + n_fft / 2 -
//     f * hop (torch.istft with center = True)
//   istft_tail: the same inverse fed straight from the vocoder's last conv, channels-last
//     h[r, f, 2 * bins]: magnitude = min(exp(h[.., b]), mag_clip), phase = sin(h[.., bins + b]),
//     re = magnitude * cos(phase), im = magnitude * sin(phase), and the output clamped to
//     +-audio_limit (hift_channels_last.py:269-276 with hift_channels_last.py:117-125).
#include "common.h"

namespace {

constexpr int kMaxFft = 64;
constexpr int kThreads = 256;
constexpr int kFramesPerBlock = 256;   // spectrum: frames per workgroup (one per thread)
constexpr int kSamplesPerBlock = 256;  // inverse: output samples per workgroup (one per thread)

// Reflection of index i into [0, n) (torch's "reflect" padding: the edge sample is not repeated).
__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
  if (n == 1) return 0;
  const int64_t period = 2 * (n - 1);
  i = i % period;
  if (i < 0) i += period;
  return i < n ? i : period - i;
}

struct StftParams {
  const float* x;
  int64_t x_stride;  // elements between rows
  int64_t samples;   // samples per row of x
  int center;        // 1: reflect-pad by n_fft / 2 here; 0: x is already padded
  const float* basis;  // [2 * bins][n_fft]
  int n_fft, hop, bins;
  int64_t frames;
  float* out;  // [rows][2 * bins][frames]
};

// Dynamic LDS: the basis [2 * bins][n_fft], then the block's signal span.
size_t stft_lds_bytes(int n_fft, int hop, int bins) {
  return (size_t)(2 * bins * n_fft + (kFramesPerBlock - 1) * hop + n_fft) * sizeof(float);
}

// NF, HP: the transform's n_fft and hop when known at compile time (the loops unroll and the
// frame's samples stay in registers), 0 for the runtime values of the parameters.
template <int NF, int HP>
__global__ void __launch_bounds__(kThreads) short_time_spectrum_kernel(const StftParams p) {
  extern __shared__ float smem[];
  const int n_fft = NF ? NF : p.n_fft;
  const int hop = HP ? HP : p.hop;
  const int bins = n_fft / 2 + 1;
  const int comps = 2 * bins;
  float* basis = smem;
  float* seg = smem + comps * n_fft;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t f0 = (int64_t)blockIdx.x * kFramesPerBlock;
  if constexpr (NF == 0)
    for (int e = tid; e < comps * n_fft; e += kThreads) basis[e] = p.basis[e];
  // the block's signal span: frames f0 .. f0 + kFramesPerBlock - 1 read padded samples
  // f0 * hop .. (f0 + kFramesPerBlock - 1) * hop + n_fft - 1
  const int64_t nframes = min((int64_t)kFramesPerBlock, p.frames - f0);
  const int span = (int)((nframes - 1) * hop + n_fft);
  const int pad = p.center ? n_fft / 2 : 0;
  const float* xr = p.x + row * p.x_stride;
  for (int e = tid; e < span; e += kThreads) {
    int64_t i = f0 * hop + e - pad;
    if (p.center) i = reflect(i, p.samples);
    seg[e] = xr[i];
  }
  __syncthreads();
  if (tid >= nframes) return;
  float* o = p.out + (row * comps) * p.frames + f0 + tid;
  if constexpr (NF != 0) {
    // the bases are the same for every thread: read through the constant address space, they
    // arrive by scalar loads and feed the FMAs as scalar operands (no LDS traffic)
    typedef __attribute__((address_space(4))) const float cfloat;
    cfloat* gbasis = (cfloat*)(p.basis);
    float s[NF];
#pragma unroll
    for (int k = 0; k < NF; ++k) s[k] = seg[tid * hop + k];
#pragma unroll 2
    for (int c = 0; c < comps; ++c) {
      cfloat* b = gbasis + c * NF;
      float acc = 0.f;
#pragma unroll
      for (int k = 0; k < NF; ++k) acc = __builtin_fmaf(s[k], b[k], acc);
      o[(int64_t)c * p.frames] = acc;
    }
  } else {
    const float* s = seg + tid * hop;
    for (int c = 0; c < comps; ++c) {
      const float* b = basis + c * n_fft;
      float acc = 0.f;
      for (int k = 0; k < n_fft; ++k) acc = __builtin_fmaf(s[k], b[k], acc);
      o[(int64_t)c * p.frames] = acc;
    }
  }
}

struct IstftParams {
  // spectrum source: either separate real / imaginary [rows][bins][frames] (tail = 0), or the
  // vocoder's channels-last conv output h [rows][frames][h_stride] (tail = 1)
  const float* re;
  const float* im;
  const float* h;
  int64_t h_row_stride, h_frame_stride;
  int tail;
  float mag_clip, audio_limit;
  const float* basis;     // [2 * bins][n_fft], the one-sided inverse's windowed bases / n_fft
  const float* win2;      // [n_fft] squared window
  int n_fft, hop, bins;
  int64_t frames, samples;
  float* out;  // [rows][out_stride]
  int64_t out_stride;
};

// The frames one inverse workgroup reads: its samples' padded positions span
// (kSamplesPerBlock - 1) / hop + 1 frame starts, plus n_fft / hop - 1 earlier overlapping frames.
int inverse_frames_per_block(int n_fft, int hop) {
  return (kSamplesPerBlock - 1) / hop + n_fft / hop + 1;
}

// Dynamic LDS: the basis [2 * bins][n_fft], the squared window [n_fft], then the workgroup's
// frames [nf][2 * bins].
size_t inverse_lds_bytes(int n_fft, int hop, int bins) {
  return (size_t)(2 * bins * n_fft + n_fft + inverse_frames_per_block(n_fft, hop) * 2 * bins) *
         sizeof(float);
}

template <int NF, int HP>
__global__ void __launch_bounds__(kThreads) overlap_add_inverse_kernel(const IstftParams p) {
  extern __shared__ float smem[];
  const int n_fft = NF ? NF : p.n_fft;
  const int hop = HP ? HP : p.hop;
  const int bins = n_fft / 2 + 1;
  const int comps = 2 * bins;
  const int half = n_fft / 2;
  const int overlaps = n_fft / hop;
  float* basis = smem;
  float* win2 = basis + comps * n_fft;
  float* spec = win2 + n_fft;
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t i0 = (int64_t)blockIdx.x * kSamplesPerBlock;
  for (int e = tid; e < comps * n_fft; e += kThreads) basis[e] = p.basis[e];
  for (int e = tid; e < n_fft; e += kThreads) win2[e] = p.win2[e];
  // frames whose window covers samples i0 .. i0 + kSamplesPerBlock - 1 (padded positions
  // i + half): from (i0 + half) / hop - (overlaps - 1) to (i0 + kSamplesPerBlock - 1 + half) / hop
  const int64_t fa = (i0 + half) / hop - (overlaps - 1);
  const int64_t fb = (i0 + kSamplesPerBlock - 1 + half) / hop;
  const int nf = (int)(fb - fa + 1);
  if (p.tail) {
    // one thread per (frame, bin): magnitude and phase once, both parts out
    for (int e = tid; e < nf * bins; e += kThreads) {
      const int j = e / bins;  // frame within the window
      const int b = e - j * bins;
      const int64_t f = fa + j;
      float re = 0.f, im = 0.f;
      if (f >= 0 && f < p.frames) {
        const float* hf = p.h + row * p.h_row_stride + f * p.h_frame_stride;
        const float mag = fminf(expf(hf[b]), p.mag_clip);
        const float phase = sinf(hf[bins + b]);
        re = mag * cosf(phase);
        im = mag * sinf(phase);
      }
      spec[j * comps + b] = re;
      spec[j * comps + bins + b] = im;
    }
  } else {
    for (int e = tid; e < nf * comps; e += kThreads) {
      const int j = e / comps;  // frame within the window
      const int c = e - j * comps;
      const int64_t f = fa + j;
      float v = 0.f;
      if (f >= 0 && f < p.frames) {
        const float* src = c < bins ? p.re : p.im;
        const int b = c < bins ? c : c - bins;
        v = src[(row * bins + b) * p.frames + f];
      }
      spec[j * comps + c] = v;
    }
  }
  __syncthreads();
  const int64_t i = i0 + tid;
  if (i >= p.samples) return;
  const int64_t pos = i + half;
  float signal = 0.f, envelope = 0.f;
#pragma unroll
  for (int o = 0; o < (NF ? NF / HP : kMaxFft); ++o) {
    if (!NF && o >= overlaps) break;
    const int64_t f = pos / hop - o;
    if (f < 0 || f >= p.frames) continue;
    const int t = (int)(pos - f * hop);
    const float* s = spec + (int)(f - fa) * comps;
#pragma unroll
    for (int b = 0; b < (NF ? NF / 2 + 1 : kMaxFft / 2 + 1); ++b) {
      if (!NF && b >= bins) break;
      signal += __builtin_fmaf(s[b], basis[b * n_fft + t],
                               s[bins + b] * basis[(bins + b) * n_fft + t]);
    }
    envelope += win2[t];
  }
  float y = signal / envelope;
  if (p.tail) y = fminf(fmaxf(y, -p.audio_limit), p.audio_limit);
  p.out[row * p.out_stride + i] = y;
}

// HiFT's geometry (n_fft 16, hop 4, 9 bins): each thread finishes 4 samples of one window phase
// r = sample % 4 (samples i0 + tid + 256 k), so its 4 x 18 basis values and 4 squared-window
// values stay in registers for all of them (2 or 8 samples per thread measured slower: 8 leaves
// each workgroup's exp / sin / sincos staging too long a serial chain); the workgroup's frames sit in LDS as rows of 20
// floats (18 components, 2 pad) read 16 bytes at a time. Every output takes the generic kernel's
// terms in its order (overlaps ascending, then bins), so the two give the same bits.
constexpr int kInv16Samples = 4 * kThreads;  // samples per workgroup
constexpr int kInv16Pitch = 20;              // floats per frame row in LDS
constexpr int inverse16_frames() { return (kInv16Samples - 1) / 4 + 16 / 4 + 1; }
constexpr size_t inverse16_lds_bytes() { return (size_t)inverse16_frames() * kInv16Pitch * 4; }

__global__ void __launch_bounds__(kThreads) overlap_add_inverse16_kernel(const IstftParams p) {
  constexpr int NF = 16, HP = 4, BINS = 9, COMPS = 18, OV = NF / HP, HALF = NF / 2;
  extern __shared__ float smem[];
  float* spec = smem;  // [frames of the window][kInv16Pitch]
  const int tid = threadIdx.x;
  const int64_t row = blockIdx.y;
  const int64_t i0 = (int64_t)blockIdx.x * kInv16Samples;
  const int64_t fa = (i0 + HALF) / HP - (OV - 1);
  const int64_t fb = (i0 + kInv16Samples - 1 + HALF) / HP;
  const int nf = (int)(fb - fa + 1);
  if (p.tail) {
    for (int e = tid; e < nf * BINS; e += kThreads) {
      const int j = e / BINS;
      const int b = e - j * BINS;
      const int64_t f = fa + j;
      float re = 0.f, im = 0.f;
      if (f >= 0 && f < p.frames) {
        const float* hf = p.h + row * p.h_row_stride + f * p.h_frame_stride;
        const float mag = fminf(expf(hf[b]), p.mag_clip);
        const float phase = sinf(hf[BINS + b]);
        float sn, cs;
        sincosf(phase, &sn, &cs);
        re = mag * cs;
        im = mag * sn;
      }
      spec[j * kInv16Pitch + b] = re;
      spec[j * kInv16Pitch + BINS + b] = im;
    }
  } else {
    for (int e = tid; e < nf * COMPS; e += kThreads) {
      const int j = e / COMPS;
      const int c = e - j * COMPS;
      const int64_t f = fa + j;
      float v = 0.f;
      if (f >= 0 && f < p.frames) {
        const float* src = c < BINS ? p.re : p.im;
        const int b = c < BINS ? c : c - BINS;
        v = src[(row * BINS + b) * p.frames + f];
      }
      spec[j * kInv16Pitch + c] = v;
    }
  }
  // this thread's window phase (i0 is a multiple of HP): t = r + HP o for overlap o
  const int r = (tid + HALF) % HP;
  float bas[OV][COMPS], w2[OV];
#pragma unroll
  for (int o = 0; o < OV; ++o) {
    w2[o] = p.win2[r + HP * o];
#pragma unroll
    for (int c = 0; c < COMPS; ++c) bas[o][c] = p.basis[c * NF + r + HP * o];
  }
  __syncthreads();
#pragma unroll 1
  for (int k = 0; k < kInv16Samples / kThreads; ++k) {
    const int64_t i = i0 + tid + (int64_t)k * kThreads;
    if (i >= p.samples) break;
    const int64_t pos = i + HALF;
    float signal = 0.f, envelope = 0.f;
#pragma unroll
    for (int o = 0; o < OV; ++o) {
      const int64_t f = pos / HP - o;
      if (f < 0 || f >= p.frames) continue;
      const f32x4* sv = reinterpret_cast<const f32x4*>(spec + (int)(f - fa) * kInv16Pitch);
      float s[kInv16Pitch];
#pragma unroll
      for (int q = 0; q < kInv16Pitch / 4; ++q) {
        const f32x4 v = sv[q];
        s[4 * q] = v[0];
        s[4 * q + 1] = v[1];
        s[4 * q + 2] = v[2];
        s[4 * q + 3] = v[3];
      }
#pragma unroll
      for (int b = 0; b < BINS; ++b)
        signal += __builtin_fmaf(s[b], bas[o][b], s[BINS + b] * bas[o][BINS + b]);
      envelope += w2[o];
    }
    float y = signal / envelope;
    if (p.tail) y = fminf(fmaxf(y, -p.audio_limit), p.audio_limit);
    p.out[row * p.out_stride + i] = y;
  }
}

bool valid_fft(int64_t n_fft, int64_t hop, int64_t bins) {
  return n_fft >= 2 && n_fft <= kMaxFft && hop >= 1 && hop <= n_fft && n_fft % hop == 0 &&
         bins == n_fft / 2 + 1;
}

}  // namespace

extern "C" int omni_short_time_spectrum(const float* signal, int64_t rows, int64_t samples,
                                        int64_t signal_stride_row, int center,
                                        const float* basis, int64_t bins, int64_t n_fft,
                                        int64_t hop, float* spectrum, int64_t frames,
                                        omni_stream_t stream) {
  if (!signal || !basis || !spectrum) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || samples < 1 || signal_stride_row < samples || !valid_fft(n_fft, hop, bins))
    return OMNI_ERR_INVALID_ARG;
  const int64_t padded = center ? samples + n_fft : samples;  // 2 * (n_fft / 2) padding
  if (padded < n_fft || frames != (padded - n_fft) / hop + 1) return OMNI_ERR_INVALID_ARG;
  if (center && samples <= n_fft / 2) return OMNI_ERR_INVALID_ARG;  // reflect needs pad < samples
  if (rows == 0) return OMNI_OK;
  if (rows > 65535 || frames > 0x7fffffffLL / kFramesPerBlock) return OMNI_ERR_UNSUPPORTED;
  StftParams p{};
  p.x = signal;
  p.x_stride = signal_stride_row;
  p.samples = samples;
  p.center = center;
  p.basis = basis;
  p.n_fft = (int)n_fft;
  p.hop = (int)hop;
  p.bins = (int)bins;
  p.frames = frames;
  p.out = spectrum;
  dim3 grid((unsigned)((frames + kFramesPerBlock - 1) / kFramesPerBlock), (unsigned)rows);
  const size_t lds = stft_lds_bytes(p.n_fft, p.hop, p.bins);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.n_fft == 16 && p.hop == 4)
    hipLaunchKernelGGL((short_time_spectrum_kernel<16, 4>), grid, dim3(kThreads), lds, s, p);
  else
    hipLaunchKernelGGL((short_time_spectrum_kernel<0, 0>), grid, dim3(kThreads), lds, s, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

namespace {

int launch_inverse(IstftParams& p, int64_t rows, omni_stream_t stream) {
  // a workgroup's frame window in LDS stays within the default 64 KiB (HiFT: n_fft 16, hop 4
  // takes 6 KiB)
  if (inverse_lds_bytes(p.n_fft, p.hop, p.bins) > 64 * 1024) return OMNI_ERR_UNSUPPORTED;
  if (rows == 0 || p.samples == 0) return OMNI_OK;
  if (rows > 65535 || p.samples > 0x7fffffffLL - kSamplesPerBlock) return OMNI_ERR_UNSUPPORTED;
  dim3 grid((unsigned)((p.samples + kSamplesPerBlock - 1) / kSamplesPerBlock), (unsigned)rows);
  const size_t lds = inverse_lds_bytes(p.n_fft, p.hop, p.bins);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (p.n_fft == 16 && p.hop == 4) {
    dim3 grid16((unsigned)((p.samples + kInv16Samples - 1) / kInv16Samples), (unsigned)rows);
    hipLaunchKernelGGL(overlap_add_inverse16_kernel, grid16, dim3(kThreads), inverse16_lds_bytes(),
                       s, p);
  } else {
    hipLaunchKernelGGL((overlap_add_inverse_kernel<0, 0>), grid, dim3(kThreads), lds, s, p);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

}  // namespace

extern "C" int omni_overlap_add_inverse(const float* real, const float* imag, int64_t rows,
                                        int64_t bins, int64_t frames, const float* basis,
                                        const float* squared_window, int64_t n_fft, int64_t hop,
                                        float* out, int64_t out_stride_row,
                                        omni_stream_t stream) {
  if (!real || !imag || !basis || !squared_window || !out) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || frames < 1 || !valid_fft(n_fft, hop, bins)) return OMNI_ERR_INVALID_ARG;
  const int64_t samples = hop * (frames - 1);
  if (out_stride_row < samples) return OMNI_ERR_INVALID_ARG;
  IstftParams p{};
  p.re = real;
  p.im = imag;
  p.basis = basis;
  p.win2 = squared_window;
  p.n_fft = (int)n_fft;
  p.hop = (int)hop;
  p.bins = (int)bins;
  p.frames = frames;
  p.samples = samples;
  p.out = out;
  p.out_stride = out_stride_row;
  return launch_inverse(p, rows, stream);
}

extern "C" int omni_istft_tail(const float* h, int64_t rows, int64_t frames, int64_t h_stride_row,
                               int64_t h_stride_frame, const float* basis,
                               const float* squared_window, int64_t bins, int64_t n_fft,
                               int64_t hop, float magnitude_clip, float audio_limit, float* out,
                               int64_t out_stride_row, omni_stream_t stream) {
  if (!h || !basis || !squared_window || !out) return OMNI_ERR_INVALID_ARG;
  if (rows < 0 || frames < 1 || !valid_fft(n_fft, hop, bins)) return OMNI_ERR_INVALID_ARG;
  if (h_stride_frame < 2 * bins || h_stride_row < frames * h_stride_frame)
    return OMNI_ERR_INVALID_ARG;
  if (!(magnitude_clip > 0.f) || !(audio_limit > 0.f)) return OMNI_ERR_INVALID_ARG;
  const int64_t samples = hop * (frames - 1);
  if (out_stride_row < samples) return OMNI_ERR_INVALID_ARG;
  IstftParams p{};
  p.h = h;
  p.h_row_stride = h_stride_row;
  p.h_frame_stride = h_stride_frame;
  p.tail = 1;
  p.mag_clip = magnitude_clip;
  p.audio_limit = audio_limit;
  p.basis = basis;
  p.win2 = squared_window;
  p.n_fft = (int)n_fft;
  p.hop = (int)hop;
  p.bins = (int)bins;
  p.frames = frames;
  p.samples = samples;
  p.out = out;
  p.out_stride = out_stride_row;
  return launch_inverse(p, rows, stream);
}
