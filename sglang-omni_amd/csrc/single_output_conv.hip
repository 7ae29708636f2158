// Conv from channels-last activations to one output channel (the decoder's last layer), with
// tanh or clamp, accumulated in float32 in one fixed order per position.
//
// A workgroup owns 256 consecutive positions of one row, one per thread. Per chunk of up to 128
// channels it stages the rows [i0 - left_pad, i0 + 256 + taps - 1 - left_pad) of the activated
// input in LDS (vector loads, the input activation applied on the way, rows padded by 16 bytes so
// the 16-byte reads of 16 consecutive positions hit distinct banks), then every thread
// accumulates its own position: chunk by chunk, tap by tap, channel by channel. That order
// depends on nothing but the position, so any split of positions or rows gives identical bits.
// The weights are wave-uniform and come through the scalar cache.
//
// Inputs are staged as float32 (exact, the reference kernel's semantics) unless the conv is the
// decoder's last layer, whose activated inputs are rounded to bf16 like every other conv operand
// and like the streaming history it keeps.
#include <type_traits>

#include "common.h"

namespace {

constexpr int kPositions = 256;
constexpr int kMaxChunk = 128;  // channels staged per pass
constexpr int kMaxTaps = 16;

struct SocParams {
  const void* x;
  int64_t x_sb, x_st, batch, length, channels;
  int ctx_in_buffer;
  int in_act;
  const float* in_a;
  const float* in_b;
  const float* weight;  // [taps][channels]
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

template <int DT>
__device__ __forceinline__ void load4(const void* base, int64_t idx, float v[4]) {
  if constexpr (DT == OMNI_DTYPE_F32) {
    const float4 f = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(base) + idx);
    v[0] = f.x; v[1] = f.y; v[2] = f.z; v[3] = f.w;
  } else {
    const uint2 w = *reinterpret_cast<const uint2*>(reinterpret_cast<const u16*>(base) + idx);
    const u16 h[4] = {(u16)(w.x & 0xffff), (u16)(w.x >> 16), (u16)(w.y & 0xffff),
                      (u16)(w.y >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e)
      v[e] = DT == OMNI_DTYPE_BF16 ? bits_to_float_bf16(h[e]) : bits_to_float_f16(h[e]);
  }
}

template <int DT>
__device__ __forceinline__ void store_val(void* base, int64_t idx, float v) {
  if constexpr (DT == OMNI_DTYPE_F32) reinterpret_cast<float*>(base)[idx] = v;
  else if constexpr (DT == OMNI_DTYPE_BF16)
    reinterpret_cast<u16*>(base)[idx] = float_to_bits_bf16(v);
  else reinterpret_cast<u16*>(base)[idx] = float_to_bits_f16(v);
}

template <int XDT, int ODT, bool STAGE_BF16>
__global__ void __launch_bounds__(kPositions) single_output_conv_kernel(const SocParams p) {
  using S = typename std::conditional<STAGE_BF16, u16, float>::type;
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_raw[];
  S* xs = reinterpret_cast<S*>(lds_raw);
  const int tid = threadIdx.x;
  const int64_t tiles = (p.length + kPositions - 1) / kPositions;
  const int64_t b = blockIdx.x / tiles;
  const int i0 = (int)(blockIdx.x - b * tiles) * kPositions;
  const int ctx = p.lpad;  // positions read left of i
  const int rows = kPositions + p.taps - 1;
  const int L = (int)p.length;
  const int C = (int)p.channels;

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
  for (int c0 = 0; c0 < C; c0 += kMaxChunk) {
    const int cn = min(kMaxChunk, C - c0);
    const int groups = cn / 4;          // 4-channel pieces per row
    const int pitch = cn + 16 / (int)sizeof(S);  // elements per LDS row (16 bytes of padding)
    __syncthreads();
    for (int e = tid; e < rows * groups; e += kPositions) {
      const int r = e / groups;
      const int c = c0 + (e - r * groups) * 4;
      const int pos = i0 - ctx + r;
      float v[4] = {0.f, 0.f, 0.f, 0.f};
      bool activated = false;  // history and padding are already activated inputs
      if (pos >= 0 && pos < L) {
        load4<XDT>(p.x, b * p.x_sb + (int64_t)pos * p.x_st + c, v);
        activated = true;
      } else if (pos < 0) {
        if (p.ctx_in_buffer) {
          load4<XDT>(p.x, b * p.x_sb + (int64_t)pos * p.x_st + c, v);
          activated = true;
        } else if (hist_read) {
          load4<OMNI_DTYPE_BF16>(hist_read, (int64_t)(ctx + pos) * C + c, v);
        }
      }
      if (activated && p.in_act != OMNI_ACT_NONE) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          v[q] = apply_act(p.in_act, v[q], p.in_a[c + q], p.in_b[c + q], 0.f);
      }
      uint2 o;  // the bf16 form: the history's, and the staged one when STAGE_BF16
      o.x = (uint32_t)float_to_bits_bf16(v[0]) | ((uint32_t)float_to_bits_bf16(v[1]) << 16);
      o.y = (uint32_t)float_to_bits_bf16(v[2]) | ((uint32_t)float_to_bits_bf16(v[3]) << 16);
      if constexpr (STAGE_BF16)
        *reinterpret_cast<uint2*>(xs + r * pitch + (c - c0)) = o;
      else
        *reinterpret_cast<float4*>(xs + r * pitch + (c - c0)) = make_float4(v[0], v[1], v[2], v[3]);
      // History (streaming only, where ctx = taps - 1): the last ctx samples of history ++ input,
      // each written by the workgroup whose positions hold it (those left of 0 by the first).
      if (hist_write != nullptr && pos >= L - ctx && pos < L &&
          ((pos >= i0 && pos < i0 + kPositions) || (i0 == 0 && pos < 0)))
        *reinterpret_cast<uint2*>(hist_write + (int64_t)(pos - (L - ctx)) * C + c) = o;
    }
    __syncthreads();
    for (int j = 0; j < p.taps; ++j) {
      const float* wrow = p.weight + j * C + c0;
      const S* xrow = xs + (tid + j) * pitch;
      if constexpr (STAGE_BF16) {
        for (int c = 0; c < cn; c += 8) {
          const uint4 w = *reinterpret_cast<const uint4*>(xrow + c);
          acc = __builtin_fmaf(wrow[c + 0], __uint_as_float(w.x << 16), acc);
          acc = __builtin_fmaf(wrow[c + 1], __uint_as_float(w.x & 0xffff0000u), acc);
          acc = __builtin_fmaf(wrow[c + 2], __uint_as_float(w.y << 16), acc);
          acc = __builtin_fmaf(wrow[c + 3], __uint_as_float(w.y & 0xffff0000u), acc);
          acc = __builtin_fmaf(wrow[c + 4], __uint_as_float(w.z << 16), acc);
          acc = __builtin_fmaf(wrow[c + 5], __uint_as_float(w.z & 0xffff0000u), acc);
          acc = __builtin_fmaf(wrow[c + 6], __uint_as_float(w.w << 16), acc);
          acc = __builtin_fmaf(wrow[c + 7], __uint_as_float(w.w & 0xffff0000u), acc);
        }
      } else {
        for (int c = 0; c < cn; c += 4) {
          const float4 w = *reinterpret_cast<const float4*>(xrow + c);
          acc = __builtin_fmaf(wrow[c + 0], w.x, acc);
          acc = __builtin_fmaf(wrow[c + 1], w.y, acc);
          acc = __builtin_fmaf(wrow[c + 2], w.z, acc);
          acc = __builtin_fmaf(wrow[c + 3], w.w, acc);
        }
      }
    }
  }
  const int i = i0 + tid;
  if (i < L) {
    const float v = acc + (p.bias ? p.bias[0] : 0.f);
    store_val<ODT>(p.out, b * p.o_sb + i, apply_act(p.act, v, 0.f, 0.f, 0.f));
  }
}

// The decoder's form, bf16 input used as is with G * 8 <= 128 channels and at most 8 taps: the
// same tile, order and history handling as above, but every thread issues all of its 16-byte
// staging loads (buffer loads: pieces past an edge read zeros) before the first LDS store, so a
// workgroup waits for HBM once rather than once per piece.
constexpr int kFastMaxTaps = 8;

struct SocFastParams {
  const u16* x;
  int x_sb, x_st, length, tiles;
  const float* weight;  // [taps][channels]
  const float* bias;
  int taps, lpad;
  const u16* hist;
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_slots;
  int hist_slot_stride;
  int hist_cold;
  int act;
  void* out;
  int64_t o_sb;
  uint32_t x_bytes, hist_bytes;
};

template <int G, int ODT>
__global__ void __launch_bounds__(kPositions) single_output_conv_bf16_kernel(const SocFastParams p) {
  constexpr int C = G * 8;
  constexpr int PITCH = C + 8;  // elements per LDS row (16 bytes of padding)
  constexpr int PIECES = ((kPositions + kFastMaxTaps - 1) * G + kPositions - 1) / kPositions;
  extern __shared__ __attribute__((aligned(16))) u16 xs[];
  const int tid = threadIdx.x;
  const int b = blockIdx.x / p.tiles;
  const int i0 = (blockIdx.x - b * p.tiles) * kPositions;
  const int ctx = p.lpad;
  const int rows = kPositions + p.taps - 1;
  const int L = p.length;

  int hread = -1, hwrite = -1;  // element offsets of this row's two history copies in the pool
  if (p.hist != nullptr) {
    const int64_t slot = p.slot_index[b];
    if (slot >= 0 && slot < p.hist_slots) {
      const int parity = (int)(p.slot_parity[slot] & 1);
      const int base = (int)slot * p.hist_slot_stride;
      hread = p.hist_cold ? -1 : base + parity * ctx * C;
      hwrite = base + (1 - parity) * ctx * C;
    }
  }
  const auto x_rsrc = buffer_rsrc(p.x, p.x_bytes);
  const auto h_rsrc = buffer_rsrc(p.hist, p.hist_bytes);
  u32x4 v[PIECES];
#pragma unroll
  for (int u = 0; u < PIECES; ++u) {
    const int piece = tid + u * kPositions;
    const int r = piece / G;
    const int c = (piece - r * G) * 8;
    const int pos = i0 - ctx + r;
    uint32_t xo = kOutOfRange, ho = kOutOfRange;
    if (r < rows) {
      if (pos >= 0 && pos < L) xo = (uint32_t)(b * p.x_sb + pos * p.x_st + c) * 2;
      else if (pos < 0 && hread >= 0) ho = (uint32_t)(hread + (ctx + pos) * C + c) * 2;
    }
    v[u] = __builtin_amdgcn_raw_buffer_load_b128(x_rsrc, xo, 0, 0) |
           __builtin_amdgcn_raw_buffer_load_b128(h_rsrc, ho, 0, 0);
  }
  // the weights [taps][C] go to LDS behind the rows (at most 8 x 128 floats: one float4 a
  // thread), loaded with the rows, so the tap loop reads no global memory
  float* ws = reinterpret_cast<float*>(xs + rows * PITCH);
  const int wq = p.taps * C / 4;
  f32x4 wv = {0.f, 0.f, 0.f, 0.f};
  if (tid < wq) wv = *reinterpret_cast<const f32x4*>(p.weight + 4 * tid);
#pragma unroll
  for (int u = 0; u < PIECES; ++u) {
    const int piece = tid + u * kPositions;
    const int r = piece / G;
    const int c = (piece - r * G) * 8;
    if (r < rows) *reinterpret_cast<u32x4*>(xs + r * PITCH + c) = v[u];
  }
  if (tid < wq) *reinterpret_cast<f32x4*>(ws + 4 * tid) = wv;
  if (hwrite >= 0) {
    // the last ctx samples of history ++ input, each written by the workgroup whose positions
    // hold it (those left of 0 by the first)
#pragma unroll
    for (int u = 0; u < PIECES; ++u) {
      const int piece = tid + u * kPositions;
      const int r = piece / G;
      const int c = (piece - r * G) * 8;
      const int pos = i0 - ctx + r;
      const bool own = r < rows && pos >= L - ctx && pos < L &&
                       ((pos >= i0 && pos < i0 + kPositions) || (i0 == 0 && pos < 0));
      const uint32_t wo = own ? (uint32_t)(hwrite + (pos - (L - ctx)) * C + c) * 2 : kOutOfRange;
      __builtin_amdgcn_raw_buffer_store_b128(v[u], h_rsrc, wo, 0, 0);
    }
  }
  __syncthreads();
  float acc = 0.f;
  const u16* xrow = xs + tid * PITCH;
  for (int j = 0; j < p.taps; ++j) {
    const float* wrow = ws + j * C;
#pragma unroll
    for (int c = 0; c < C; c += 8) {
      const u32x4 w = *reinterpret_cast<const u32x4*>(xrow + j * PITCH + c);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc = __builtin_fmaf(wrow[c + 2 * e], __uint_as_float(w[e] << 16), acc);
        acc = __builtin_fmaf(wrow[c + 2 * e + 1], __uint_as_float(w[e] & 0xffff0000u), acc);
      }
    }
  }
  const int i = i0 + tid;
  if (i < L) {
    const float y = acc + (p.bias ? p.bias[0] : 0.f);
    store_val<ODT>(p.out, b * p.o_sb + i, apply_act(p.act, y, 0.f, 0.f, 0.f));
  }
}

template <int G, int ODT>
int launch_soc_fast(const SocFastParams& p, hipStream_t s, dim3 grid) {
  auto k = single_output_conv_bf16_kernel<G, ODT>;
  static const bool raised = [&] {
    const hipError_t e = hipFuncSetAttribute((const void*)k,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipGetLastError();
    return e == hipSuccess;
  }();
  (void)raised;
  const size_t lds = (size_t)(kPositions + p.taps - 1) * (G * 8 + 8) * 2 + (size_t)p.taps * G * 8 * 4;
  hipLaunchKernelGGL(k, grid, dim3(kPositions), lds, s, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

template <int G>
int launch_soc_fast_o(const SocFastParams& p, int out_dtype, hipStream_t s, dim3 grid) {
  if (out_dtype == OMNI_DTYPE_F32) return launch_soc_fast<G, OMNI_DTYPE_F32>(p, s, grid);
  if (out_dtype == OMNI_DTYPE_BF16) return launch_soc_fast<G, OMNI_DTYPE_BF16>(p, s, grid);
  return launch_soc_fast<G, OMNI_DTYPE_F16>(p, s, grid);
}

size_t lds_bytes(int64_t channels, int taps, bool stage_bf16) {
  const int64_t cn = channels < kMaxChunk ? channels : kMaxChunk;
  const int64_t elem = stage_bf16 ? 2 : 4;
  return (size_t)(kPositions + taps - 1) * (cn * elem + 16);
}

// Raise a kernel's dynamic-LDS limit to the CU's 160 KiB, once per instantiation (so launches
// inside a graph capture make no attribute calls). A refusal is not an error here: the launch
// check reports a launch the runtime cannot make.
template <int XDT, int ODT, bool STAGE_BF16>
int launch_soc(const SocParams& p, hipStream_t s, dim3 grid) {
  auto k = single_output_conv_kernel<XDT, ODT, STAGE_BF16>;
  static const bool raised = [&] {
    const hipError_t e = hipFuncSetAttribute((const void*)k,
                                             hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    (void)hipGetLastError();
    return e == hipSuccess;
  }();
  (void)raised;
  const size_t lds = lds_bytes(p.channels, (int)p.taps, STAGE_BF16);
  hipLaunchKernelGGL(k, grid, dim3(kPositions), lds, s, p);
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

template <int XDT, bool STAGE_BF16>
int launch_soc_x(const SocParams& p, int out_dtype, hipStream_t s, dim3 grid) {
  if (out_dtype == OMNI_DTYPE_F32) return launch_soc<XDT, OMNI_DTYPE_F32, STAGE_BF16>(p, s, grid);
  if (out_dtype == OMNI_DTYPE_BF16) return launch_soc<XDT, OMNI_DTYPE_BF16, STAGE_BF16>(p, s, grid);
  return launch_soc<XDT, OMNI_DTYPE_F16, STAGE_BF16>(p, s, grid);
}

bool float_like(int dt) {
  return dt == OMNI_DTYPE_F32 || dt == OMNI_DTYPE_BF16 || dt == OMNI_DTYPE_F16;
}

}  // namespace

extern "C" int omni_single_output_conv(const void* x, int x_dtype, int64_t x_stride_b,
                                       int64_t x_stride_t, int64_t batch, int64_t length,
                                       int64_t channels, int context_in_buffer,
                                       int in_activation, const float* in_act_a,
                                       const float* in_act_b, const float* weight,
                                       const float* bias, int64_t taps, int64_t left_pad,
                                       const void* hist_pool, const int64_t* slot_index,
                                       const int64_t* slot_parity, int64_t hist_num_slots,
                                       int64_t hist_slot_stride, int history_cold, int activation,
                                       void* out, int out_dtype, int64_t out_stride_b,
                                       omni_stream_t stream) {
  if (!x || !weight || !out) return OMNI_ERR_INVALID_ARG;
  if (batch < 0 || length < 0 || channels < 4 || channels % 4 || taps < 1 || taps > kMaxTaps)
    return OMNI_ERR_INVALID_ARG;
  if (left_pad < 0 || left_pad > taps - 1) return OMNI_ERR_INVALID_ARG;
  if (!float_like(x_dtype) || !float_like(out_dtype)) return OMNI_ERR_INVALID_ARG;
  if (in_activation != OMNI_ACTIVATION_NONE && in_activation != OMNI_ACTIVATION_SNAKE)
    return OMNI_ERR_INVALID_ARG;
  if (in_activation == OMNI_ACTIVATION_SNAKE && (!in_act_a || !in_act_b))
    return OMNI_ERR_INVALID_ARG;
  if (activation != OMNI_ACTIVATION_NONE && activation != OMNI_ACTIVATION_TANH &&
      activation != OMNI_ACTIVATION_CLAMP)
    return OMNI_ERR_INVALID_ARG;
  // 16-byte (float32) or 8-byte (16-bit) loads of 4 channels
  const int64_t align = x_dtype == OMNI_DTYPE_F32 ? 16 : 8;
  const int64_t elem = x_dtype == OMNI_DTYPE_F32 ? 4 : 2;
  if (x_stride_t < channels || (reinterpret_cast<uintptr_t>(x) % align) ||
      (x_stride_t * elem) % align || (x_stride_b * elem) % align)
    return OMNI_ERR_INVALID_ARG;
  if (hist_pool) {
    if (context_in_buffer || !slot_index || !slot_parity || left_pad != taps - 1)
      return OMNI_ERR_INVALID_ARG;
    if (hist_slot_stride < 2 * (taps - 1) * channels || hist_num_slots < 1 ||
        (reinterpret_cast<uintptr_t>(hist_pool) & 7) || hist_slot_stride % 4)
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
  p.in_act = in_activation;
  p.in_a = in_act_a;
  p.in_b = in_act_b;
  p.weight = weight;
  p.bias = bias;
  p.taps = (int)taps;
  p.lpad = (int)left_pad;
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
  if (batch * tiles > 0x7fffffffLL || length > 0x3fffffffLL) return OMNI_ERR_UNSUPPORTED;
  const dim3 grid((unsigned)(batch * tiles));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // the decoder's form (an input activation or a slot history): bf16 operands, like the history
  const bool stage_bf16 = in_activation != OMNI_ACTIVATION_NONE || hist_pool != nullptr;
  if (stage_bf16 && channels % 8) return OMNI_ERR_UNSUPPORTED;
  if (x_dtype == OMNI_DTYPE_BF16 && in_activation == OMNI_ACTIVATION_NONE && !context_in_buffer &&
      (channels == 32 || channels == 64 || channels == 96 || channels == 128) &&
      taps <= kFastMaxTaps && (reinterpret_cast<uintptr_t>(x) & 15) == 0 && x_stride_t % 8 == 0 &&
      x_stride_b % 8 == 0 && (!hist_pool || (reinterpret_cast<uintptr_t>(hist_pool) & 15) == 0) &&
      (reinterpret_cast<uintptr_t>(weight) & 15) == 0) {
    // 32-bit element offsets and buffer extents
    const int64_t x_bytes = ((batch - 1) * x_stride_b + (length - 1) * x_stride_t + channels) * 2;
    const int64_t hist_bytes = hist_pool ? hist_num_slots * hist_slot_stride * 2 : 0;
    if (x_bytes <= 0x7fffffffLL && hist_bytes <= 0x7fffffffLL && x_stride_b <= 0x7fffffffLL &&
        hist_slot_stride % 8 == 0) {
      SocFastParams f{};
      f.x = reinterpret_cast<const u16*>(x);
      f.x_sb = (int)x_stride_b;
      f.x_st = (int)x_stride_t;
      f.length = (int)length;
      f.tiles = (int)tiles;
      f.weight = weight;
      f.bias = bias;
      f.taps = (int)taps;
      f.lpad = (int)left_pad;
      f.hist = p.hist;
      f.slot_index = slot_index;
      f.slot_parity = slot_parity;
      f.hist_slots = hist_num_slots;
      f.hist_slot_stride = (int)hist_slot_stride;
      f.hist_cold = history_cold;
      f.act = activation;
      f.out = out;
      f.o_sb = out_stride_b;
      f.x_bytes = (uint32_t)x_bytes;
      f.hist_bytes = (uint32_t)hist_bytes;
      switch (channels) {
        case 32: return launch_soc_fast_o<4>(f, out_dtype, s, grid);
        case 64: return launch_soc_fast_o<8>(f, out_dtype, s, grid);
        case 96: return launch_soc_fast_o<12>(f, out_dtype, s, grid);
        default: return launch_soc_fast_o<16>(f, out_dtype, s, grid);
      }
    }
  }
  if (stage_bf16) {
    if (x_dtype == OMNI_DTYPE_F32) return launch_soc_x<OMNI_DTYPE_F32, true>(p, out_dtype, s, grid);
    if (x_dtype == OMNI_DTYPE_BF16) return launch_soc_x<OMNI_DTYPE_BF16, true>(p, out_dtype, s, grid);
    return launch_soc_x<OMNI_DTYPE_F16, true>(p, out_dtype, s, grid);
  }
  if (x_dtype == OMNI_DTYPE_F32) return launch_soc_x<OMNI_DTYPE_F32, false>(p, out_dtype, s, grid);
  if (x_dtype == OMNI_DTYPE_BF16) return launch_soc_x<OMNI_DTYPE_BF16, false>(p, out_dtype, s, grid);
  return launch_soc_x<OMNI_DTYPE_F16, false>(p, out_dtype, s, grid);
}
