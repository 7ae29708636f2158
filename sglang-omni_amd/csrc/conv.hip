// Fused polyphase convolution on bf16 MFMA (gfx950 v_mfma_f32_16x16x32_bf16).
//
//   acc[b, i, n] = sum_{j < taps} sum_{ci} W[n, j, ci] * x[b, i + j*dil - left_pad, ci]
//
// is an implicit GEMM with the output channels n as the MFMA M dimension, positions i as the N
// dimension and (tap, ci) as K. One workgroup owns a tile of BCO output columns x BP positions of
// one batch row; per 32-channel K chunk it stages
//   * the input rows [i0 - left_pad, i0 + BP + halo - left_pad) x 32 channels (the tile plus its
//     (taps-1)*dil halo) once in LDS, and every tap reads them shifted by j*dil rows, and
//   * the weights [taps][BCO][32] in LDS,
// both with 80-byte rows (64 B of data + 16 B pad) so that the 16-byte ds_read of an MFMA
// operand (16 rows x 4 lanes) hits distinct banks. The next chunk's global loads are issued into
// registers before the current chunk's MFMAs, so HBM latency hides behind the matrix cores.
//
// The epilogue works on the MFMA accumulator layout (lane = position, 4 consecutive channels per
// lane) and fuses the per-column weight scale (fp8), bias, the float32 residual add, the float32
// residual-stream store and the activation (Snake / LeakyReLU / tanh / clamp) into the stores of
// the next conv's bf16 input.
//
// Streaming: positions left of 0 come from the slot's history copy (slot_parity & 1); the
// workgroups of column tile 0 write the last left_pad input samples into the other copy while
// they stage them, so no separate exchange launch is needed.
#include "common.h"

namespace {

constexpr int kChunk = 32;      // input channels per K chunk (one MFMA K step)
constexpr int kRowElems = 40;   // LDS row: 32 bf16 + 8 pad (80 B)

struct ConvParams {
  const u16* x;
  int64_t x_sb, x_st;
  int64_t batch, length, c_in, x_length;
  const void* weight;
  const float* wscale;
  int64_t n_cols, c_out, taps, dil, lpad;
  const float* bias;
  const u16* hist;  // pool base, NULL if no history
  const int64_t* slot_index;
  const int64_t* slot_parity;
  int64_t hist_slots;
  int64_t hist_slot_stride;
  int hist_cold;
  const float* residual;
  int64_t r_sb, r_st;  // shared by residual, mix_a, mix_b and sum_out
  const float* mix_a;
  const float* mix_b;
  float mix_scale;
  float* sum_out;
  void* out;
  int out_bf16;
  int64_t o_sb, o_st;
  int act;
  const float* act_a;
  const float* act_b;
  float slope;
  int64_t p_tiles, n_tiles;
};

// OCP e4m3fn -> float (exact). 0x7f / 0xff are NaN; there are no infinities.
__device__ __forceinline__ float fp8_e4m3_to_float(uint32_t v) {
  const uint32_t s = (v & 0x80u) << 24;
  const uint32_t e = (v >> 3) & 0xfu;
  const uint32_t m = v & 0x7u;
  float f;
  if (e == 0) {
    f = (float)m * 0.001953125f;  // m * 2^-9
  } else if (e == 15 && m == 7) {
    f = __uint_as_float(0x7fc00000u);
  } else {
    f = __uint_as_float(((e + 120u) << 23) | (m << 20));
  }
  return __uint_as_float(__float_as_uint(f) | s);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return (uint32_t)float_to_bits_bf16(a) | ((uint32_t)float_to_bits_bf16(b) << 16);
}

__device__ __forceinline__ uint4 fp8x8_to_bf16x8(uint2 raw) {
  uint4 o;
  o.x = pack_bf16x2(fp8_e4m3_to_float(raw.x & 0xff), fp8_e4m3_to_float((raw.x >> 8) & 0xff));
  o.y = pack_bf16x2(fp8_e4m3_to_float((raw.x >> 16) & 0xff), fp8_e4m3_to_float(raw.x >> 24));
  o.z = pack_bf16x2(fp8_e4m3_to_float(raw.y & 0xff), fp8_e4m3_to_float((raw.y >> 8) & 0xff));
  o.w = pack_bf16x2(fp8_e4m3_to_float((raw.y >> 16) & 0xff), fp8_e4m3_to_float(raw.y >> 24));
  return o;
}

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_HALO, int MAX_TAPS, bool W_FP8>
struct ConvTile {
  static constexpr int NT = 64 * WAVES_CO * WAVES_P;
  static constexpr int BCO = WAVES_CO * TCO * 16;
  static constexpr int BP = WAVES_P * TP * 16;
  static constexpr int X_PIECES = ((BP + MAX_HALO) * 4 + NT - 1) / NT;
  static constexpr int W_PIECES = (BCO * MAX_TAPS * 4 + NT - 1) / NT;
  static size_t lds_bytes(int64_t halo, int64_t taps) {
    return (size_t)((BP + halo) + taps * BCO) * kRowElems * 2;
  }
};

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_HALO, int MAX_TAPS, bool W_FP8>
__global__ void __launch_bounds__(64 * WAVES_CO * WAVES_P)
    conv_mfma_kernel(const ConvParams p) {
  using Tile = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_HALO, MAX_TAPS, W_FP8>;
  constexpr int NT = Tile::NT;
  constexpr int BCO = Tile::BCO;
  constexpr int BP = Tile::BP;
  extern __shared__ __attribute__((aligned(16))) u16 lds[];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wave_co = wave % WAVES_CO;
  const int wave_p = wave / WAVES_CO;

  // blockIdx -> (b, position tile, column tile), column tile fastest so the workgroups that share
  // an input tile run back to back.
  const int n_tiles = (int)p.n_tiles;
  const int p_tiles = (int)p.p_tiles;
  const int bid = blockIdx.x;
  const int n_tile = bid % n_tiles;
  const int p_tile = (bid / n_tiles) % p_tiles;
  const int64_t b = bid / (n_tiles * p_tiles);
  const int n0 = n_tile * BCO;
  const int i0 = p_tile * BP;

  const int taps = (int)p.taps;
  const int dil = (int)p.dil;
  const int lpad = (int)p.lpad;
  const int rows = BP + (taps - 1) * dil;
  const int L = (int)p.length;     // output positions
  const int XL = (int)p.x_length;  // input positions (the history ends at XL)
  const int H = lpad;              // history samples when streaming
  const int c_in = (int)p.c_in;
  const int n_cols = (int)p.n_cols;

  u16* xs = lds;                     // [rows][40]
  u16* ws = lds + rows * kRowElems;  // [taps][BCO][40]

  const u16* hist_read = nullptr;
  u16* hist_write = nullptr;
  const int64_t slot = p.hist != nullptr ? p.slot_index[b] : -1;
  if (slot >= 0 && slot < p.hist_slots) {
    const int64_t parity = p.slot_parity[slot] & 1;
    const u16* base = p.hist + slot * p.hist_slot_stride;
    hist_read = p.hist_cold ? nullptr : base + parity * H * c_in;
    hist_write = const_cast<u16*>(base) + (1 - parity) * H * c_in;
  }
  const bool writes_history = hist_write != nullptr && n_tile == 0 && H > 0;

  const int chunks = (c_in + kChunk - 1) / kChunk;
  const int x_pieces = rows * 4;
  const int w_pieces = BCO * taps * 4;
  // NT is a multiple of 4, so a thread stages the same 8-channel quarter q of every row it loads.
  const int q8 = (tid & 3) * 8;

  // Per-thread staging descriptors, computed once: each input piece's element offset at channel
  // q8 of chunk 0 (from the x row or from the slot history, 2 bits of xmode per piece: 0 zeros,
  // 1 x, 2 history), and each weight piece's LDS slot (-1 = none) and whether it is a real column.
  const u16* xrow = p.x + b * p.x_sb;
  int xoff[Tile::X_PIECES];
  unsigned xmode = 0;
#pragma unroll
  for (int u = 0; u < Tile::X_PIECES; ++u) {
    const int piece = tid + u * NT;
    const int pos = i0 - lpad + (piece >> 2);
    int off = 0;
    if (piece < x_pieces) {
      if (pos >= 0 && pos < XL) {
        off = pos * (int)p.x_st + q8;
        xmode |= 1u << (2 * u);
      } else if (pos < 0 && hist_read != nullptr) {
        off = (H + pos) * c_in + q8;
        xmode |= 2u << (2 * u);
      }
    }
    xoff[u] = off;
  }
  int wlds[Tile::W_PIECES];
  unsigned wreal = 0;
#pragma unroll
  for (int u = 0; u < Tile::W_PIECES; ++u) {
    const int piece = tid + u * NT;
    int off = -1;
    if (piece < w_pieces) {
      // packed order within a chunk is [n][tap][32]
      const int nl = piece / (taps * 4);
      const int rem = piece - nl * taps * 4;
      off = ((rem >> 2) * BCO + nl) * kRowElems + (rem & 3) * 8;
      if (n0 + nl < n_cols) wreal |= 1u << u;
    }
    wlds[u] = off;
  }

  uint4 xr[Tile::X_PIECES];
  uint4 wr[W_FP8 ? 1 : Tile::W_PIECES];
  uint2 wr8[W_FP8 ? Tile::W_PIECES : 1];

  auto load_chunk = [&](int kc) {
    const bool in_range = kc * kChunk + q8 < c_in;
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      const unsigned mode = (xmode >> (2 * u)) & 3u;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (mode != 0 && in_range) {
        const u16* base = mode == 1 ? xrow : hist_read;
        v = *reinterpret_cast<const uint4*>(base + xoff[u] + kc * kChunk);
      }
      xr[u] = v;
    }
    const int64_t wbase = ((int64_t)kc * n_cols + n0) * taps * kChunk;
#pragma unroll
    for (int u = 0; u < Tile::W_PIECES; ++u) {
      const int64_t off = wbase + (int64_t)(tid + u * NT) * 8;
      if constexpr (W_FP8) {
        uint2 v = make_uint2(0, 0);
        if (wreal & (1u << u))
          v = *reinterpret_cast<const uint2*>(reinterpret_cast<const uint8_t*>(p.weight) + off);
        wr8[u] = v;
      } else {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (wreal & (1u << u))
          v = *reinterpret_cast<const uint4*>(reinterpret_cast<const u16*>(p.weight) + off);
        wr[u] = v;
      }
    }
  };

  auto store_chunk = [&](int kc) {
    const bool in_range = kc * kChunk + q8 < c_in;
#pragma unroll
    for (int u = 0; u < Tile::X_PIECES; ++u) {
      const int piece = tid + u * NT;
      if (piece < x_pieces) {
        *reinterpret_cast<uint4*>(xs + (piece >> 2) * kRowElems + q8) = xr[u];
        if (writes_history && in_range) {
          // the new history is the last H samples of (history ++ x); each sample is written by
          // the workgroup whose own positions hold it (negative ones by the first tile)
          const int pos = i0 - lpad + (piece >> 2);
          const bool owned = (pos >= i0 && pos < i0 + BP) || (i0 == 0 && pos < 0);
          if (owned && pos >= XL - H && pos < XL)
            *reinterpret_cast<uint4*>(hist_write + (int64_t)(pos - (XL - H)) * c_in + q8 +
                                      kc * kChunk) = xr[u];
        }
      }
    }
#pragma unroll
    for (int u = 0; u < Tile::W_PIECES; ++u) {
      if (wlds[u] >= 0) {
        uint4 v;
        if constexpr (W_FP8) v = fp8x8_to_bf16x8(wr8[u]);
        else v = wr[u];
        *reinterpret_cast<uint4*>(ws + wlds[u]) = v;
      }
    }
  };

  f32x4 acc[TCO][TP];
#pragma unroll
  for (int c = 0; c < TCO; ++c)
#pragma unroll
    for (int t = 0; t < TP; ++t) acc[c][t] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lrow = lane & 15;
  const int lk = (lane >> 4) * 8;
  const int wco0 = wave_co * TCO * 16;
  const int wp0 = wave_p * TP * 16;

  load_chunk(0);
  for (int kc = 0; kc < chunks; ++kc) {
    __syncthreads();
    store_chunk(kc);
    __syncthreads();
    if (kc + 1 < chunks) load_chunk(kc + 1);
    const u16* wtap = ws + (wco0 + lrow) * kRowElems + lk;
    const u16* xtap = xs + (wp0 + lrow) * kRowElems + lk;
    for (int j = 0; j < taps; ++j) {
      bf16x8 a[TCO];
#pragma unroll
      for (int c = 0; c < TCO; ++c)
        a[c] = *reinterpret_cast<const bf16x8*>(wtap + c * 16 * kRowElems);
#pragma unroll
      for (int t = 0; t < TP; ++t) {
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(xtap + t * 16 * kRowElems);
#pragma unroll
        for (int c = 0; c < TCO; ++c)
          acc[c][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[c], bv, acc[c][t], 0, 0, 0);
      }
      wtap += BCO * kRowElems;
      xtap += dil * kRowElems;
    }
  }

  // Epilogue: lane holds D[co = 4*(lane/16) + e][pos = lane % 16] of each 16x16 tile. Column by
  // column, every position's residual / mix operands are loaded before the first store (they
  // may alias sum_out), so the loads of a column overlap.
  const int ch_in_tile = (lane >> 4) * 4;
#pragma unroll
  for (int c = 0; c < TCO; ++c) {
    const int n = n0 + wco0 + c * 16 + ch_in_tile;
    if (n >= n_cols) continue;
    float scale[4], bias[4], aa[4], bb[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int co = (n + e) % (int)p.c_out;
      scale[e] = p.wscale ? p.wscale[n + e] : 1.f;
      bias[e] = p.bias ? p.bias[co] : 0.f;
      aa[e] = p.act_a ? p.act_a[co] : 0.f;
      bb[e] = p.act_b ? p.act_b[co] : 0.f;
    }
    float4 res[TP];
#pragma unroll
    for (int t = 0; t < TP; ++t) {
      const int pos = i0 + wp0 + t * 16 + lrow;
      res[t] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (pos < L && p.residual)
        res[t] = *reinterpret_cast<const float4*>(p.residual + b * p.r_sb +
                                                  (int64_t)pos * p.r_st + n);
    }
#pragma unroll
    for (int t = 0; t < TP; ++t) {
      const int pos = i0 + wp0 + t * 16 + lrow;
      if (pos >= L) continue;
      float v[4];
      v[0] = acc[c][t][0] * scale[0] + bias[0] + res[t].x;
      v[1] = acc[c][t][1] * scale[1] + bias[1] + res[t].y;
      v[2] = acc[c][t][2] * scale[2] + bias[2] + res[t].z;
      v[3] = acc[c][t][3] * scale[3] + bias[3] + res[t].w;
      const int64_t roff = b * p.r_sb + (int64_t)pos * p.r_st + n;
      if (p.mix_a) {
        const float4 ma = *reinterpret_cast<const float4*>(p.mix_a + roff);
        const float4 mb = *reinterpret_cast<const float4*>(p.mix_b + roff);
        v[0] = ((ma.x + mb.x) + v[0]) * p.mix_scale;
        v[1] = ((ma.y + mb.y) + v[1]) * p.mix_scale;
        v[2] = ((ma.z + mb.z) + v[2]) * p.mix_scale;
        v[3] = ((ma.w + mb.w) + v[3]) * p.mix_scale;
      }
      if (p.sum_out)
        *reinterpret_cast<float4*>(p.sum_out + roff) = make_float4(v[0], v[1], v[2], v[3]);
      if (p.out == nullptr) continue;
      float y[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) y[e] = apply_act(p.act, v[e], aa[e], bb[e], p.slope);
      const int64_t ooff = b * p.o_sb + (int64_t)pos * p.o_st + n;
      if (p.out_bf16) {
        uint2 o;
        o.x = pack_bf16x2(y[0], y[1]);
        o.y = pack_bf16x2(y[2], y[3]);
        *reinterpret_cast<uint2*>(reinterpret_cast<u16*>(p.out) + ooff) = o;
      } else {
        *reinterpret_cast<float4*>(reinterpret_cast<float*>(p.out) + ooff) =
            make_float4(y[0], y[1], y[2], y[3]);
      }
    }
  }
}

// Raise a kernel's dynamic-LDS limit to the CU's 160 KiB. A refusal is not an error here (the
// launch check reports a launch the runtime cannot make), so its status is cleared.
bool raise_lds_limit(const void* kernel) {
  const hipError_t e =
      hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
  (void)hipGetLastError();
  return e == hipSuccess;
}

template <int WAVES_CO, int WAVES_P, int TCO, int TP, int MAX_HALO, int MAX_TAPS>
int launch_tile(ConvParams p, bool fp8, hipStream_t stream) {
  using Tile = ConvTile<WAVES_CO, WAVES_P, TCO, TP, MAX_HALO, MAX_TAPS, false>;
  const int64_t halo = (p.taps - 1) * p.dil;
  if (halo > MAX_HALO || p.taps > MAX_TAPS) return OMNI_ERR_UNSUPPORTED;
  p.p_tiles = (p.length + Tile::BP - 1) / Tile::BP;
  p.n_tiles = (p.n_cols + Tile::BCO - 1) / Tile::BCO;
  const int64_t blocks = p.batch * p.p_tiles * p.n_tiles;
  if (blocks == 0) return OMNI_OK;
  // in-block offsets are 32-bit: a row of x, a slot's history and a chunk of weights
  if (blocks > 0x7fffffffLL || p.n_cols * p.taps * kChunk > 0x7fffffffLL ||
      p.length > 0x3fffffffLL || (p.x_length + p.lpad) * p.x_st > 0x7fffffffLL ||
      p.lpad * p.c_in > 0x7fffffffLL)
    return OMNI_ERR_UNSUPPORTED;
  const size_t lds = Tile::lds_bytes(halo, p.taps);
  if (lds > 160 * 1024) return OMNI_ERR_UNSUPPORTED;
  // The dynamic-LDS limit is raised once per kernel instantiation (to the 160 KiB maximum), on
  // its first launch, so launches inside a graph capture make no attribute calls.
  if (fp8) {
    auto k = conv_mfma_kernel<WAVES_CO, WAVES_P, TCO, TP, MAX_HALO, MAX_TAPS, true>;
    static const bool raised = raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(Tile::NT), lds, stream, p);
  } else {
    auto k = conv_mfma_kernel<WAVES_CO, WAVES_P, TCO, TP, MAX_HALO, MAX_TAPS, false>;
    static const bool raised = raise_lds_limit((const void*)k);
    (void)raised;
    hipLaunchKernelGGL(k, dim3((unsigned)blocks), dim3(Tile::NT), lds, stream, p);
  }
  OMNI_LAUNCH_CHECK();
  return OMNI_OK;
}

// Tile choice by row length: short rows (streaming chunks at the frame rate) take narrow
// position tiles with wide column tiles so few MFMA lanes idle; long rows take 256-position tiles,
// 96 columns wide for the 96/192-channel layers and 64 wide otherwise. Long kernels (k = 11)
// use the variants with the larger tap budget.
int dispatch(ConvParams p, bool fp8, hipStream_t stream) {
  const int64_t halo = (p.taps - 1) * p.dil;
  if (halo > 64) return OMNI_ERR_UNSUPPORTED;
  if (p.taps <= 7) {
    if (p.length <= 16) return launch_tile<4, 1, 2, 1, 64, 7>(p, fp8, stream);
    if (p.length <= 32) return launch_tile<4, 1, 2, 2, 64, 7>(p, fp8, stream);
    if (p.length <= 128) return launch_tile<2, 2, 4, 2, 64, 7>(p, fp8, stream);
    if (p.n_cols % 96 == 0 && p.n_cols <= 192)
      return launch_tile<1, 4, 6, 4, 64, 7>(p, fp8, stream);
    return launch_tile<1, 4, 4, 4, 64, 7>(p, fp8, stream);
  }
  if (p.taps <= 11) {
    if (p.length <= 128) return launch_tile<2, 2, 2, 2, 64, 11>(p, fp8, stream);
    return launch_tile<1, 4, 4, 4, 64, 11>(p, fp8, stream);
  }
  return OMNI_ERR_UNSUPPORTED;
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15) == 0; }

}  // namespace

extern "C" int omni_conv1d_fused(const omni_conv_args* a, omni_stream_t stream) {
  if (!a || !a->x || !a->weight) return OMNI_ERR_INVALID_ARG;
  if (!a->out && !a->sum_out) return OMNI_ERR_INVALID_ARG;
  if (a->batch < 0 || a->length < 0 || a->c_in < 1 || a->n_cols < 1 || a->c_out < 1 ||
      a->taps < 1 || a->dilation < 1 || a->left_pad < 0)
    return OMNI_ERR_INVALID_ARG;
  if (a->n_cols % 16 || a->n_cols % a->c_out || a->c_out % 4 || a->c_in % 8)
    return OMNI_ERR_UNSUPPORTED;
  if (a->left_pad > (a->taps - 1) * a->dilation) return OMNI_ERR_INVALID_ARG;
  if (a->weight_dtype != OMNI_DTYPE_BF16 && a->weight_dtype != OMNI_DTYPE_FP8_E4M3)
    return OMNI_ERR_INVALID_ARG;
  const bool fp8 = a->weight_dtype == OMNI_DTYPE_FP8_E4M3;
  if (fp8 && !a->weight_scale) return OMNI_ERR_INVALID_ARG;
  if (a->out_dtype != OMNI_DTYPE_BF16 && a->out_dtype != OMNI_DTYPE_F32)
    return OMNI_ERR_INVALID_ARG;
  if (a->activation < OMNI_ACTIVATION_NONE || a->activation > OMNI_ACTIVATION_CLAMP)
    return OMNI_ERR_INVALID_ARG;
  if (a->activation == OMNI_ACTIVATION_SNAKE && (!a->act_a || !a->act_b))
    return OMNI_ERR_INVALID_ARG;
  // 16-byte staging loads of x and history, 16/8-byte epilogue accesses.
  if (!aligned16(a->x) || a->x_stride_t % 8 || a->x_stride_b % 8 || a->x_stride_t < a->c_in)
    return OMNI_ERR_INVALID_ARG;
  if (!aligned16(a->weight)) return OMNI_ERR_INVALID_ARG;
  if (a->x_length < 0) return OMNI_ERR_INVALID_ARG;
  const bool has_r = a->residual || a->sum_out || a->mix_a;
  if (has_r && (a->residual_stride_t % 4 || a->residual_stride_b % 4 ||
                a->residual_stride_t < a->n_cols))
    return OMNI_ERR_INVALID_ARG;
  if ((a->residual && !aligned16(a->residual)) || (a->sum_out && !aligned16(a->sum_out)))
    return OMNI_ERR_INVALID_ARG;
  if (a->mix_a && (!a->mix_b || !aligned16(a->mix_a) || !aligned16(a->mix_b)))
    return OMNI_ERR_INVALID_ARG;
  if (a->out && a->out_stride_t < a->n_cols) return OMNI_ERR_INVALID_ARG;
  if (a->out) {
    if ((reinterpret_cast<uintptr_t>(a->out) & 7) || a->out_stride_t % 4 || a->out_stride_b % 4)
      return OMNI_ERR_INVALID_ARG;
    if (a->out_dtype == OMNI_DTYPE_F32 && !aligned16(a->out)) return OMNI_ERR_INVALID_ARG;
  }
  if (a->hist_pool) {
    if (!a->slot_index || !a->slot_parity || !aligned16(a->hist_pool) || a->hist_num_slots < 1)
      return OMNI_ERR_INVALID_ARG;
    if (a->left_pad != (a->taps - 1) * a->dilation) return OMNI_ERR_INVALID_ARG;
    if (a->x_length != 0 && a->x_length != a->length) return OMNI_ERR_INVALID_ARG;
    if (a->hist_slot_stride < 2 * a->left_pad * a->c_in || a->hist_slot_stride % 8)
      return OMNI_ERR_INVALID_ARG;
  }
  if (a->batch == 0 || a->length == 0) return OMNI_OK;

  ConvParams p{};
  p.x = reinterpret_cast<const u16*>(a->x);
  p.x_sb = a->x_stride_b;
  p.x_st = a->x_stride_t;
  p.batch = a->batch;
  p.length = a->length;
  p.c_in = a->c_in;
  p.x_length = a->x_length ? a->x_length : a->length;
  p.weight = a->weight;
  p.wscale = fp8 ? a->weight_scale : nullptr;
  p.n_cols = a->n_cols;
  p.c_out = a->c_out;
  p.taps = a->taps;
  p.dil = a->dilation;
  p.lpad = a->left_pad;
  p.bias = a->bias;
  p.hist = reinterpret_cast<const u16*>(a->hist_pool);
  p.slot_index = a->slot_index;
  p.slot_parity = a->slot_parity;
  p.hist_slots = a->hist_num_slots;
  p.hist_slot_stride = a->hist_slot_stride;
  p.hist_cold = a->history_cold;
  p.residual = a->residual;
  p.r_sb = a->residual_stride_b;
  p.r_st = a->residual_stride_t;
  p.mix_a = a->mix_a;
  p.mix_b = a->mix_b;
  p.mix_scale = a->mix_scale;
  p.sum_out = a->sum_out;
  p.out = a->out;
  p.out_bf16 = a->out_dtype == OMNI_DTYPE_BF16;
  p.o_sb = a->out_stride_b;
  p.o_st = a->out_stride_t;
  p.act = a->activation;
  p.act_a = a->act_a;
  p.act_b = a->act_b;
  p.slope = a->act_slope;
  return dispatch(p, fp8, reinterpret_cast<hipStream_t>(stream));
}
